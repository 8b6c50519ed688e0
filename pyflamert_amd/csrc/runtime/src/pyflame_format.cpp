// .pfm v1/v2 reader and writer (format described in pyflame_format.hpp).
// Every read is length-checked against DeserializationLimits before
// allocating.
#include "pyflame_rt/pyflame_format.hpp"

#include <algorithm>
#include <cstring>
#include <fstream>

#include "pyflame_rt/errors.hpp"

namespace pyflame_rt {

namespace {

void read_exact(std::istream& is, void* buf, size_t n, const char* what) {
    is.read(static_cast<char*>(buf), static_cast<std::streamsize>(n));
    const std::streamsize got = is.gcount();
    if (is.fail() || got < 0 || static_cast<size_t>(got) != n)
        throw InvalidModelError(std::string("Incomplete read: ") + what + " (expected " + std::to_string(n) +
                                " bytes, got " + std::to_string(got) + ")");
}

template <class T>
T rd(std::istream& is, const char* what) {
    T v{};
    read_exact(is, &v, sizeof(T), what);
    return v;
}

std::string rd_string(std::istream& is) {
    const uint64_t n = rd<uint64_t>(is, "uint64");
    if (n > DeserializationLimits::MAX_STRING_SIZE)
        throw InvalidModelError("String size exceeds limit: " + std::to_string(n) + " > " +
                                std::to_string(DeserializationLimits::MAX_STRING_SIZE));
    std::string s((size_t)n, '\0');
    if (n) read_exact(is, &s[0], (size_t)n, "string data");
    return s;
}

DType rd_dtype(std::istream& is, const std::string& ctx) {
    const uint32_t v = rd<uint32_t>(is, "uint32");
    if (!validate_dtype_value(v)) throw InvalidModelError("Invalid dtype value" + ctx + ": " + std::to_string(v));
    return static_cast<DType>(v);
}

uint64_t rd_count(std::istream& is, uint64_t limit, const std::string& what) {
    const uint64_t n = rd<uint64_t>(is, "uint64");
    if (n > limit) throw InvalidModelError(what + ": " + std::to_string(n));
    return n;
}

TensorInfo rd_info(std::istream& is) {
    TensorInfo info;
    info.name = rd_string(is);
    info.dtype = rd_dtype(is, "");
    const uint64_t nd = rd_count(is, DeserializationLimits::MAX_DIMS, "Too many dimensions");
    for (uint64_t i = 0; i < nd; ++i) {
        const int64_t d = rd<int64_t>(is, "int64");
        info.shape.push_back(d < 0 ? std::optional<int64_t>() : std::optional<int64_t>(d));
    }
    return info;
}

std::pair<std::string, Tensor> rd_tensor(std::istream& is) {
    std::string name = rd_string(is);
    const DType dt = rd_dtype(is, " in tensor '" + name + "'");
    const uint64_t nd = rd_count(is, DeserializationLimits::MAX_DIMS, "Too many dimensions in tensor '" + name + "'");
    std::vector<int64_t> shape((size_t)nd);
    for (uint64_t i = 0; i < nd; ++i) {
        shape[i] = rd<int64_t>(is, "int64");
        if (shape[i] < 0)
            throw InvalidModelError("Negative dimension in tensor '" + name + "' at axis " + std::to_string(i));
        if (shape[i] > DeserializationLimits::MAX_DIMENSION_SIZE)
            throw InvalidModelError("Dimension too large in tensor '" + name + "' at axis " + std::to_string(i));
    }
    int64_t total;
    try {
        total = checked_product(shape);
    } catch (const std::overflow_error&) {
        throw InvalidModelError("Tensor '" + name + "' dimension product overflows int64");
    }
    if (total > DeserializationLimits::MAX_TOTAL_ELEMENTS)
        throw InvalidModelError("Tensor '" + name + "' has too many elements: " + std::to_string(total));
    Tensor t(shape, dt);
    const uint64_t nbytes = rd<uint64_t>(is, "uint64");
    if (nbytes > DeserializationLimits::MAX_TENSOR_DATA_SIZE)
        throw InvalidModelError("Data size exceeds limit: " + std::to_string(nbytes));
    if (nbytes != t.size_bytes())
        throw InvalidModelError("Data size mismatch for tensor '" + name + "': got " + std::to_string(nbytes) +
                                ", expected " + std::to_string(t.size_bytes()));
    if (nbytes) read_exact(is, t.data(), (size_t)nbytes, "byte data");
    return {name, std::move(t)};
}

std::shared_ptr<Node> rd_node(std::istream& is) {
    std::string name = rd_string(is), op = rd_string(is);
    std::vector<std::string> ins, outs;
    const uint64_t ni = rd_count(is, DeserializationLimits::MAX_ARRAY_COUNT, "Too many inputs for node '" + name + "'");
    for (uint64_t i = 0; i < ni; ++i) ins.push_back(rd_string(is));
    const uint64_t no = rd_count(is, DeserializationLimits::MAX_ARRAY_COUNT, "Too many outputs for node '" + name + "'");
    for (uint64_t i = 0; i < no; ++i) outs.push_back(rd_string(is));
    auto node = std::make_shared<Node>(name, op, ins, outs);
    const uint64_t na = rd_count(is, DeserializationLimits::MAX_ATTRIBUTES, "Too many attributes for node '" + name + "'");
    for (uint64_t i = 0; i < na; ++i) {
        const std::string an = rd_string(is);
        const uint32_t type = rd<uint32_t>(is, "uint32");
        switch (type) {
            case 0: node->set_attr(an, rd<int64_t>(is, "int64")); break;
            case 1: node->set_attr(an, rd<float>(is, "float attribute")); break;
            case 2: node->set_attr(an, rd_string(is)); break;
            case 3: {
                const uint64_t n = rd_count(is, DeserializationLimits::MAX_ARRAY_COUNT,
                                            "Vector attribute '" + an + "' too large");
                std::vector<int64_t> v((size_t)n);
                for (auto& x : v) x = rd<int64_t>(is, "int64");
                node->set_attr(an, v);
                break;
            }
            case 4: {
                const uint64_t n = rd_count(is, DeserializationLimits::MAX_ARRAY_COUNT,
                                            "Vector attribute '" + an + "' too large");
                std::vector<float> v((size_t)n);
                for (auto& x : v) x = rd<float>(is, "float vector element");
                node->set_attr(an, v);
                break;
            }
            case 255: break;
            default:
                throw InvalidModelError("Unknown attribute type " + std::to_string(type) + " for attribute '" + an +
                                        "' in node '" + name + "'");
        }
    }
    return node;
}

// Bulk read of n elements of T into v, after the byte count is checked.
template <class T>
void rd_array(std::istream& is, std::vector<T>& v, uint64_t n, const std::string& what) {
    if (n > DeserializationLimits::MAX_TENSOR_DATA_SIZE / sizeof(T))
        throw InvalidModelError("Data size exceeds limit: " + what);
    v.resize((size_t)n);
    if (n) read_exact(is, v.data(), (size_t)n * sizeof(T), what.c_str());
}

std::pair<std::string, SparseInitializer> rd_sparse(std::istream& is) {
    std::string name = rd_string(is);
    SparseInitializer s;
    const uint32_t fmt = rd<uint32_t>(is, "uint32");
    if (fmt != SparseInitializer::Csr && fmt != SparseInitializer::Nm24)
        throw InvalidModelError("Unknown sparse format " + std::to_string(fmt) + " for tensor '" + name + "'");
    s.format = static_cast<SparseInitializer::Format>(fmt);
    s.dtype = rd_dtype(is, " in sparse tensor '" + name + "'");
    s.rows = rd<int64_t>(is, "int64");
    s.cols = rd<int64_t>(is, "int64");
    if (s.rows < 0 || s.cols < 0 || s.rows > DeserializationLimits::MAX_DIMENSION_SIZE ||
        s.cols > DeserializationLimits::MAX_DIMENSION_SIZE)
        throw InvalidModelError("Invalid dimensions in sparse tensor '" + name + "'");
    if (s.format == SparseInitializer::Csr) {
        const uint64_t nnz = rd<uint64_t>(is, "uint64");
        if (nnz > (uint64_t)DeserializationLimits::MAX_TOTAL_ELEMENTS)
            throw InvalidModelError("Sparse tensor '" + name + "' has too many nonzeros: " + std::to_string(nnz));
        const uint32_t ib = rd<uint32_t>(is, "uint32");
        if (ib != 2 && ib != 4)
            throw InvalidModelError("Sparse tensor '" + name + "': index width must be 2 or 4 bytes");
        rd_array(is, s.indptr, (uint64_t)s.rows + 1, "sparse indptr");
        if (ib == 2) {
            std::vector<uint16_t> c16;
            rd_array(is, c16, nnz, "sparse indices");
            s.indices.assign(c16.begin(), c16.end());
        } else {
            rd_array(is, s.indices, nnz, "sparse indices");
        }
        if (!validate_dtype_value((uint32_t)s.dtype) || dtype_size(s.dtype) > 4)
            throw InvalidModelError("Sparse tensor '" + name + "': unsupported value type");
        rd_array(is, s.values, nnz * dtype_size(s.dtype), "sparse values");
        s.scale_axis = rd<uint32_t>(is, "uint32");
        const uint64_t ns = rd_count(is, DeserializationLimits::MAX_ARRAY_COUNT * 100,
                                     "Too many scales in sparse tensor '" + name + "'");
        rd_array(is, s.scales, ns, "sparse scales");
    } else {
        if (s.cols % 4)
            throw InvalidModelError("Sparse tensor '" + name + "': 2:4 needs cols divisible by 4");
        rd_array(is, s.values, (uint64_t)s.rows * (uint64_t)(s.cols / 2), "2:4 values");
        rd_array(is, s.positions, (uint64_t)s.rows * (uint64_t)(s.cols / 4), "2:4 positions");
    }
    return {name, std::move(s)};
}

template <class T>
void wr(std::ostream& os, T v) {
    os.write(reinterpret_cast<const char*>(&v), sizeof(T));
}

void wr_string(std::ostream& os, const std::string& s) {
    wr<uint64_t>(os, s.size());
    os.write(s.data(), (std::streamsize)s.size());
}

void wr_info(std::ostream& os, const TensorInfo& i) {
    wr_string(os, i.name);
    wr<uint32_t>(os, static_cast<uint32_t>(i.dtype));
    wr<uint64_t>(os, i.shape.size());
    for (const auto& d : i.shape) wr<int64_t>(os, d ? *d : -1);
}

template <class T>
void wr_array(std::ostream& os, const std::vector<T>& v) {
    os.write(reinterpret_cast<const char*>(v.data()), (std::streamsize)(v.size() * sizeof(T)));
}

// Column indices go to disk as uint16 when every index fits (cols <= 65536).
void wr_sparse(std::ostream& os, const std::string& name, const SparseInitializer& s) {
    wr_string(os, name);
    wr<uint32_t>(os, s.format);
    wr<uint32_t>(os, static_cast<uint32_t>(s.dtype));
    wr<int64_t>(os, s.rows);
    wr<int64_t>(os, s.cols);
    if (s.format == SparseInitializer::Csr) {
        wr<uint64_t>(os, (uint64_t)s.indices.size());
        const bool narrow = s.cols <= 65536;
        wr<uint32_t>(os, narrow ? 2 : 4);
        wr_array(os, s.indptr);
        if (narrow) {
            std::vector<uint16_t> c16(s.indices.begin(), s.indices.end());
            wr_array(os, c16);
        } else {
            wr_array(os, s.indices);
        }
        wr_array(os, s.values);
        wr<uint32_t>(os, s.scale_axis);
        wr<uint64_t>(os, s.scales.size());
        wr_array(os, s.scales);
    } else {
        wr_array(os, s.values);
        wr_array(os, s.positions);
    }
}

}  // namespace

std::unique_ptr<Graph> PyFlameFormat::load(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw InvalidModelError("Cannot open file", path);
    char magic[4];
    read_exact(f, magic, 4, "magic bytes");
    if (std::memcmp(magic, MAGIC, 4) != 0) throw InvalidModelError("Invalid magic bytes", path);
    const uint32_t version = rd<uint32_t>(f, "uint32");
    if (version > VERSION) throw InvalidModelError("Unsupported version: " + std::to_string(version), path);
    if (version == 0) throw InvalidModelError("Unsupported version: 0", path);
    auto g = std::make_unique<Graph>(rd_string(f));
    const uint64_t ni = rd_count(f, DeserializationLimits::MAX_ARRAY_COUNT, "Too many graph inputs");
    for (uint64_t i = 0; i < ni; ++i) g->add_input(rd_info(f));
    const uint64_t no = rd_count(f, DeserializationLimits::MAX_ARRAY_COUNT, "Too many graph outputs");
    for (uint64_t i = 0; i < no; ++i) g->add_output(rd_info(f));
    const uint64_t nt = rd_count(f, DeserializationLimits::MAX_ARRAY_COUNT, "Too many initializers");
    for (uint64_t i = 0; i < nt; ++i) {
        auto nt_pair = rd_tensor(f);
        g->add_initializer(nt_pair.first, std::move(nt_pair.second));
    }
    const uint64_t nn = rd_count(f, DeserializationLimits::MAX_NODES, "Too many nodes");
    for (uint64_t i = 0; i < nn; ++i) g->add_node(rd_node(f));
    if (version >= 2) {
        const uint64_t ns = rd_count(f, DeserializationLimits::MAX_ARRAY_COUNT, "Too many sparse initializers");
        for (uint64_t i = 0; i < ns; ++i) {
            auto sp = rd_sparse(f);
            try {
                g->add_sparse_initializer(sp.first, std::move(sp.second));
            } catch (const InvalidModelError&) {
                throw;
            } catch (const std::exception& e) {
                throw InvalidModelError(e.what(), path);
            }
        }
    }
    if (f.fail()) throw InvalidModelError("Stream read failed: end of file");
    return g;
}

void PyFlameFormat::save(const Graph& g, const std::string& path) {
    std::ofstream f(path, std::ios::binary);
    if (!f) throw InvalidModelError("Cannot create file", path);
    f.write(MAGIC, 4);
    // A model without sparse initializers stays version 1, readable by the
    // reference loader.
    const bool sparse = !g.sparse_initializers().empty();
    wr<uint32_t>(f, sparse ? VERSION : 1u);
    wr_string(f, g.name());
    wr<uint64_t>(f, g.inputs().size());
    for (const auto& i : g.inputs()) wr_info(f, i);
    wr<uint64_t>(f, g.outputs().size());
    for (const auto& o : g.outputs()) wr_info(f, o);
    // Initializers in name order, so a saved model is byte-reproducible.
    std::vector<std::string> names;
    for (const auto& kv : g.initializers()) names.push_back(kv.first);
    std::sort(names.begin(), names.end());
    wr<uint64_t>(f, names.size());
    for (const auto& n : names) {
        const Tensor& t = g.initializers().at(n);
        wr_string(f, n);
        wr<uint32_t>(f, static_cast<uint32_t>(t.dtype()));
        wr<uint64_t>(f, t.ndim());
        for (int64_t d : t.shape()) wr<int64_t>(f, d);
        wr<uint64_t>(f, t.size_bytes());
        f.write(static_cast<const char*>(t.data()), (std::streamsize)t.size_bytes());
    }
    wr<uint64_t>(f, g.num_nodes());
    for (const auto& n : g.nodes()) {
        wr_string(f, n->name());
        wr_string(f, n->op_type());
        wr<uint64_t>(f, n->inputs().size());
        for (const auto& s : n->inputs()) wr_string(f, s);
        wr<uint64_t>(f, n->outputs().size());
        for (const auto& s : n->outputs()) wr_string(f, s);
        std::vector<std::string> an;
        for (const auto& kv : n->attributes()) an.push_back(kv.first);
        std::sort(an.begin(), an.end());
        wr<uint64_t>(f, an.size());
        for (const auto& k : an) {
            wr_string(f, k);
            const AttributeValue& v = n->attributes().at(k);
            if (auto* p = std::get_if<int64_t>(&v)) { wr<uint32_t>(f, 0); wr<int64_t>(f, *p); }
            else if (auto* p = std::get_if<float>(&v)) { wr<uint32_t>(f, 1); wr<float>(f, *p); }
            else if (auto* p = std::get_if<std::string>(&v)) { wr<uint32_t>(f, 2); wr_string(f, *p); }
            else if (auto* p = std::get_if<std::vector<int64_t>>(&v)) {
                wr<uint32_t>(f, 3);
                wr<uint64_t>(f, p->size());
                for (int64_t x : *p) wr<int64_t>(f, x);
            } else if (auto* p = std::get_if<std::vector<float>>(&v)) {
                wr<uint32_t>(f, 4);
                wr<uint64_t>(f, p->size());
                for (float x : *p) wr<float>(f, x);
            } else {
                wr<uint32_t>(f, 255);
            }
        }
    }
    if (sparse) {
        std::vector<std::string> sn;
        for (const auto& kv : g.sparse_initializers()) sn.push_back(kv.first);
        std::sort(sn.begin(), sn.end());
        wr<uint64_t>(f, sn.size());
        for (const auto& n : sn) wr_sparse(f, n, g.sparse_initializers().at(n));
    }
    if (!f) throw InvalidModelError("Write failed", path);
}

namespace {
// Null bytes, "..' path components and control characters are rejected
// (src/io/loader.cpp:15-60).
void validate_path(const std::string& path) {
    if (path.empty()) throw InvalidModelError("Empty path provided");
    if (path.find('\0') != std::string::npos)
        throw InvalidModelError("Path contains null byte - potential path injection");
    for (size_t pos = 0; (pos = path.find("..", pos)) != std::string::npos; pos += 2) {
        const bool pre = pos == 0 || path[pos - 1] == '/' || path[pos - 1] == '\\';
        const bool post = pos + 2 >= path.size() || path[pos + 2] == '/' || path[pos + 2] == '\\';
        if (pre && post)
            throw InvalidModelError("Path contains directory traversal sequence '..' - potential path traversal attack");
    }
    for (char c : path)
        if (c >= 0 && c < 32 && c != '\t')
            throw InvalidModelError("Path contains control character (ASCII " + std::to_string((int)c) +
                                    ") - potential injection");
}

std::string extension(const std::string& path) {
    const size_t p = path.rfind('.');
    if (p == std::string::npos) return "";
    std::string e = path.substr(p);
    std::transform(e.begin(), e.end(), e.begin(), ::tolower);
    return e;
}
}  // namespace

std::unique_ptr<Graph> load_model(const std::string& path) {
    validate_path(path);
    if (extension(path) == ".pfm") return PyFlameFormat::load(path);
    throw UnsupportedFormatError(extension(path), {".pfm"});
}

void save_model(const Graph& g, const std::string& path) {
    validate_path(path);
    if (extension(path) == ".pfm") return PyFlameFormat::save(g, path);
    throw UnsupportedFormatError(extension(path), {".pfm"});
}

}  // namespace pyflame_rt
