// extern "C" wrapper of InferenceSession (include/pfr_session.h).
#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "pfr_session.h"
#include "pyflame_rt/errors.hpp"
#include "pyflame_rt/pyflame_format.hpp"
#include "pyflame_rt/quantize.hpp"
#include "pyflame_rt/session.hpp"
#include "../backends/rocm/rocm_executor.hpp"

#include <cmath>
#include <cstdio>
#include <sstream>

using namespace pyflame_rt;

struct pfr_session {
    std::unique_ptr<InferenceSession> sess;
    std::vector<Tensor> results;
};

namespace {
thread_local std::string g_err;

template <class F>
int guard(F&& f) {
    try {
        g_err.clear();
        f();
        return PFR_S_OK;
    } catch (const InvalidModelError& e) {
        g_err = e.what();
        return PFR_S_INVALID_MODEL;
    } catch (const ValidationError& e) {
        g_err = e.what();
        return PFR_S_VALIDATION;
    } catch (const UnsupportedOperatorError& e) {
        g_err = e.what();
        return PFR_S_UNSUPPORTED_OP;
    } catch (const UnsupportedFormatError& e) {
        g_err = e.what();
        return PFR_S_FORMAT;
    } catch (const InputError& e) {
        g_err = e.what();
        return PFR_S_INPUT;
    } catch (const ShapeMismatchError& e) {
        g_err = e.what();
        return PFR_S_INPUT;
    } catch (const BackendError& e) {
        g_err = e.what();
        return PFR_S_BACKEND;
    } catch (const PyFlameRTError& e) {
        g_err = e.what();
        return PFR_S_RUNTIME;
    } catch (const std::exception& e) {
        g_err = e.what();
        return PFR_S_OTHER;
    }
}
}  // namespace

extern "C" {

const char* pfr_session_last_error(void) { return g_err.c_str(); }

int pfr_session_create(const char* path, const char* device, int strict_math_mode, int math_mode, int device_id,
                       int optimization_level, const char* quantization, pfr_session** out) {
    return guard([&] {
        if (!out || !path || !device) throw PyFlameRTError("null argument");
        *out = nullptr;
        SessionOptions o;
        o.device = device;
        o.strict_math_mode = strict_math_mode != 0;
        o.rocm_math_mode = math_mode;
        o.rocm_device_id = device_id;
        if (optimization_level < 0 || optimization_level > 3)
            throw PyFlameRTError("optimization_level must be 0 (None) .. 3 (All), got " +
                                 std::to_string(optimization_level));
        o.optimization_level = static_cast<OptLevel>(optimization_level);
        o.quantization = quantization ? quantization : "";
        auto s = std::make_unique<pfr_session>();
        s->sess = std::make_unique<InferenceSession>(path, o);
        *out = s.release();
    });
}

int pfr_session_destroy(pfr_session* s) {
    return guard([&] { delete s; });
}

int pfr_session_io_count(pfr_session* s, int* ni, int* no) {
    return guard([&] {
        if (!s) throw PyFlameRTError("null session");
        if (ni) *ni = (int)s->sess->graph().inputs().size();
        if (no) *no = (int)s->sess->graph().outputs().size();
    });
}

int pfr_session_io_info(pfr_session* s, int is_output, int index, const char** name, int* dtype, int64_t* shape,
                        int* ndim) {
    return guard([&] {
        if (!s) throw PyFlameRTError("null session");
        const auto& v = is_output ? s->sess->graph().outputs() : s->sess->graph().inputs();
        if (index < 0 || index >= (int)v.size()) throw PyFlameRTError("io index out of range");
        const TensorInfo& i = v[(size_t)index];
        if (name) *name = i.name.c_str();
        if (dtype) *dtype = (int)i.dtype;
        if (ndim) *ndim = (int)i.shape.size();
        if (shape)
            for (size_t d = 0; d < i.shape.size() && d < 16; ++d) shape[d] = i.shape[d] ? *i.shape[d] : -1;
    });
}

int pfr_session_run(pfr_session* s, int n_in, const char* const* names, const void* const* data, const int* dtypes,
                    const int64_t* const* shapes, const int* ndims, int n_out, const char* const* out_names,
                    int* n_results) {
    return guard([&] {
        if (!s) throw PyFlameRTError("null session");
        std::unordered_map<std::string, Tensor> feed;
        for (int i = 0; i < n_in; ++i) {
            if (!validate_dtype_value((uint32_t)dtypes[i])) throw InputError("bad dtype code for input");
            std::vector<int64_t> sh(shapes[i], shapes[i] + ndims[i]);
            // Borrowed view of the caller's buffer (run copies nothing it does not need).
            feed.emplace(names[i], Tensor(const_cast<void*>(data[i]), sh, static_cast<DType>(dtypes[i])));
        }
        std::vector<std::string> outs;
        for (int i = 0; i < n_out; ++i) outs.emplace_back(out_names[i]);
        s->results = s->sess->run(outs, feed);
        if (n_results) *n_results = (int)s->results.size();
    });
}

int pfr_session_result(pfr_session* s, int index, int* dtype, int64_t* shape, int* ndim, const void** data) {
    return guard([&] {
        if (!s) throw PyFlameRTError("null session");
        if (index < 0 || index >= (int)s->results.size()) throw PyFlameRTError("result index out of range");
        const Tensor& t = s->results[(size_t)index];
        if (dtype) *dtype = (int)t.dtype();
        if (ndim) *ndim = (int)t.ndim();
        if (shape)
            for (size_t d = 0; d < t.ndim() && d < 16; ++d) shape[d] = t.shape()[d];
        if (data) *data = t.data();
    });
}

namespace {
std::string jstr(const std::string& s) {
    std::string r = "\"";
    for (char c : s) {
        if (c == '"' || c == '\\') { r += '\\'; r += c; }
        else if ((unsigned char)c < 32) { char b[8]; std::snprintf(b, sizeof b, "\\u%04x", c); r += b; }
        else r += c;
    }
    return r + "\"";
}
std::string jshape(const Shape& s) {
    std::string r = "[";
    for (size_t i = 0; i < s.size(); ++i) r += (i ? "," : "") + std::to_string(s[i] ? *s[i] : -1);
    return r + "]";
}
std::string jfloat(float f) {
    if (!std::isfinite(f)) return "null";
    char b[32];
    std::snprintf(b, sizeof b, "%.9g", (double)f);
    return b;
}
std::string jattr(const AttributeValue& v) {
    if (auto* p = std::get_if<int64_t>(&v)) return std::to_string(*p);
    if (auto* p = std::get_if<float>(&v)) return jfloat(*p);
    if (auto* p = std::get_if<std::string>(&v)) return jstr(*p);
    std::string r = "[";
    if (auto* p = std::get_if<std::vector<int64_t>>(&v))
        for (size_t i = 0; i < p->size(); ++i) r += (i ? "," : "") + std::to_string((*p)[i]);
    if (auto* p = std::get_if<std::vector<float>>(&v))
        for (size_t i = 0; i < p->size(); ++i) r += (i ? "," : "") + jfloat((*p)[i]);
    if (auto* p = std::get_if<std::vector<std::string>>(&v))
        for (size_t i = 0; i < p->size(); ++i) r += (i ? "," : "") + jstr((*p)[i]);
    return r + "]";
}
int64_t count_nonzero_bytes(const Tensor& t) {
    // nonzero elements by value (+-0 count as zero for floats)
    int64_t n = 0;
    const int64_t e = t.num_elements();
    switch (t.dtype()) {
        case DType::Float32:
            for (int64_t i = 0; i < e; ++i) n += t.data_ptr<float>()[i] != 0.0f;
            break;
        case DType::Int8: case DType::UInt8: case DType::Bool:
            for (int64_t i = 0; i < e; ++i) n += t.data_ptr<uint8_t>()[i] != 0;
            break;
        default:
            n = -1;
    }
    return n;
}
}  // namespace

int pfr_model_describe(const char* path, char* buf, int64_t cap, int64_t* needed) {
    return guard([&] {
        if (!path) throw PyFlameRTError("null path");
        auto g = load_model(path);
        auto errs = g->validate();
        if (!errs.empty()) throw ValidationError(errs);
        std::ostringstream o;
        o << "{\"name\":" << jstr(g->name()) << ",\"inputs\":[";
        for (size_t i = 0; i < g->inputs().size(); ++i) {
            const auto& t = g->inputs()[i];
            o << (i ? "," : "") << "{\"name\":" << jstr(t.name) << ",\"dtype\":" << (int)t.dtype
              << ",\"shape\":" << jshape(t.shape) << "}";
        }
        o << "],\"outputs\":[";
        for (size_t i = 0; i < g->outputs().size(); ++i) {
            const auto& t = g->outputs()[i];
            o << (i ? "," : "") << "{\"name\":" << jstr(t.name) << ",\"dtype\":" << (int)t.dtype
              << ",\"shape\":" << jshape(t.shape) << "}";
        }
        o << "],\"initializers\":{";
        std::vector<std::string> names;
        for (const auto& kv : g->initializers()) names.push_back(kv.first);
        std::sort(names.begin(), names.end());
        for (size_t i = 0; i < names.size(); ++i) {
            const Tensor& t = g->initializers().at(names[i]);
            std::string sh = "[";
            for (size_t d = 0; d < t.ndim(); ++d) sh += (d ? "," : "") + std::to_string(t.shape()[d]);
            o << (i ? "," : "") << jstr(names[i]) << ":{\"dtype\":" << (int)t.dtype() << ",\"shape\":" << sh
              << "],\"nnz\":" << count_nonzero_bytes(t) << "}";
        }
        o << "},\"sparse_initializers\":{";
        std::vector<std::string> sn;
        for (const auto& kv : g->sparse_initializers()) sn.push_back(kv.first);
        std::sort(sn.begin(), sn.end());
        for (size_t i = 0; i < sn.size(); ++i) {
            const SparseInitializer& s = g->sparse_initializers().at(sn[i]);
            o << (i ? "," : "") << jstr(sn[i]) << ":{\"format\":"
              << (s.format == SparseInitializer::Csr ? "\"csr\"" : "\"2:4\"") << ",\"dtype\":" << (int)s.dtype
              << ",\"shape\":[" << s.rows << "," << s.cols << "],\"nnz\":" << s.nnz()
              << ",\"stored_bytes\":" << s.stored_bytes() << ",\"scales\":" << s.scales.size()
              << ",\"scale_axis\":" << s.scale_axis << "}";
        }
        o << "},\"total_initializer_bytes\":" << g->total_initializer_bytes();
        o << ",\"nodes\":[";
        auto order = g->topological_sort();
        for (size_t i = 0; i < order.size(); ++i) {
            const Node& n = *order[i];
            o << (i ? "," : "") << "{\"name\":" << jstr(n.name()) << ",\"op\":" << jstr(n.op_type())
              << ",\"inputs\":[";
            for (size_t j = 0; j < n.inputs().size(); ++j) o << (j ? "," : "") << jstr(n.inputs()[j]);
            o << "],\"outputs\":[";
            for (size_t j = 0; j < n.outputs().size(); ++j) o << (j ? "," : "") << jstr(n.outputs()[j]);
            o << "],\"attrs\":{";
            std::vector<std::string> an;
            for (const auto& kv : n.attributes()) an.push_back(kv.first);
            std::sort(an.begin(), an.end());
            for (size_t j = 0; j < an.size(); ++j)
                o << (j ? "," : "") << jstr(an[j]) << ":" << jattr(n.attributes().at(an[j]));
            o << "}}";
        }
        o << "]}";
        const std::string s = o.str();
        if (needed) *needed = (int64_t)s.size() + 1;
        if (buf && cap > 0) {
            const size_t n = std::min((size_t)cap - 1, s.size());
            std::memcpy(buf, s.data(), n);
            buf[n] = '\0';
        }
    });
}

int pfr_model_quantize(const char* in_path, const char* out_path, const char* mode, int* rewritten) {
    return guard([&] {
        if (!in_path || !out_path || !mode) throw PyFlameRTError("null argument");
        if (std::string(mode) != "dynamic_int8")
            throw PyFlameRTError(std::string("Invalid quantization mode: ") + mode + " (supported: dynamic_int8)");
        auto g = load_model(in_path);
        auto errs = g->validate();
        if (!errs.empty()) throw ValidationError(errs);
        QuantizeStats st;
        auto q = quantize_dynamic_int8(*g, &st);
        errs = q->validate();
        if (!errs.empty()) throw ValidationError(errs);
        save_model(*q, out_path);
        if (rewritten) *rewritten = st.rewritten;
    });
}

int pfr_model_resave(const char* in_path, const char* out_path) {
    return guard([&] {
        if (!in_path || !out_path) throw PyFlameRTError("null path");
        auto g = load_model(in_path);
        save_model(*g, out_path);
    });
}

int pfr_session_supported_ops(pfr_session* s, char* buf, int64_t cap) {
    return guard([&] {
        if (!s || !buf || cap <= 0) throw PyFlameRTError("null argument");
        std::string r = s->sess->backend().name();
        for (const auto& op : s->sess->backend().get_supported_ops()) r += "\n" + op;
        const size_t n = std::min((size_t)cap - 1, r.size());
        std::memcpy(buf, r.data(), n);
        buf[n] = '\0';
    });
}

int pfr_session_device_plan(pfr_session* s, int* device_resident, int* steps) {
    return guard([&] {
        if (!s || !device_resident || !steps) throw PyFlameRTError("null argument");
        auto* ex = dynamic_cast<RocmExecutor*>(&s->sess->backend());
        *device_resident = ex && ex->device_plan() ? 1 : 0;
        *steps = *device_resident ? (int)ex->device_plan_steps() : 0;
    });
}

int pfr_session_weight_forms(pfr_session* s, int* csr, int* dense, int* sp24) {
    return guard([&] {
        if (!s || !csr || !dense || !sp24) throw PyFlameRTError("null argument");
        auto* ex = dynamic_cast<RocmExecutor*>(&s->sess->backend());
        if (ex) ex->weight_forms(csr, dense, sp24);
        else *csr = *dense = *sp24 = 0;
    });
}

}  // extern "C"
