// Tensor, Graph, OperatorRegistry, Backend::validate_inputs and
// SessionOptions::validate.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <queue>
#include <unordered_set>

#include "pyflame_rt/backend.hpp"
#include "pyflame_rt/errors.hpp"
#include "pyflame_rt/graph.hpp"
#include "pyflame_rt/options.hpp"
#include "pyflame_rt/registry.hpp"
#include "pyflame_rt/tensor.hpp"

namespace pyflame_rt {

// ---- Tensor -----------------------------------------------------------------

namespace {
void check_shape(const std::vector<int64_t>& s) {
    for (size_t i = 0; i < s.size(); ++i)
        if (s[i] < 0)
            throw std::invalid_argument("Negative dimension at axis " + std::to_string(i) + ": " +
                                        std::to_string(s[i]));
}

std::shared_ptr<void> alloc64(size_t bytes) {
    const size_t rounded = (bytes + 63) / 64 * 64;
    void* p = std::aligned_alloc(64, rounded);
    if (!p) throw std::bad_alloc();
    std::memset(p, 0, rounded);
    return std::shared_ptr<void>(p, [](void* q) { std::free(q); });
}
}  // namespace

Tensor::Tensor(const std::vector<int64_t>& shape, DType dtype) : shape_(shape), dtype_(dtype) {
    check_shape(shape_);
    const size_t b = size_bytes();
    if (b) {
        owned_ = alloc64(b);
        data_ = owned_.get();
    }
}

Tensor::Tensor(void* data, const std::vector<int64_t>& shape, DType dtype)
    : data_(data), shape_(shape), dtype_(dtype) {}

Tensor::Tensor(const Tensor& o) : shape_(o.shape_), dtype_(o.dtype_) {
    if (o.is_valid() && o.size_bytes()) {
        owned_ = alloc64(o.size_bytes());
        data_ = owned_.get();
        std::memcpy(data_, o.data_, o.size_bytes());
    }
}

Tensor::Tensor(Tensor&& o) noexcept
    : data_(o.data_), shape_(std::move(o.shape_)), dtype_(o.dtype_), owned_(std::move(o.owned_)) {
    o.data_ = nullptr;
}

Tensor& Tensor::operator=(const Tensor& o) {
    if (this != &o) {
        Tensor t(o);
        *this = std::move(t);
    }
    return *this;
}

Tensor& Tensor::operator=(Tensor&& o) noexcept {
    if (this != &o) {
        data_ = o.data_;
        shape_ = std::move(o.shape_);
        dtype_ = o.dtype_;
        owned_ = std::move(o.owned_);
        o.data_ = nullptr;
    }
    return *this;
}

void Tensor::zero() {
    if (is_valid()) std::memset(data_, 0, size_bytes());
}

Tensor Tensor::reshape(const std::vector<int64_t>& s) const {
    check_shape(s);
    if (checked_product(s) != num_elements()) throw std::invalid_argument("reshape: element count differs");
    Tensor t = *this;
    t.shape_ = s;
    return t;
}

// ---- Graph ------------------------------------------------------------------

void Graph::add_node(std::shared_ptr<Node> node) {
    if (node_map_.count(node->name()))
        throw std::invalid_argument("Node '" + node->name() + "' already exists in graph");
    if (nodes_.size() >= limits_.max_nodes)
        throw std::runtime_error("Graph node limit exceeded: max " + std::to_string(limits_.max_nodes) +
                                 " nodes allowed");
    nodes_.push_back(node);
    node_map_[node->name()] = node;
    for (const auto& o : node->outputs()) producers_[o] = node->name();
}

const Node* Graph::get_node(const std::string& name) const {
    auto it = node_map_.find(name);
    return it == node_map_.end() ? nullptr : it->second.get();
}

void Graph::add_initializer(const std::string& name, Tensor t) {
    if (sparse_.count(name)) throw std::runtime_error("Initializer '" + name + "' is already a sparse initializer");
    if (initializers_.size() + sparse_.size() >= limits_.max_initializers && !initializers_.count(name))
        throw std::runtime_error("Graph initializer limit exceeded: max " +
                                 std::to_string(limits_.max_initializers) + " initializers allowed");
    size_t base = init_bytes_;
    auto it = initializers_.find(name);
    if (it != initializers_.end()) base -= it->second.size_bytes();
    if (base + t.size_bytes() > limits_.max_initializer_bytes)
        throw std::runtime_error("Graph initializer memory limit exceeded: max " +
                                 std::to_string(limits_.max_initializer_bytes / (1024 * 1024)) + " MB allowed");
    init_bytes_ = base + t.size_bytes();
    initializers_[name] = std::move(t);
}

void Graph::add_sparse_initializer(const std::string& name, SparseInitializer s) {
    if (initializers_.count(name)) throw std::runtime_error("Initializer '" + name + "' is already a dense initializer");
    if (initializers_.size() + sparse_.size() >= limits_.max_initializers && !sparse_.count(name))
        throw std::runtime_error("Graph initializer limit exceeded: max " +
                                 std::to_string(limits_.max_initializers) + " initializers allowed");
    s.validate(name);
    size_t base = init_bytes_;
    auto it = sparse_.find(name);
    if (it != sparse_.end()) base -= it->second.stored_bytes();
    if (base + s.stored_bytes() > limits_.max_initializer_bytes)
        throw std::runtime_error("Graph initializer memory limit exceeded: max " +
                                 std::to_string(limits_.max_initializer_bytes / (1024 * 1024)) + " MB allowed");
    init_bytes_ = base + s.stored_bytes();
    sparse_[name] = std::move(s);
}

const SparseInitializer* Graph::get_sparse_initializer(const std::string& name) const {
    auto it = sparse_.find(name);
    return it == sparse_.end() ? nullptr : &it->second;
}

std::optional<std::reference_wrapper<const Tensor>> Graph::get_initializer(const std::string& name) const {
    auto it = initializers_.find(name);
    if (it == initializers_.end()) return std::nullopt;
    return std::cref(it->second);
}

const std::string* Graph::get_producer(const std::string& t) const {
    auto it = producers_.find(t);
    return it == producers_.end() ? nullptr : &it->second;
}

// Kahn's algorithm (src/graph.cpp:115-164); ties broken by node insertion
// order so the order is deterministic.
std::vector<std::shared_ptr<Node>> Graph::topological_sort() const {
    std::unordered_map<std::string, size_t> index;
    for (size_t i = 0; i < nodes_.size(); ++i) index[nodes_[i]->name()] = i;
    std::vector<int> indeg(nodes_.size(), 0);
    std::vector<std::vector<size_t>> deps(nodes_.size());
    for (size_t i = 0; i < nodes_.size(); ++i)
        for (const auto& in : nodes_[i]->inputs()) {
            const std::string* p = get_producer(in);
            if (p && index.count(*p)) {
                ++indeg[i];
                deps[index[*p]].push_back(i);
            }
        }
    std::queue<size_t> q;
    for (size_t i = 0; i < nodes_.size(); ++i)
        if (indeg[i] == 0) q.push(i);
    std::vector<std::shared_ptr<Node>> out;
    out.reserve(nodes_.size());
    while (!q.empty()) {
        const size_t i = q.front();
        q.pop();
        out.push_back(nodes_[i]);
        for (size_t d : deps[i])
            if (--indeg[d] == 0) q.push(d);
    }
    if (out.size() != nodes_.size()) throw ValidationError({"Graph contains a cycle"});
    return out;
}

std::vector<std::string> Graph::validate() const {
    std::vector<std::string> errors;
    std::unordered_set<std::string> avail;
    for (const auto& i : inputs_) avail.insert(i.name);
    for (const auto& kv : initializers_) avail.insert(kv.first);
    for (const auto& kv : sparse_) avail.insert(kv.first);
    std::vector<std::shared_ptr<Node>> sorted;
    try {
        sorted = topological_sort();
    } catch (const ValidationError& e) {
        return e.errors();
    }
    for (const auto& n : sorted) {
        for (const auto& in : n->inputs())
            if (!avail.count(in)) errors.push_back("Node '" + n->name() + "' input '" + in + "' not found");
        for (const auto& o : n->outputs()) avail.insert(o);
    }
    for (const auto& o : outputs_)
        if (!avail.count(o.name)) errors.push_back("Graph output '" + o.name + "' not produced");
    return errors;
}

// ---- OperatorRegistry ---------------------------------------------------------

OperatorRegistry& OperatorRegistry::instance() {
    static OperatorRegistry r;
    return r;
}

std::vector<std::string> OperatorRegistry::list_ops() const {
    std::vector<std::string> r;
    r.reserve(ops_.size());
    for (const auto& kv : ops_) r.push_back(kv.first);
    std::sort(r.begin(), r.end());
    return r;
}

// ---- Backend ------------------------------------------------------------------

void Backend::validate_inputs(const Graph& graph, const std::unordered_map<std::string, Tensor>& feed) const {
    std::unordered_set<std::string> expected;
    for (const auto& i : graph.inputs()) expected.insert(i.name);
    for (const auto& n : expected)
        if (!feed.count(n)) throw InputError("Missing input: " + n);
    for (const auto& kv : feed)
        if (!expected.count(kv.first)) throw InputError("Unexpected input: " + kv.first);
    for (const auto& info : graph.inputs()) {
        const Tensor& t = feed.at(info.name);
        if (info.shape.size() != t.shape().size())
            throw ShapeMismatchError(info.name, shape_to_string(info.shape),
                                     "[" + std::to_string(t.shape().size()) + " dims]");
        for (size_t d = 0; d < info.shape.size(); ++d)
            if (info.shape[d] && *info.shape[d] != t.shape()[d]) {
                std::string got = "[";
                for (size_t j = 0; j < t.shape().size(); ++j) got += (j ? ", " : "") + std::to_string(t.shape()[j]);
                throw ShapeMismatchError(info.name, shape_to_string(info.shape), got + "]");
            }
    }
}

// ---- SessionOptions -----------------------------------------------------------

std::vector<std::string> SessionOptions::validate() const {
    std::vector<std::string> e;
    static const std::unordered_set<std::string> devices = {"cpu", "wse", "wse2", "wse3", "rocm"};
    if (!devices.count(device)) e.push_back("Invalid device: " + device);
    if (execution_mode != "sequential" && execution_mode != "parallel")
        e.push_back("Invalid execution_mode: " + execution_mode);
    static const std::unordered_set<std::string> levels = {"debug", "info", "warning", "error"};
    if (!levels.count(log_level)) e.push_back("Invalid log_level: " + log_level);
    if (num_threads < 0) e.push_back("num_threads must be >= 0");
    else if (num_threads > 256)
        e.push_back("num_threads must be <= 256 (got " + std::to_string(num_threads) + ")");
    if (rocm_math_mode != 0 && rocm_math_mode != 1) e.push_back("rocm_math_mode must be 0 (strict) or 1 (fast)");
    if (rocm_device_id < 0) e.push_back("rocm_device_id must be >= 0");
    if (!quantization.empty() && quantization != "dynamic_int8")
        e.push_back("Invalid quantization mode: " + quantization + " (supported: dynamic_int8)");
    return e;
}

}  // namespace pyflame_rt
