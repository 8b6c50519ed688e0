// Operator registry: the kernel plug-in interface of PyFlameRT.  OpContext,
// OpFunc and OperatorRegistry have the reference's signatures
// (include/pyflame_rt/registry.hpp:14-70) so backends register kernels the
// same way.  The ROCm backend registers its kernels under "rocm::<OpType>".
#pragma once

#include <functional>
#include <string>
#include <unordered_map>
#include <vector>

#include "pyflame_rt/node.hpp"
#include "pyflame_rt/tensor.hpp"

namespace pyflame_rt {

struct OpContext {
    const Node* node;
    bool strict_math_mode = false;
};

using OpFunc = std::function<std::vector<Tensor>(const std::vector<const Tensor*>& inputs, const OpContext& ctx)>;

class OperatorRegistry {
public:
    static OperatorRegistry& instance();
    void register_op(const std::string& op_type, OpFunc impl) { ops_[op_type] = std::move(impl); }
    const OpFunc* get(const std::string& op_type) const {
        auto it = ops_.find(op_type);
        return it == ops_.end() ? nullptr : &it->second;
    }
    bool has(const std::string& op_type) const { return ops_.count(op_type) > 0; }
    std::vector<std::string> list_ops() const;
    bool unregister_op(const std::string& op_type) { return ops_.erase(op_type) > 0; }
    void clear() { ops_.clear(); }

private:
    OperatorRegistry() = default;
    std::unordered_map<std::string, OpFunc> ops_;
};

class OpRegistrar {
public:
    OpRegistrar(const std::string& op_type, OpFunc impl) {
        OperatorRegistry::instance().register_op(op_type, std::move(impl));
    }
};

}  // namespace pyflame_rt
