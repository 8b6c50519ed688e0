// Graph node: name, op type, input/output tensor names and typed attributes
// (the attribute variant and get_attr semantics of the reference,
// include/pyflame_rt/node.hpp:13-97: a missing or differently typed attribute
// yields the default).
#pragma once

#include <optional>
#include <string>
#include <unordered_map>
#include <variant>
#include <vector>

namespace pyflame_rt {

using AttributeValue = std::variant<int64_t, float, std::string, std::vector<int64_t>, std::vector<float>,
                                    std::vector<std::string>>;

class Node {
public:
    Node() = default;
    Node(std::string name, std::string op_type, std::vector<std::string> inputs, std::vector<std::string> outputs)
        : name_(std::move(name)), op_type_(std::move(op_type)), inputs_(std::move(inputs)),
          outputs_(std::move(outputs)) {}

    const std::string& name() const { return name_; }
    const std::string& op_type() const { return op_type_; }
    const std::vector<std::string>& inputs() const { return inputs_; }
    const std::vector<std::string>& outputs() const { return outputs_; }
    const std::unordered_map<std::string, AttributeValue>& attributes() const { return attributes_; }

    template <class T>
    T get_attr(const std::string& name, const T& def) const {
        auto it = attributes_.find(name);
        if (it == attributes_.end()) return def;
        if (auto* v = std::get_if<T>(&it->second)) return *v;
        return def;
    }
    template <class T>
    std::optional<T> get_attr(const std::string& name) const {
        auto it = attributes_.find(name);
        if (it == attributes_.end()) return std::nullopt;
        if (auto* v = std::get_if<T>(&it->second)) return *v;
        return std::nullopt;
    }
    void set_attr(const std::string& name, AttributeValue v) { attributes_[name] = std::move(v); }
    bool has_attr(const std::string& name) const { return attributes_.count(name) > 0; }

private:
    std::string name_, op_type_;
    std::vector<std::string> inputs_, outputs_;
    std::unordered_map<std::string, AttributeValue> attributes_;
};

}  // namespace pyflame_rt
