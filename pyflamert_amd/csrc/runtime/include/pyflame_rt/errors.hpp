// Exception types of the runtime, with the reference's class names and
// message forms (include/pyflame_rt/errors.hpp) so callers catch the same
// types.  Paths in messages keep only the file name.
#pragma once

#include <exception>
#include <optional>
#include <string>
#include <vector>

namespace pyflame_rt {

inline std::string sanitize_path_for_error(const std::string& path) {
    const size_t p = path.find_last_of("/\\");
    return p == std::string::npos ? path : path.substr(p + 1);
}

class PyFlameRTError : public std::exception {
public:
    explicit PyFlameRTError(std::string m) : message_(std::move(m)) {}
    const char* what() const noexcept override { return message_.c_str(); }

protected:
    std::string message_;
};

class InvalidModelError : public PyFlameRTError {
public:
    explicit InvalidModelError(const std::string& m, std::optional<std::string> path = std::nullopt)
        : PyFlameRTError(path ? m + " (file: " + sanitize_path_for_error(*path) + ")" : m) {}
};

class UnsupportedFormatError : public PyFlameRTError {
public:
    UnsupportedFormatError(const std::string& fmt, const std::vector<std::string>& supported)
        : PyFlameRTError(build(fmt, supported)) {}

private:
    static std::string build(const std::string& f, const std::vector<std::string>& s) {
        std::string m = "Unsupported format: '" + f + "'. Supported: ";
        for (size_t i = 0; i < s.size(); ++i) m += (i ? ", " : "") + s[i];
        return m;
    }
};

class UnsupportedOperatorError : public PyFlameRTError {
public:
    UnsupportedOperatorError(const std::string& op, const std::string& backend)
        : PyFlameRTError("Operator '" + op + "' is not supported by the '" + backend + "' backend"),
          op_type_(op) {}
    const std::string& op_type() const { return op_type_; }

private:
    std::string op_type_;
};

class ShapeMismatchError : public PyFlameRTError {
public:
    ShapeMismatchError(const std::string& name, const std::string& expected, const std::string& got)
        : PyFlameRTError("Shape mismatch for '" + name + "': expected " + expected + ", got " + got) {}
};

class ValidationError : public PyFlameRTError {
public:
    explicit ValidationError(const std::vector<std::string>& errors)
        : PyFlameRTError(build(errors)), errors_(errors) {}
    const std::vector<std::string>& errors() const { return errors_; }

private:
    static std::string build(const std::vector<std::string>& e) {
        std::string m = "Graph validation failed:\n";
        for (const auto& x : e) m += "  - " + x + "\n";
        return m;
    }
    std::vector<std::string> errors_;
};

class InputError : public PyFlameRTError {
public:
    explicit InputError(const std::string& m) : PyFlameRTError(m) {}
};

// Message "[node] text" when a node name is given (errors.hpp:157-170).
class BackendError : public PyFlameRTError {
public:
    explicit BackendError(const std::string& m, std::optional<std::string> node = std::nullopt)
        : PyFlameRTError(node ? "[" + *node + "] " + m : m), node_(std::move(node)) {}
    const std::optional<std::string>& node_name() const { return node_; }

private:
    std::optional<std::string> node_;
};

}  // namespace pyflame_rt
