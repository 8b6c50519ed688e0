// Session and run options (include/pyflame_rt/options.hpp:16-67 of the
// reference) with "rocm" added to the accepted devices.
#pragma once

#include <optional>
#include <string>
#include <vector>

#include "pyflame_rt/types.hpp"

namespace pyflame_rt {

struct SessionOptions {
    std::string device = "cpu";  // "cpu", "wse", "wse2", "wse3", "rocm"
    int num_threads = 0;
    bool enable_profiling = false;
    std::optional<int> memory_limit_mb;
    std::string execution_mode = "sequential";
    OptLevel optimization_level = OptLevel::Extended;
    bool strict_math_mode = false;
    std::string log_level = "warning";
    // rocm: 0 = strict (bit-exact fp32 sums, the default), 1 = fast (fused
    // multiply-add in the same order).
    int rocm_math_mode = 0;
    int rocm_device_id = 0;
    // The reference's SessionOptions::quantization (a QuantConfig,
    // include/pyflame_rt/options.hpp) reduced to its mode: "" for none, or
    // "dynamic_int8" (QuantMode::DynamicInt8 with per-channel weights): the
    // 2:4-pruned MatMul(W, X) nodes run as DynamicQuantizeLinear +
    // QuantizedMatMul (quantize.hpp).
    std::string quantization;

    std::vector<std::string> validate() const;
};

struct RunOptions {
    std::optional<std::string> log_level;
    std::optional<std::string> tag;
    std::optional<int> timeout_ms;
};

}  // namespace pyflame_rt
