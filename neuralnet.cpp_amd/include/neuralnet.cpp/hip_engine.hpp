#pragma once
// hip_engine.hpp — factory of the MI355X engine in libnn-hip.so, the third engine next to the
// reference's libnn-cpu.so / libnn-gpu.so. Mirrors nn::create_gpu_engine(const char* device)
// and nn::last_error() (modules/nn.engine.cpp:36-48; cli/cli_engine_factory.hpp:51-76).
// The engine talks to the GPU only through the C ABI of include/nnhip.h.

#include <memory>

#include "compute_engine.hpp"

namespace nn
{

// device: nullptr, "", "0", "hip:1", ... (index of the HIP device). Returns nullptr on failure
// (no gfx950 device, HIP error); the reason is in last_error().
[[nodiscard]] std::unique_ptr<ComputeEngine> create_hip_engine(const char* device = nullptr);

// Message of the last failed factory call on this thread.
[[nodiscard]] const char* last_error() noexcept;

}  // namespace nn
