#pragma once
// cli_engine_factory.hpp — nn::cli::create_engine with a HIP branch.
// Mirrors cli/cli_engine_factory.hpp:32-77: the requested backend is created or an error is
// returned; an explicitly requested GPU backend never silently falls back to the CPU.
// libnn-hip.so carries only the HIP engine, so use_gpu / use_hip both select it, and a CPU
// request is an error here (the reference's CPU engine lives in libnn-cpu.so).

#include <memory>
#include <string>

#include "compute_engine.hpp"
#include "hip_engine.hpp"

namespace nn::cli
{

struct EngineConfig
{
    bool use_gpu = false;   // reference flag (--gpu); on this build it selects the HIP engine
    bool use_hip = false;   // --hip
    std::string device;     // "", "0", "hip:1", ...
};

[[nodiscard]] inline Result<std::unique_ptr<ComputeEngine>> create_engine(const EngineConfig& cfg)
{
    if (!cfg.use_gpu && !cfg.use_hip)
        return Error{"create_engine: libnn-hip.so provides only the HIP engine (request use_hip)"};
    auto e = create_hip_engine(cfg.device.c_str());
    if (!e) return Error{std::string("create_engine: HIP engine unavailable: ") + last_error()};
    return std::unique_ptr<ComputeEngine>(std::move(e));
}

}  // namespace nn::cli
