#pragma once
// cli_engine_factory.hpp — nn::cli::create_engine, shaped as the reference's
// (include/neuralnet.cpp/cli/cli_engine_factory.hpp:32-77): the same EngineConfig fields, the same
// Result<std::shared_ptr<ComputeEngine>> and the same log stream argument, so a call site written
// for the reference compiles unchanged. The explicitly requested backend is created or an error is
// returned; a GPU request never falls back to the CPU. libnn-hip.so carries the HIP engine only:
// use_gpu selects it (gpu_device: "" or an index such as "0" / "hip:1"), and a CPU request is an
// error here (the reference's CPU engine lives in libnn-cpu.so).

#include <iostream>
#include <memory>
#include <string>

#include "compute_engine.hpp"
#include "hip_engine.hpp"

namespace nn::cli
{

struct EngineConfig
{
    bool use_gpu = false;            // --gpu: the HIP engine of this library
    std::string gpu_device = {};     // "", "0", "hip:1", ...
};

[[nodiscard]] inline Result<std::shared_ptr<ComputeEngine>> create_engine(const EngineConfig& cfg,
                                                                         std::ostream& log = std::cerr)
{
    if (!cfg.use_gpu)
        return Error{"create_engine: libnn-hip.so provides only the HIP engine (request use_gpu); "
                     "the CPU engine is libnn-cpu.so's"};
    std::unique_ptr<ComputeEngine> e = create_hip_engine(cfg.gpu_device.c_str());
    if (!e)
        return Error{std::string("create_engine: GPU requested but the HIP engine failed to start: ") + last_error() +
                     " (no fallback to the CPU)"};
    log << "GPU acceleration enabled (HIP engine: " << e->describe().device << ")\n\n";
    return std::shared_ptr<ComputeEngine>(std::move(e));
}

}  // namespace nn::cli
