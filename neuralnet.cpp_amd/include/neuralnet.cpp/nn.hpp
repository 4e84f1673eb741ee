#pragma once
// nn.hpp — umbrella header of the libnn-hip.so C++ layer (the reference exposes the same
// names through its C++ modules nn.core / nn.engine / nn.layer / nn.model / nn.cli).
#include "cli_engine_factory.hpp"
#include "compute_engine.hpp"
#include "decoder.hpp"
#include "hip_engine.hpp"
#include "int8_pack.hpp"
#include "layers.hpp"
#include "matrix.hpp"
#include "model_container.hpp"
#include "model_serialization.hpp"
#include "precision.hpp"
#include "result.hpp"
#include "sha256.hpp"
#include "ternary_pack.hpp"
