#pragma once
// model_serialization.hpp — reading and writing neuralnet.cpp model files (v7 / v8) for the
// BitLinear path: the header, the per-parameter entries and the v8 integrity tail.
//
// Layout (include/neuralnet.cpp/model_serialization.hpp:38-82, little-endian):
//   [magic u32 = 0x4E4E4E4E "NNNN"][version u32][precision u8 (0 = f32)][role u8 (v7+)]
//   [spec_len u64][spec bytes]                       (a KeyValueRecord; skipped here)
//   [state_len u64][state bytes][optimizer entries]  (v8; a Model-role file has state_len 0)
//   [param entries ...]                              (one per layer parameter, layer order)
//   [extra state entries ...]                        (none for the layers of this path)
//   [tokenizer_len u64][tokenizer bytes]
//   [sha256 32B]["NNEND"]                            (v8; the digest covers every byte before it)
// Param entry (:579-590, :640-700):
//   [kind u8][precision tag u8][rows u64][cols u64][aux_len u64][payload_len u64][aux][payload]
//   Dense / TernaryLatent: rows*cols elements (tag 0 = f32, 2 = f16);
//   TernaryPacked2: rows rows of 2-bit containers + aux = tau (rows f32);
//   TernaryPacked3: base-3 rows (5 trits per byte).
//
// What is read: Dense (f32/f16), TernaryLatent and TernaryPacked2 entries. TernaryPacked3 is
// refused: its byte layout (digit order, premultiplication) lives in the absent engine and
// no reference file or test fixes it. A v8 training-state section is refused too (its entry
// count sits in a KeyValueRecord whose format is not in the reference tree). The byte size of
// a TernaryPacked2 row for K % 16 != 0 is not fixed by the reference either; rows of whole
// words (ceil(K/16) * 4 bytes, what this writer emits) and rows trimmed to ceil(K/4) bytes
// are both accepted, the missing tail bytes read as code 2 (trit 0).

#include <cstdint>
#include <string>
#include <vector>

#include "layers.hpp"
#include "model_container.hpp"

namespace nn
{

inline constexpr std::uint32_t kModelMagic = 0x4E4E4E4Eu;  // "NNNN"
inline constexpr std::uint32_t kModelVersion = 8;

// per-entry precision tags (src/precision_type_test.cpp:388-392)
inline constexpr std::uint8_t kTagF32 = 0, kTagF16 = 2, kTagT158 = 4;

// One entry as bytes on the host.
struct ParamBlob
{
    ParamKind kind = ParamKind::Dense;
    std::uint8_t precision_tag = kTagF32;
    std::uint64_t rows = 0, cols = 0;
    std::vector<std::uint8_t> aux, payload;
};

// What a file holds, read on the host only (no engine): header fields, the opaque spec bytes,
// `n_params` entries (the caller's layer count decides), the tokenizer bytes.
struct ModelFile
{
    std::uint32_t version = 0;
    ModelRole role = ModelRole::Model;
    std::string spec;
    std::vector<ParamBlob> params;
    std::string tokenizer;
};

[[nodiscard]] Result<ModelFile> read_model_file(const std::string& filename, std::size_t n_params);

// Entries of every layer of `model`, in order, imported through Layer::import_param. Returns the
// embedded tokenizer bytes (empty when none). Mirrors load_model (:1175-1311) for v7 / v8.
[[nodiscard]] Result<std::string> load_model(const std::string& filename, Model& model,
                                             std::uint32_t* version_out = nullptr, ModelRole* role_out = nullptr);

// Writes a v8 file of `model` (:999-1073): Model role = ternary layers as TernaryPacked2 + tau
// (the reference writes base-3 there; see above), Checkpoint role = TernaryLatent. `spec` is
// written as given (opaque to this library), no training state, the sha256 tail at the end.
[[nodiscard]] Result<void> save_model(const std::string& filename, Model& model, ModelRole role = ModelRole::Model,
                                      const std::string& spec = {}, const std::string& tokenizer = {});

}  // namespace nn
