// model_serialization.cpp — v7 / v8 model files: host-side parsing with untrusted-length checks
// before any allocation, the v8 sha256 tail, and the bridge between byte entries and the
// layers' ParamEntry protocol. The file layout is summarized in model_serialization.hpp.
#include "neuralnet.cpp/model_serialization.hpp"

#include <array>
#include <bit>
#include <cstring>
#include <fstream>
#include <string_view>

#include "neuralnet.cpp/sha256.hpp"
#include "neuralnet.cpp/ternary_pack.hpp"

namespace nn
{

namespace
{

constexpr std::string_view kTail = "NNEND";
constexpr std::size_t kTailBytes = 32 + 5;
constexpr std::uint64_t kMaxStringBytes = 64ull << 20;  // spec / tokenizer bound, as the reference

// ---- bounded little-endian reader over the file bytes
struct Reader
{
    const std::vector<std::uint8_t>& buf;
    std::size_t pos;
    std::size_t end;  // first byte that may not be read (the v8 tail)

    template <class T>
    Result<T> get(const char* what)
    {
        if (end - pos < sizeof(T)) return Error{std::string("model file truncated while reading ") + what};
        T v;
        std::memcpy(&v, buf.data() + pos, sizeof(T));
        pos += sizeof(T);
        return v;
    }
    Result<void> bytes(std::uint64_t n, std::vector<std::uint8_t>& out, const char* what)
    {
        if (n > end - pos) return Error{std::string("model file: ") + what + " length exceeds the file (corrupt?)"};
        out.assign(buf.begin() + static_cast<std::ptrdiff_t>(pos), buf.begin() + static_cast<std::ptrdiff_t>(pos + n));
        pos += static_cast<std::size_t>(n);
        return {};
    }
};

template <class T>
void put(std::string& out, T v)
{
    char b[sizeof(T)];
    std::memcpy(b, &v, sizeof(T));
    out.append(b, sizeof(T));
}

// IEEE binary16 -> binary32 (exact for every input, NaN payloads kept in the high bits)
float half_to_float(std::uint16_t h)
{
    const std::uint32_t sign = (std::uint32_t(h) & 0x8000u) << 16;
    std::uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
    if (exp == 0x1F) bits = sign | 0x7F800000u | (man << 13);
    else if (exp != 0) bits = sign | ((exp + 112u) << 23) | (man << 13);
    else if (man == 0) bits = sign;
    else
    {
        int e = -1;
        do
        {
            man <<= 1;
            ++e;
        } while ((man & 0x400u) == 0);
        bits = sign | (std::uint32_t(112 - e) << 23) | ((man & 0x3FFu) << 13);
    }
    return std::bit_cast<float>(bits);
}

Result<ParamBlob> read_blob(Reader& r)
{
    ParamBlob b;
    EX_TRY(kind, r.get<std::uint8_t>("entry kind"));
    if (*kind > static_cast<std::uint8_t>(ParamKind::I8Packed4))
        return Error{"model file: invalid entry kind " + std::to_string(*kind)};
    b.kind = static_cast<ParamKind>(*kind);
    EX_TRY(tag, r.get<std::uint8_t>("entry precision"));
    b.precision_tag = *tag;
    EX_TRY(rows, r.get<std::uint64_t>("entry rows"));
    EX_TRY(cols, r.get<std::uint64_t>("entry cols"));
    EX_TRY(alen, r.get<std::uint64_t>("entry aux length"));
    EX_TRY(plen, r.get<std::uint64_t>("entry payload length"));
    b.rows = *rows;
    b.cols = *cols;
    EX_TRY_CHECK(r.bytes(*alen, b.aux, "entry aux"));
    EX_TRY_CHECK(r.bytes(*plen, b.payload, "entry payload"));
    return b;
}

std::string shape_of(const ParamBlob& b) { return std::to_string(b.rows) + "x" + std::to_string(b.cols); }

// entry bytes -> device tensors
Result<ParamEntry> to_entry(ComputeEngine& engine, const ParamBlob& b)
{
    ParamEntry e;
    e.kind = b.kind;
    e.rows = static_cast<std::size_t>(b.rows);
    e.cols = static_cast<std::size_t>(b.cols);
    e.precision = Precision::F32;
    if (b.rows > (1ull << 31) || b.cols > (1ull << 31)) return Error{"model file: entry shape " + shape_of(b) + " too large"};
    switch (b.kind)
    {
    case ParamKind::Dense:
    case ParamKind::TernaryLatent:
    {
        Matrix m(e.rows, e.cols);
        const std::size_t n = m.size();
        if (b.precision_tag == kTagF32)
        {
            if (b.payload.size() != n * 4) return Error{"model file: f32 payload of " + shape_of(b) + " has the wrong length"};
            if (n) std::memcpy(m.data(), b.payload.data(), n * 4);
        }
        else if (b.precision_tag == kTagF16)
        {
            if (b.payload.size() != n * 2) return Error{"model file: f16 payload of " + shape_of(b) + " has the wrong length"};
            e.precision = Precision::F16;
            for (std::size_t i = 0; i < n; ++i)
            {
                std::uint16_t h;
                std::memcpy(&h, b.payload.data() + 2 * i, 2);
                m.data()[i] = half_to_float(h);
            }
        }
        else
            return Error{"model file: unsupported precision tag " + std::to_string(b.precision_tag) + " for a " +
                         param_kind_name(b.kind) + " entry"};
        EX_TRY(t, engine.from_matrix(m, Precision::F32));
        e.payload = *t;
        return e;
    }
    case ParamKind::TernaryPacked2:
    {
        const std::size_t K = e.cols, wpr = trit_pack::words_per_row(K), rows = e.rows;
        const std::size_t whole = wpr * 4, trimmed = (K + 3) / 4;
        std::size_t bpr;
        if (b.payload.size() == rows * whole) bpr = whole;
        else if (b.payload.size() == rows * trimmed) bpr = trimmed;
        else return Error{"model file: TernaryPacked2 payload of " + shape_of(b) + " has the wrong length"};
        if (b.aux.size() != rows * 4) return Error{"model file: TernaryPacked2 entry needs tau (rows f32) as aux"};
        Matrix words(rows, wpr);
        std::vector<std::uint8_t> row(whole);
        for (std::size_t r = 0; r < rows; ++r)
        {
            std::memset(row.data(), 0xAA, whole);  // code 2 in every byte the file does not carry
            std::memcpy(row.data(), b.payload.data() + r * bpr, bpr);
            std::memcpy(words.data() + r * wpr, row.data(), whole);  // raw bits, no float arithmetic
        }
        Matrix tau(rows, 1);
        if (rows) std::memcpy(tau.data(), b.aux.data(), rows * 4);
        EX_TRY(pw, engine.from_matrix(words, Precision::F32));
        EX_TRY(pt, engine.from_matrix(tau, Precision::F32));
        e.payload = *pw;
        e.aux = *pt;
        return e;
    }
    case ParamKind::TernaryPacked3:
        return Error{"model file: TernaryPacked3 (base-3) entries are not supported: their byte layout is not "
                     "fixed by the reference tree; re-export the weights as TernaryPacked2"};
    default:
        return Error{std::string("model file: entry kind ") + param_kind_name(b.kind) + " is not supported"};
    }
}

Result<ParamBlob> to_blob(ComputeEngine& engine, const ParamEntry& e)
{
    ParamBlob b;
    b.kind = e.kind;
    b.rows = e.rows;
    b.cols = e.cols;
    b.precision_tag = kTagF32;
    auto bytes_of = [&engine](const Tensor& t, std::vector<std::uint8_t>& out) -> Result<void> {
        EX_TRY(m, engine.to_matrix(t, Precision::F32));
        out.resize(m->size() * 4);
        if (m->size()) std::memcpy(out.data(), m->data(), out.size());
        return {};
    };
    switch (e.kind)
    {
    case ParamKind::Dense:
    case ParamKind::TernaryLatent:
        EX_TRY_CHECK(bytes_of(e.payload, b.payload));
        return b;
    case ParamKind::TernaryPacked2:
        if (e.payload.rows() != e.rows || e.payload.cols() != trit_pack::words_per_row(e.cols))
            return Error{"save_model: packed container shape does not match the entry"};
        EX_TRY_CHECK(bytes_of(e.payload, b.payload));
        EX_TRY_CHECK(bytes_of(e.aux, b.aux));
        return b;
    default:
        return Error{std::string("save_model: entry kind ") + param_kind_name(e.kind) + " cannot be written"};
    }
}

std::size_t total_params(Model& model)
{
    std::size_t n = 0;
    for (std::size_t i = 0; i < model.num_layers(); ++i) n += model.layer_at(i).param_count();
    return n;
}

}  // namespace

Result<ModelFile> read_model_file(const std::string& filename, std::size_t n_params)
{
    std::ifstream f(filename, std::ios::binary | std::ios::ate);
    if (!f) return Error{"cannot open model file " + filename};
    const std::streamoff size = f.tellg();
    if (size < 0) return Error{"cannot size model file " + filename};
    std::vector<std::uint8_t> buf(static_cast<std::size_t>(size));
    f.seekg(0);
    if (size > 0 && !f.read(reinterpret_cast<char*>(buf.data()), size)) return Error{"cannot read model file " + filename};

    ModelFile out;
    Reader r{buf, 0, buf.size()};
    EX_TRY(magic, r.get<std::uint32_t>("magic"));
    if (*magic != kModelMagic) return Error{filename + ": not a model file (bad magic)"};
    EX_TRY(version, r.get<std::uint32_t>("version"));
    out.version = *version;
    if (out.version < 7)
        return Error{filename + ": format v" + std::to_string(out.version) +
                     " stores flat matrices; this loader reads the per-parameter entries of v7 and v8"};
    if (out.version > kModelVersion) return Error{filename + ": format v" + std::to_string(out.version) + " is newer than v8"};
    EX_TRY(prec, r.get<std::uint8_t>("precision"));
    if (*prec != 0) return Error{filename + ": file was written with f64 scalars; this build uses f32"};
    EX_TRY(role, r.get<std::uint8_t>("role"));
    if (*role > 1) return Error{filename + ": invalid role byte"};
    out.role = static_cast<ModelRole>(*role);

    if (out.version >= 8)
    {
        if (buf.size() < r.pos + kTailBytes) return Error{filename + ": too short for the integrity tail"};
        const std::size_t body = buf.size() - kTailBytes;
        if (std::memcmp(buf.data() + body + 32, kTail.data(), kTail.size()) != 0)
            return Error{filename + ": missing the NNEND tail (truncated or damaged)"};
        Sha256 h;
        h.update(buf.data(), body);
        const auto d = h.digest();
        if (std::memcmp(d.data(), buf.data() + body, 32) != 0) return Error{filename + ": checksum mismatch (damaged file)"};
        r.end = body;
    }

    EX_TRY(spec_len, r.get<std::uint64_t>("spec length"));
    if (*spec_len > kMaxStringBytes) return Error{filename + ": spec length out of range"};
    std::vector<std::uint8_t> tmp;
    EX_TRY_CHECK(r.bytes(*spec_len, tmp, "spec"));
    out.spec.assign(tmp.begin(), tmp.end());
    if (out.version >= 8)
    {
        EX_TRY(state_len, r.get<std::uint64_t>("training-state length"));
        if (*state_len != 0)
            return Error{filename + ": the file carries a training-state section, which this loader does not read"};
    }
    out.params.reserve(n_params);
    for (std::size_t i = 0; i < n_params; ++i)
    {
        EX_TRY(b, read_blob(r));
        out.params.push_back(std::move(*b));
    }
    EX_TRY(tok_len, r.get<std::uint64_t>("tokenizer length"));
    if (*tok_len > kMaxStringBytes) return Error{filename + ": tokenizer length out of range"};
    EX_TRY_CHECK(r.bytes(*tok_len, tmp, "tokenizer"));
    out.tokenizer.assign(tmp.begin(), tmp.end());
    if (r.pos != r.end)
        return Error{filename + ": " + std::to_string(r.end - r.pos) +
                     " bytes left after the tokenizer (the file has more entries than the model's layers)"};
    return out;
}

Result<std::string> load_model(const std::string& filename, Model& model, std::uint32_t* version_out, ModelRole* role_out)
{
    EX_TRY(file, read_model_file(filename, total_params(model)));
    if (version_out) *version_out = file->version;
    if (role_out) *role_out = file->role;
    std::size_t k = 0;
    for (std::size_t li = 0; li < model.num_layers(); ++li)
    {
        Layer& L = model.layer_at(li);
        for (std::size_t i = 0; i < L.param_count(); ++i, ++k)
        {
            EX_TRY(e, to_entry(model.engine(), file->params[k]));
            auto ok = L.import_param(i, *e);
            if (!ok)
                return Error{std::string(L.layer_name()) + " (layer " + std::to_string(li) + ", entry " + std::to_string(i) +
                             "): " + ok.error().message};
        }
    }
    return file->tokenizer;
}

Result<void> save_model(const std::string& filename, Model& model, ModelRole role, const std::string& spec,
                        const std::string& tokenizer)
{
    std::string out;
    put<std::uint32_t>(out, kModelMagic);
    put<std::uint32_t>(out, kModelVersion);
    put<std::uint8_t>(out, 0);  // f32 scalars
    put<std::uint8_t>(out, static_cast<std::uint8_t>(role));
    put<std::uint64_t>(out, spec.size());
    out += spec;
    put<std::uint64_t>(out, 0);  // no training-state section
    for (std::size_t li = 0; li < model.num_layers(); ++li)
    {
        Layer& L = model.layer_at(li);
        for (std::size_t i = 0; i < L.param_count(); ++i)
        {
            EX_TRY(e, L.export_param(i, role));
            EX_TRY(b, to_blob(model.engine(), *e));
            put<std::uint8_t>(out, static_cast<std::uint8_t>(b->kind));
            put<std::uint8_t>(out, b->precision_tag);
            put<std::uint64_t>(out, b->rows);
            put<std::uint64_t>(out, b->cols);
            put<std::uint64_t>(out, b->aux.size());
            put<std::uint64_t>(out, b->payload.size());
            out.append(reinterpret_cast<const char*>(b->aux.data()), b->aux.size());
            out.append(reinterpret_cast<const char*>(b->payload.data()), b->payload.size());
        }
    }
    put<std::uint64_t>(out, tokenizer.size());
    out += tokenizer;
    Sha256 h;
    h.update(out.data(), out.size());
    const auto d = h.digest();
    out.append(reinterpret_cast<const char*>(d.data()), d.size());
    out.append(kTail.data(), kTail.size());
    std::ofstream f(filename, std::ios::binary | std::ios::trunc);
    if (!f) return Error{"cannot open " + filename + " for writing"};
    f.write(out.data(), static_cast<std::streamsize>(out.size()));
    if (!f) return Error{"write error on " + filename};
    return {};
}

}  // namespace nn
