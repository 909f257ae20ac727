// model_file.hpp — the reference's model file, format v4 ("NNNN"), for GPT
// models (reference include/neuralnet.cpp/model_serialization.hpp:36-52 for
// the layout, :150-300 for matrices and the spec record, :380-503 for the
// save / load order; keyvalue_record.hpp:20-200 for the record encoding).
//
// Layout, all integers little-endian:
//   u32 magic "NNNN" (0x4E4E4E4E), u32 version 4, u8 precision (0 = f32),
//   u64 spec length, spec record,
//   per parameter in parameters() order: u64 rows, u64 cols, rows*cols f32,
//   (no extra-state matrices: a GPT has none),
//   u64 tokenizer length, tokenizer bytes (0 = none embedded).
// Spec record: u32 field count; per field u32 key length, key, u8 type
// (0 u64, 1 string, 2 u64 array), u32 value length, value. A GPT's spec holds
// the fields spec_to_kv writes, in its order (model_serialization.hpp:190-207).
#pragma once

#include <cstdint>
#include <cstring>
#include <fstream>
#include <string>
#include <string_view>
#include <vector>

#include "core_errors.hpp"
#include "matrix.hpp"

namespace nn::model_file
{

constexpr std::uint32_t kMagic = 0x4E4E4E4Eu, kVersion = 4;
constexpr std::uint8_t kPrecisionF32 = 0;
// ModelSpec enum values (reference model_spec.hpp:24-55).
constexpr std::uint64_t kTypeGpt = 3, kPosALiBi = 2, kActivationSwiGLU = 1, kNormRMSNorm = 1;

// The GPT fields of a ModelSpec. Fields a file leaves out keep ModelSpec's
// defaults (model_spec.hpp:58-77: pos_encoding Learned, activation GeLU,
// norm_type LayerNorm), as spec_from_kv leaves them (model_serialization.hpp:238-266).
struct GptSpec
{
    std::uint64_t d_model = 0, num_heads = 0, d_ff = 0, num_layers = 0, vocab_size = 0, seq_len = 0,
                  pos_encoding = 0, activation = 0, norm_type = 0, type = kTypeGpt;
};

inline void put_u32(std::string& o, std::uint32_t v)
{
    for (int i = 0; i < 4; ++i) o.push_back(static_cast<char>((v >> (8 * i)) & 0xff));
}
inline void put_u64(std::string& o, std::uint64_t v)
{
    for (int i = 0; i < 8; ++i) o.push_back(static_cast<char>((v >> (8 * i)) & 0xff));
}
inline bool take(std::string_view& s, std::uint64_t& v, int bytes)
{
    if (s.size() < static_cast<std::size_t>(bytes)) return false;
    v = 0;
    for (int i = 0; i < bytes; ++i) v |= static_cast<std::uint64_t>(static_cast<unsigned char>(s[i])) << (8 * i);
    s.remove_prefix(static_cast<std::size_t>(bytes));
    return true;
}

inline std::string encode_spec(const GptSpec& g)
{
    std::string o;
    const std::pair<const char*, std::uint64_t> u[] = {
        {"d_model", g.d_model},       {"num_heads", g.num_heads},   {"d_ff", g.d_ff},
        {"num_layers", g.num_layers}, {"patch_size", 0},            {"vocab_size", g.vocab_size},
        {"seq_len", g.seq_len},       {"pos_encoding", g.pos_encoding}, {"activation", g.activation},
        {"norm_type", g.norm_type}};
    put_u32(o, 2 + static_cast<std::uint32_t>(std::size(u)));
    auto field = [&](const char* key, std::uint8_t type) {
        put_u32(o, static_cast<std::uint32_t>(std::strlen(key)));
        o.append(key);
        o.push_back(static_cast<char>(type));
    };
    field("type", 0);
    put_u32(o, 8);
    put_u64(o, g.type);
    field("layer_dims", 2);   // empty for a GPT
    put_u32(o, 0);
    for (const auto& [k, v] : u)
    {
        field(k, 0);
        put_u32(o, 8);
        put_u64(o, v);
    }
    return o;
}

// Reads the u64 fields of a spec record (unknown types are skipped by length,
// as KeyValueRecord::parse does); type must be present and non-zero.
inline Result<GptSpec> decode_spec(std::string_view s)
{
    std::uint64_t count = 0, type = 0;
    if (!take(s, count, 4)) return fail("model file: spec record has no field count");
    GptSpec g;
    for (std::uint64_t i = 0; i < count; ++i)
    {
        std::uint64_t klen = 0, vlen = 0;
        if (!take(s, klen, 4) || s.size() < klen + 1) return fail("model file: truncated spec key");
        const std::string key(s.substr(0, klen));
        s.remove_prefix(klen);
        const auto t = static_cast<unsigned char>(s[0]);
        s.remove_prefix(1);
        if (!take(s, vlen, 4) || s.size() < vlen) return fail("model file: truncated spec value");
        std::string_view val = s.substr(0, vlen);
        s.remove_prefix(vlen);
        std::uint64_t v = 0;
        if (t != 0 || !take(val, v, 8)) continue;
        if (key == "type") type = v;
        else if (key == "d_model") g.d_model = v;
        else if (key == "num_heads") g.num_heads = v;
        else if (key == "d_ff") g.d_ff = v;
        else if (key == "num_layers") g.num_layers = v;
        else if (key == "vocab_size") g.vocab_size = v;
        else if (key == "seq_len") g.seq_len = v;
        else if (key == "pos_encoding") g.pos_encoding = v;
        else if (key == "activation") g.activation = v;
        else if (key == "norm_type") g.norm_type = v;
    }
    if (type == 0) return fail("model file: spec has no valid type field");
    g.type = type;
    return g;
}

inline Result<void> save(const std::string& path, const GptSpec& spec, const std::vector<Matrix>& params,
                         std::string_view tokenizer)
{
    std::string o;
    put_u32(o, kMagic);
    put_u32(o, kVersion);
    o.push_back(static_cast<char>(kPrecisionF32));
    const std::string rec = encode_spec(spec);
    put_u64(o, rec.size());
    o.append(rec);
    std::ofstream f(path, std::ios::binary);
    if (!f) return fail("model file: cannot open for writing: " + path);
    f.write(o.data(), static_cast<std::streamsize>(o.size()));
    for (const Matrix& m : params)
    {
        std::string h;
        put_u64(h, m.rows());
        put_u64(h, m.cols());
        f.write(h.data(), static_cast<std::streamsize>(h.size()));
        f.write(reinterpret_cast<const char*>(m.data()), static_cast<std::streamsize>(m.size() * sizeof(float)));
    }
    std::string t;
    put_u64(t, tokenizer.size());
    t.append(tokenizer);
    f.write(t.data(), static_cast<std::streamsize>(t.size()));
    if (!f) return fail("model file: write error: " + path);
    return {};
}

// Reads a file into matrices of the given shapes (a shape mismatch is an
// error, as in detail::read_matrix); returns the spec and the tokenizer bytes.
inline Result<GptSpec> load(const std::string& path, std::vector<Matrix>& params, std::string& tokenizer)
{
    std::ifstream f(path, std::ios::binary);
    if (!f) return fail("model file: cannot open for reading: " + path);
    const std::string all((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    std::string_view s(all);
    std::uint64_t magic = 0, version = 0, prec = 0, speclen = 0;
    if (!take(s, magic, 4) || magic != kMagic) return fail("Invalid model file: bad magic number");
    if (!take(s, version, 4)) return fail("model file: truncated header");
    if (version < kVersion) return fail("model file: old format v" + std::to_string(version) + " is not supported");
    if (version > kVersion) return fail("model file: format v" + std::to_string(version) + " is newer than v4");
    if (!take(s, prec, 1)) return fail("model file: missing precision tag");
    if (prec != kPrecisionF32) return fail("Precision mismatch: file uses f64, this build uses f32");
    if (!take(s, speclen, 8) || s.size() < speclen) return fail("model file: truncated spec header");
    NN_TRY(spec, decode_spec(s.substr(0, speclen)));
    s.remove_prefix(speclen);
    for (Matrix& m : params)
    {
        std::uint64_t r = 0, c = 0;
        if (!take(s, r, 8) || !take(s, c, 8)) return fail("model file: truncated matrix header");
        if (r != m.rows() || c != m.cols())
            return fail("Matrix shape mismatch: expected (" + std::to_string(m.rows()) + ", " +
                        std::to_string(m.cols()) + "), got (" + std::to_string(r) + ", " + std::to_string(c) + ")");
        const std::size_t bytes = m.size() * sizeof(float);
        if (s.size() < bytes) return fail("model file: unexpected end of matrix data");
        std::memcpy(m.data(), s.data(), bytes);
        s.remove_prefix(bytes);
    }
    std::uint64_t tlen = 0;
    if (!take(s, tlen, 8) || s.size() < tlen) return fail("model file: truncated tokenizer data");
    tokenizer.assign(s.substr(0, tlen));
    return spec;
}

} // namespace nn::model_file
