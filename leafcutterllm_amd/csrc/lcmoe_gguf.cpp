// GGUF ingest of MoE layers: a bounds-checked, memory-mapped GGUF v3 reader
// and the mapping of one layer's router, stacked expert and shared-expert
// tensors onto lcmoe_desc / lcmoe_weights.  Host only; no GPU calls.
//
// The file format follows the reference reader GGUFile::open
// (rust/src/model/gguf.rs:76-119): header {magic u32, version u32,
// tensor_count u64, metadata_count u64} (gguf.rs:169-176), metadata KV
// {string key, u32 type, value} (gguf.rs:178-210), tensor infos {string name,
// u32 n_dims, u64 dims[n_dims], u32 type, u64 offset} (gguf.rs:212-227), the
// data section at the header end rounded up to general.alignment (U32 or U64,
// default 32; gguf.rs:100-110), and a tensor's bytes at data_offset + offset,
// tensor_size(type, prod(dims)) long (gguf.rs:121-127, 307-313).  Where the
// reference would index past the mapping (and panic) this reader returns
// LCMOE_ERR_CORRUPT.
//
// The reference maps dense layers only (rust/src/model/arch.rs:83-96); the
// MoE tensor names and metadata keys read here are the GGUF conventions for
// MoE models:
//   blk.N.ffn_gate_inp.weight                router, dims [d, E] (F32/F16/BF16)
//   blk.N.ffn_{gate,up,down}_exps.weight     stacked experts, dims [d, F, E]
//                                            (down: [F, d, E]); or, in older
//                                            files, per-expert 2D tensors
//                                            blk.N.ffn_{gate,up,down}.<e>.weight
//   blk.N.ffn_{gate,up,down}_shexp.weight    shared expert(s): 2D -> one shared
//                                            expert, 3D -> dims[2] of them
//   blk.N.exp_probs_b.bias                   selection bias [E] (sigmoid gating)
//   blk.N.ffn_gate_inp.bias                  router logit bias [E] (softmax gating)
//   <arch>.expert_used_count (required), .expert_count, .embedding_length,
//   .expert_feed_forward_length, .expert_gating_func, .expert_weights_norm,
//   .expert_weights_scale, .expert_group_count, .expert_group_used_count
// where <arch> is general.architecture.

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <map>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "lcmoe_internal.h"

using namespace lcmoe;

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" read little-endian
constexpr uint32_t kVersion = 3;
constexpr int kMaxDims = 4;
constexpr int kMaxNesting = 8;  // arrays of arrays

enum : uint32_t {
    KV_U8 = 0, KV_I8, KV_U16, KV_I16, KV_U32, KV_I32, KV_F32, KV_BOOL, KV_STRING, KV_ARRAY,
    KV_U64, KV_I64, KV_F64
};

// ggml type codes read here beyond the lcmoe.h ones
constexpr int32_t kTypeF16 = 1, kTypeBF16 = 30;

// (elements, bytes) per block of the GGUF types whose codes agree between
// ggml and QuantType (rust/src/model/quant.rs:45-73, 170-239); {0, 0} unknown
struct BlockGeom { int64_t n, bytes; };
BlockGeom type_geom(uint32_t t) {
    switch (t) {
    case 0: return {1, 4};       // F32
    case 1: return {1, 2};       // F16
    case 2: return {32, 18};     // Q4_0
    case 3: return {32, 20};     // Q4_1
    case 6: return {32, 22};     // Q5_0
    case 7: return {32, 24};     // Q5_1
    case 8: return {32, 34};     // Q8_0
    case 9: return {32, 36};     // Q8_1
    case 10: return {256, 84};   // Q2_K
    case 11: return {256, 110};  // Q3_K
    case 12: return {256, 144};  // Q4_K
    case 13: return {256, 176};  // Q5_K
    case 14: return {256, 210};  // Q6_K
    case 15: return {256, 292};  // Q8_K
    case 16: return {256, 66};   // IQ2_XXS
    case 17: return {256, 74};   // IQ2_XS
    case 18: return {256, 98};   // IQ3_XXS
    case 30: return {1, 2};      // BF16
    default: return {0, 0};
    }
}

struct Value {
    uint32_t type = 0;
    uint64_t u = 0;     // unsigned integers and bool
    int64_t i = 0;      // signed integers
    double f = 0;       // F32 / F64
    std::string s;      // STRING
    uint32_t arr_type = 0;
    uint64_t arr_len = 0;
    std::unique_ptr<Value> first;  // element 0 of a one-element array
};

struct TensorInfo {
    std::string name;
    int n_dims = 0;
    uint64_t dims[kMaxDims] = {1, 1, 1, 1};
    uint32_t type = 0;
    uint64_t offset = 0;
    uint64_t count = 1;
    uint64_t bytes = 0;  // 0 when the type's geometry is unknown
};

// bounds-checked little-endian cursor over the mapping
struct Cursor {
    const uint8_t *p;
    size_t n, pos = 0;
    bool ok = true;
    bool need(size_t k) {
        if (!ok || k > n - pos) ok = false;
        return ok;
    }
    template <class T> T get() {
        T v{};
        if (need(sizeof(T))) {
            std::memcpy(&v, p + pos, sizeof(T));
            pos += sizeof(T);
        }
        return v;
    }
    bool skip(uint64_t k) {
        if (!ok || k > n - pos) return ok = false;
        pos += (size_t)k;
        return true;
    }
    std::string str() {
        const uint64_t len = get<uint64_t>();
        if (!ok || len > n - pos) {
            ok = false;
            return {};
        }
        std::string s(reinterpret_cast<const char *>(p + pos), (size_t)len);
        pos += (size_t)len;
        return s;
    }
};

size_t scalar_bytes(uint32_t t) {
    switch (t) {
    case KV_U8: case KV_I8: case KV_BOOL: return 1;
    case KV_U16: case KV_I16: return 2;
    case KV_U32: case KV_I32: case KV_F32: return 4;
    case KV_U64: case KV_I64: case KV_F64: return 8;
    default: return 0;
    }
}

// read_value, gguf.rs:185-210; unknown types fail like the reference's
// InvalidTensorType.  Arrays keep their type, length and (when one element
// long) that element; the rest is skipped.
lcmoe_status read_value(Cursor &c, uint32_t t, Value &v, int depth) {
    v.type = t;
    switch (t) {
    case KV_U8: v.u = c.get<uint8_t>(); break;
    case KV_I8: v.i = c.get<int8_t>(); break;
    case KV_U16: v.u = c.get<uint16_t>(); break;
    case KV_I16: v.i = c.get<int16_t>(); break;
    case KV_U32: v.u = c.get<uint32_t>(); break;
    case KV_I32: v.i = c.get<int32_t>(); break;
    case KV_F32: v.f = c.get<float>(); break;
    case KV_BOOL: v.u = c.get<uint8_t>() != 0; break;
    case KV_STRING: v.s = c.str(); break;
    case KV_U64: v.u = c.get<uint64_t>(); break;
    case KV_I64: v.i = c.get<int64_t>(); break;
    case KV_F64: v.f = c.get<double>(); break;
    case KV_ARRAY: {
        if (depth >= kMaxNesting) return fail(LCMOE_ERR_CORRUPT, "metadata arrays nested deeper than %d", kMaxNesting);
        v.arr_type = c.get<uint32_t>();
        v.arr_len = c.get<uint64_t>();
        if (!c.ok) break;
        const size_t sb = scalar_bytes(v.arr_type);
        if (v.arr_len == 1) {
            v.first = std::make_unique<Value>();
            lcmoe_status st = read_value(c, v.arr_type, *v.first, depth + 1);
            if (st != LCMOE_OK) return st;
        } else if (sb > 0) {
            if (v.arr_len > (c.n - c.pos) / sb) c.ok = false;
            else c.skip(v.arr_len * sb);
        } else {
            // strings and nested arrays: every element takes at least 8 bytes,
            // so the loop ends within the mapping's length
            for (uint64_t k = 0; k < v.arr_len && c.ok; k++) {
                Value tmp;
                lcmoe_status st = read_value(c, v.arr_type, tmp, depth + 1);
                if (st != LCMOE_OK) return st;
            }
        }
        break;
    }
    default: return fail(LCMOE_ERR_UNSUPPORTED, "metadata value type %u unknown", t);
    }
    if (!c.ok) return fail(LCMOE_ERR_CORRUPT, "GGUF file truncated inside a metadata value");
    return LCMOE_OK;
}

// get_metadata_int, gguf.rs:133-157: every integer and float type (floats
// truncated toward zero, saturating, NaN -> 0, as Rust's `as i64`) and a
// one-element array of U32/I32/U64/I64; not bool or string
bool value_int(const Value &v, int64_t *out) {
    switch (v.type) {
    case KV_U8: case KV_U16: case KV_U32: case KV_U64: *out = (int64_t)v.u; return true;
    case KV_I8: case KV_I16: case KV_I32: case KV_I64: *out = v.i; return true;
    case KV_F32: case KV_F64: {
        const double f = v.f;
        if (std::isnan(f)) *out = 0;
        else if (f >= 9223372036854775807.0) *out = std::numeric_limits<int64_t>::max();
        else if (f <= -9223372036854775808.0) *out = std::numeric_limits<int64_t>::min();
        else *out = (int64_t)f;
        return true;
    }
    case KV_ARRAY:
        if (v.arr_len == 1 && v.first &&
            (v.arr_type == KV_U32 || v.arr_type == KV_I32 || v.arr_type == KV_U64 ||
             v.arr_type == KV_I64))
            return value_int(*v.first, out);
        return false;
    default: return false;
    }
}

}  // namespace

// host copies a layer's weights need beyond the mapping
struct LayerBufs {
    std::vector<float> router, bias;
    std::vector<uint8_t> gate, up, down;  // gathered per-expert tensors
};

struct lcmoe_gguf {
    int fd = -1;
    const uint8_t *base = nullptr;
    size_t size = 0;
    std::unordered_map<std::string, Value> meta;
    std::vector<TensorInfo> tensors;
    std::unordered_map<std::string, size_t> index;  // first tensor of each name
    uint64_t alignment = 32, data_offset = 0;
    std::map<int32_t, std::unique_ptr<LayerBufs>> layers;

    ~lcmoe_gguf() {
        if (base) munmap(const_cast<uint8_t *>(base), size);
        if (fd >= 0) close(fd);
    }
    const Value *find_meta(const std::string &k) const {
        auto it = meta.find(k);
        return it == meta.end() ? nullptr : &it->second;
    }
    const TensorInfo *find_tensor(const std::string &name) const {
        auto it = index.find(name);
        return it == index.end() ? nullptr : &tensors[it->second];
    }
    const uint8_t *data(const TensorInfo &t) const { return base + data_offset + t.offset; }
    std::string arch() const {
        const Value *v = find_meta("general.architecture");
        return v && v->type == KV_STRING ? v->s : std::string();
    }
};

namespace {

lcmoe_status parse(lcmoe_gguf &g) {
    Cursor c{g.base, g.size};
    const uint32_t magic = c.get<uint32_t>(), version = c.get<uint32_t>();
    const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
    if (!c.ok) return fail(LCMOE_ERR_CORRUPT, "GGUF file truncated inside the header (%zu bytes)", g.size);
    if (magic != kMagic) return fail(LCMOE_ERR_CORRUPT, "invalid GGUF magic 0x%08x", magic);
    if (version != kVersion)
        return fail(LCMOE_ERR_UNSUPPORTED, "GGUF version %u unsupported (version 3 only)", version);
    // a KV takes at least 13 bytes and a tensor info at least 24: larger
    // counts cannot fit in the file
    if (n_kv > g.size / 13 || n_tensors > g.size / 24)
        return fail(LCMOE_ERR_CORRUPT, "GGUF counts (%llu tensors, %llu metadata) exceed the file",
                    (unsigned long long)n_tensors, (unsigned long long)n_kv);
    for (uint64_t k = 0; k < n_kv; k++) {
        std::string key = c.str();
        const uint32_t t = c.get<uint32_t>();
        if (!c.ok) return fail(LCMOE_ERR_CORRUPT, "GGUF file truncated in metadata entry %llu", (unsigned long long)k);
        Value v;
        lcmoe_status st = read_value(c, t, v, 0);
        if (st != LCMOE_OK) return st;
        g.meta[key] = std::move(v);  // a repeated key keeps the last value
    }
    g.tensors.resize((size_t)n_tensors);
    for (uint64_t k = 0; k < n_tensors; k++) {
        TensorInfo &ti = g.tensors[(size_t)k];
        ti.name = c.str();
        const uint32_t nd = c.get<uint32_t>();
        if (!c.ok) return fail(LCMOE_ERR_CORRUPT, "GGUF file truncated in tensor info %llu", (unsigned long long)k);
        if (nd < 1 || nd > (uint32_t)kMaxDims)
            return fail(LCMOE_ERR_CORRUPT, "tensor %s has %u dims (1..4 allowed)", ti.name.c_str(), nd);
        ti.n_dims = (int)nd;
        for (int i = 0; i < ti.n_dims; i++) ti.dims[i] = c.get<uint64_t>();
        ti.type = c.get<uint32_t>();
        ti.offset = c.get<uint64_t>();
        if (!c.ok) return fail(LCMOE_ERR_CORRUPT, "GGUF file truncated in tensor info %llu", (unsigned long long)k);
        for (int i = 0; i < ti.n_dims; i++) {
            if (ti.count && ti.dims[i] > ((uint64_t)1 << 62) / ti.count)
                return fail(LCMOE_ERR_CORRUPT, "tensor %s: element count overflows", ti.name.c_str());
            ti.count *= ti.dims[i];
        }
        const BlockGeom bg = type_geom(ti.type);
        if (bg.n > 0) ti.bytes = (ti.count + bg.n - 1) / bg.n * (uint64_t)bg.bytes;  // quant.rs:256-261
        g.index.emplace(ti.name, (size_t)k);
    }
    if (const Value *a = g.find_meta("general.alignment")) {
        if (a->type == KV_U32 || a->type == KV_U64) g.alignment = a->u;
    }
    if (g.alignment == 0) return fail(LCMOE_ERR_CORRUPT, "general.alignment is 0");
    const uint64_t pos = c.pos, pad = (g.alignment - pos % g.alignment) % g.alignment;
    g.data_offset = pos + pad;
    // every tensor of known size lies inside the mapping
    for (const TensorInfo &ti : g.tensors) {
        if (ti.bytes == 0) continue;
        const uint64_t room = g.size >= g.data_offset ? g.size - g.data_offset : 0;
        if (ti.offset > room || ti.bytes > room - ti.offset)
            return fail(LCMOE_ERR_CORRUPT, "tensor %s [%llu bytes at data+%llu] ends past the file (%zu bytes)",
                        ti.name.c_str(), (unsigned long long)ti.bytes, (unsigned long long)ti.offset, g.size);
    }
    return LCMOE_OK;
}

bool meta_int(const lcmoe_gguf &g, const std::string &key, int64_t *out) {
    const Value *v = g.find_meta(key);
    return v && value_int(*v, out);
}

// bool, or any integer (nonzero = true)
bool meta_flag(const lcmoe_gguf &g, const std::string &key, bool *out) {
    const Value *v = g.find_meta(key);
    if (!v) return false;
    if (v->type == KV_BOOL) {
        *out = v->u != 0;
        return true;
    }
    int64_t i;
    if (!value_int(*v, &i)) return false;
    *out = i != 0;
    return true;
}

bool meta_float(const lcmoe_gguf &g, const std::string &key, double *out) {
    const Value *v = g.find_meta(key);
    if (!v) return false;
    if (v->type == KV_F32 || v->type == KV_F64) {
        *out = v->f;
        return true;
    }
    int64_t i;
    if (!value_int(*v, &i)) return false;
    *out = (double)i;
    return true;
}

bool dims_are(const TensorInfo &t, int n, uint64_t a, uint64_t b, uint64_t c = 1) {
    return t.n_dims == n && t.dims[0] == a && t.dims[1] == b && (n < 3 || t.dims[2] == c);
}

// f32 value i of a F32 / F16 / BF16 tensor
float float_at(const lcmoe_gguf &g, const TensorInfo &t, uint64_t i) {
    const uint8_t *p = g.data(t);
    if (t.type == LCMOE_TYPE_F32) {
        float f;
        std::memcpy(&f, p + 4 * i, 4);
        return f;
    }
    uint16_t h;
    std::memcpy(&h, p + 2 * i, 2);
    if (t.type == kTypeF16) return half_to_float(h);
    const uint32_t u = (uint32_t)h << 16;  // BF16
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// out-of-range metadata becomes -1 or INT32_MAX, which validation rejects
int32_t clamp32(int64_t v) { return (int32_t)std::min<int64_t>(std::max<int64_t>(v, -1), INT32_MAX); }

bool is_float_type(uint32_t t) { return t == LCMOE_TYPE_F32 || t == (uint32_t)kTypeF16 || t == (uint32_t)kTypeBF16; }

// The three expert tensors of one kind (routed or shared): stacked 3D, or
// (routed only) one 2D tensor per expert gathered into `own`.  rows x cols
// per expert: gate/up [F, d], down [d, F] (dims list cols first).
struct ExpertSet {
    const uint8_t *ptr[3] = {nullptr, nullptr, nullptr};
    int32_t type[3] = {0, 0, 0};
    uint64_t F = 0, n = 0;  // hidden size, experts
};

lcmoe_status stacked_set(const lcmoe_gguf &g, const std::string &pre, const char *suffix, uint64_t d,
                         ExpertSet *out, bool *found) {
    static const char *kinds[3] = {"gate", "up", "down"};
    const TensorInfo *t[3];
    for (int k = 0; k < 3; k++) t[k] = g.find_tensor(pre + "ffn_" + kinds[k] + suffix + ".weight");
    *found = t[0] || t[1] || t[2];
    if (!*found) return LCMOE_OK;
    for (int k = 0; k < 3; k++)
        if (!t[k]) return fail(LCMOE_ERR_NOT_FOUND, "%sffn_%s%s.weight missing (its gate/up/down siblings exist)",
                               pre.c_str(), kinds[k], suffix);
    const int nd = t[0]->n_dims;
    if (nd != 2 && nd != 3)
        return fail(LCMOE_ERR_CORRUPT, "%sffn_gate%s.weight has %d dims (2 or 3 expected)", pre.c_str(), suffix, nd);
    const uint64_t F = t[0]->dims[1], n = nd == 3 ? t[0]->dims[2] : 1;
    if (!dims_are(*t[0], nd, d, F, n) || !dims_are(*t[1], nd, d, F, n) || !dims_are(*t[2], nd, F, d, n))
        return fail(LCMOE_ERR_CORRUPT,
                    "%sffn_*%s.weight dims disagree: gate/up must be [%llu, F, n], down [F, %llu, n]",
                    pre.c_str(), suffix, (unsigned long long)d, (unsigned long long)d);
    for (int k = 0; k < 3; k++) {
        if (t[k]->bytes == 0)
            return fail(LCMOE_ERR_UNSUPPORTED, "%sffn_%s%s.weight has GGUF type %u, not supported", pre.c_str(),
                        kinds[k], suffix, t[k]->type);
        out->ptr[k] = g.data(*t[k]);
        out->type[k] = (int32_t)t[k]->type;
    }
    out->F = F;
    out->n = n;
    return LCMOE_OK;
}

// per-expert 2D tensors blk.N.ffn_{gate,up,down}.<e>.weight, e < E, copied
// into one stacked buffer per kind
lcmoe_status gathered_set(const lcmoe_gguf &g, const std::string &pre, uint64_t d, uint64_t E, LayerBufs &own,
                          ExpertSet *out, bool *found) {
    static const char *kinds[3] = {"gate", "up", "down"};
    *found = g.find_tensor(pre + "ffn_gate.0.weight") != nullptr;
    if (!*found) return LCMOE_OK;
    std::vector<uint8_t> *dst[3] = {&own.gate, &own.up, &own.down};
    uint64_t F = g.find_tensor(pre + "ffn_gate.0.weight")->dims[1];
    for (int k = 0; k < 3; k++) {
        uint64_t bytes = 0;
        for (uint64_t e = 0; e < E; e++) {
            const std::string name = pre + "ffn_" + kinds[k] + "." + std::to_string(e) + ".weight";
            const TensorInfo *t = g.find_tensor(name);
            if (!t) return fail(LCMOE_ERR_NOT_FOUND, "%s missing", name.c_str());
            const bool ok = k < 2 ? dims_are(*t, 2, d, F) : dims_are(*t, 2, F, d);
            if (!ok) return fail(LCMOE_ERR_CORRUPT, "%s dims disagree with expert 0", name.c_str());
            if (t->bytes == 0)
                return fail(LCMOE_ERR_UNSUPPORTED, "%s has GGUF type %u, not supported", name.c_str(), t->type);
            if (e == 0) {
                out->type[k] = (int32_t)t->type;
                bytes = t->bytes;
                dst[k]->resize(bytes * E);
            } else if ((int32_t)t->type != out->type[k]) {
                return fail(LCMOE_ERR_UNSUPPORTED, "%s has type %u, expert 0 has %d", name.c_str(), t->type,
                            out->type[k]);
            }
            std::memcpy(dst[k]->data() + e * bytes, g.data(*t), bytes);
        }
        out->ptr[k] = dst[k]->data();
    }
    out->F = F;
    out->n = E;
    return LCMOE_OK;
}

// Default of expert_weights_norm where a file omits it: the renormalisation
// each architecture's MoE applies (Mixtral, exported as "llama", and
// Qwen3-MoE renormalise; Qwen2-MoE, OLMoE and DeepSeek-V2 do not).
bool default_norm(const std::string &arch, bool *out) {
    if (arch == "llama" || arch == "mixtral" || arch == "qwen3moe") return *out = true, true;
    if (arch == "qwen2moe" || arch == "olmoe" || arch == "deepseek2") return *out = false, true;
    return false;
}

lcmoe_status moe_layer(lcmoe_gguf &g, int32_t layer, int32_t max_tokens, lcmoe_desc *desc, lcmoe_weights *w) {
    const std::string pre = "blk." + std::to_string(layer) + ".";
    const std::string arch = g.arch();
    const std::string ak = arch + ".";

    const TensorInfo *rt = g.find_tensor(pre + "ffn_gate_inp.weight");
    if (!rt) return fail(LCMOE_ERR_NOT_FOUND, "%sffn_gate_inp.weight missing: layer %d is not an MoE layer",
                         pre.c_str(), layer);
    if (rt->n_dims != 2) return fail(LCMOE_ERR_CORRUPT, "%sffn_gate_inp.weight has %d dims (2 expected)", pre.c_str(), rt->n_dims);
    if (!is_float_type(rt->type))
        return fail(LCMOE_ERR_UNSUPPORTED, "%sffn_gate_inp.weight has GGUF type %u (F32, F16 or BF16 supported)",
                    pre.c_str(), rt->type);
    const uint64_t d = rt->dims[0], E = rt->dims[1];
    if (d == 0 || d > 16384 || E == 0 || E > 256)
        return fail(LCMOE_ERR_UNSUPPORTED, "router dims [%llu, %llu] outside d <= 16384, E <= 256",
                    (unsigned long long)d, (unsigned long long)E);
    if (g.find_tensor(pre + "ffn_gate_inp_shexp.weight"))
        return fail(LCMOE_ERR_UNSUPPORTED, "%sffn_gate_inp_shexp.weight: gated shared experts are not supported",
                    pre.c_str());

    auto bufs = std::make_unique<LayerBufs>();
    ExpertSet routed, shared;
    bool found = false;
    lcmoe_status st = stacked_set(g, pre, "_exps", d, &routed, &found);
    if (st != LCMOE_OK) return st;
    if (found) {
        if (routed.n != E)
            return fail(LCMOE_ERR_CORRUPT, "%sffn_*_exps.weight hold %llu experts, the router %llu", pre.c_str(),
                        (unsigned long long)routed.n, (unsigned long long)E);
    } else {
        st = gathered_set(g, pre, d, E, *bufs, &routed, &found);
        if (st != LCMOE_OK) return st;
        if (!found) return fail(LCMOE_ERR_NOT_FOUND, "%sffn_gate_exps.weight missing (no per-expert tensors either)",
                                pre.c_str());
    }
    bool has_shared = false;
    st = stacked_set(g, pre, "_shexp", d, &shared, &has_shared);
    if (st != LCMOE_OK) return st;

    // metadata: K required; the rest checked against the tensors when present
    int64_t K = 0, v = 0;
    if (!meta_int(g, ak + "expert_used_count", &K))
        return fail(LCMOE_ERR_NOT_FOUND, "metadata %sexpert_used_count missing", ak.c_str());
    if (meta_int(g, ak + "expert_count", &v) && (uint64_t)v != E)
        return fail(LCMOE_ERR_CORRUPT, "%sexpert_count = %lld, the router has %llu experts", ak.c_str(), (long long)v,
                    (unsigned long long)E);
    if (meta_int(g, ak + "embedding_length", &v) && (uint64_t)v != d)
        return fail(LCMOE_ERR_CORRUPT, "%sembedding_length = %lld, the router has d = %llu", ak.c_str(), (long long)v,
                    (unsigned long long)d);
    if (meta_int(g, ak + "expert_feed_forward_length", &v) && (uint64_t)v != routed.F)
        return fail(LCMOE_ERR_CORRUPT, "%sexpert_feed_forward_length = %lld, the experts have %llu", ak.c_str(),
                    (long long)v, (unsigned long long)routed.F);

    // gating: 0 (unset) and 1 softmax, 2 sigmoid, 3 softmax over the selected
    int64_t gating = 1;
    meta_int(g, ak + "expert_gating_func", &gating);
    bool norm = false;
    const bool norm_set = meta_flag(g, ak + "expert_weights_norm", &norm);
    double scale = 1.0;
    meta_float(g, ak + "expert_weights_scale", &scale);
    int64_t n_group = 1, topk_group = 0;
    meta_int(g, ak + "expert_group_count", &n_group);
    const bool tg_set = meta_int(g, ak + "expert_group_used_count", &topk_group);
    if (!tg_set) topk_group = n_group;

    const TensorInfo *sel_b = g.find_tensor(pre + "exp_probs_b.bias");
    const TensorInfo *logit_b = g.find_tensor(pre + "ffn_gate_inp.bias");
    const TensorInfo *bt = sel_b ? sel_b : logit_b;
    if (sel_b && logit_b)
        return fail(LCMOE_ERR_UNSUPPORTED, "%s has both exp_probs_b.bias and ffn_gate_inp.bias", pre.c_str());
    if (bt && (bt->n_dims != 1 || bt->dims[0] != E || !is_float_type(bt->type)))
        return fail(LCMOE_ERR_CORRUPT, "%s must be a float [%llu] tensor", bt->name.c_str(), (unsigned long long)E);

    int32_t kind;
    switch (gating) {
    case 0:
    case 1:
        if (!norm_set && !default_norm(arch, &norm))
            return fail(LCMOE_ERR_NOT_FOUND, "metadata %sexpert_weights_norm missing and no default for '%s'",
                        ak.c_str(), arch.c_str());
        kind = norm ? LCMOE_ROUTE_SOFTMAX_RENORM : LCMOE_ROUTE_SOFTMAX;
        break;
    case 3: kind = LCMOE_ROUTE_SOFTMAX_RENORM; break;
    case 2:
        if (norm_set && !norm)
            return fail(LCMOE_ERR_UNSUPPORTED, "sigmoid gating without weight normalisation is not supported");
        kind = LCMOE_ROUTE_SIGMOID_GROUP;
        break;
    default:
        return fail(LCMOE_ERR_UNSUPPORTED, "%sexpert_gating_func = %lld unknown", ak.c_str(), (long long)gating);
    }
    if (kind == LCMOE_ROUTE_SIGMOID_GROUP) {
        // the selection-only bias belongs to sigmoid gating; a logit bias
        // would enter before the sigmoid, which this router does not do
        if (logit_b)
            return fail(LCMOE_ERR_UNSUPPORTED, "%sffn_gate_inp.bias with sigmoid gating is not supported", pre.c_str());
    } else {
        // softmax gating adds the bias to the logits, selection and weights
        // alike; a selection-only bias is not that
        if (sel_b)
            return fail(LCMOE_ERR_UNSUPPORTED, "%sexp_probs_b.bias with softmax gating is not supported", pre.c_str());
        if (n_group > 1)
            return fail(LCMOE_ERR_UNSUPPORTED, "%sexpert_group_count = %lld with softmax gating is not supported",
                        ak.c_str(), (long long)n_group);
    }
    if (!std::isfinite(scale)) return fail(LCMOE_ERR_CORRUPT, "%sexpert_weights_scale is not finite", ak.c_str());

    lcmoe_desc dd{};
    dd.d_model = (int32_t)d;
    dd.d_ff = clamp32((int64_t)std::min<uint64_t>(routed.F, INT32_MAX));
    dd.n_expert = (int32_t)E;
    dd.n_expert_used = clamp32(K);
    dd.route_kind = kind;
    dd.n_group = kind == LCMOE_ROUTE_SIGMOID_GROUP ? clamp32(n_group) : 1;
    dd.topk_group = kind == LCMOE_ROUTE_SIGMOID_GROUP ? clamp32(topk_group) : 1;
    dd.routed_scale = (float)scale;
    dd.has_bias = bt != nullptr;
    dd.type_gate = routed.type[0];
    dd.type_up = routed.type[1];
    dd.type_down = routed.type[2];
    if (has_shared) {
        dd.n_shared = shared.n > 8 ? 9 : (int32_t)shared.n;
        dd.d_ff_shared = clamp32((int64_t)std::min<uint64_t>(shared.F, INT32_MAX));
        dd.type_gate_sh = shared.type[0];
        dd.type_up_sh = shared.type[1];
        dd.type_down_sh = shared.type[2];
    }
    dd.max_tokens = max_tokens;
    st = validate_desc(&dd);
    if (st != LCMOE_OK) return st;

    // router: the file holds E rows of d (dims [d, E], d fastest); the ABI
    // takes [d, E], the transpose load_layer produces (loader.rs:155-160)
    bufs->router.resize(d * E);
    for (uint64_t e = 0; e < E; e++)
        for (uint64_t k = 0; k < d; k++) bufs->router[k * E + e] = float_at(g, *rt, e * d + k);
    if (bt) {
        bufs->bias.resize(E);
        for (uint64_t e = 0; e < E; e++) bufs->bias[e] = float_at(g, *bt, e);
    }

    lcmoe_weights ww{};
    ww.router = bufs->router.data();
    ww.bias = bt ? bufs->bias.data() : nullptr;
    ww.gate = routed.ptr[0];
    ww.up = routed.ptr[1];
    ww.down = routed.ptr[2];
    if (has_shared) {
        ww.gate_sh = shared.ptr[0];
        ww.up_sh = shared.ptr[1];
        ww.down_sh = shared.ptr[2];
    }
    g.layers[layer] = std::move(bufs);  // replaces (and frees) an earlier call's copies
    *desc = dd;
    *w = ww;
    return LCMOE_OK;
}

}  // namespace

extern "C" {

lcmoe_status lcmoe_gguf_open(const char *path, lcmoe_gguf **out) {
    clear_error();
    if (!path || !out) return fail(LCMOE_ERR_INVALID_ARG, "path or out is NULL");
    *out = nullptr;
    auto g = std::make_unique<lcmoe_gguf>();
    g->fd = open(path, O_RDONLY | O_CLOEXEC);
    if (g->fd < 0) return fail(LCMOE_ERR_IO, "cannot open %s: %s", path, strerror(errno));
    struct stat sb;
    if (fstat(g->fd, &sb) != 0) return fail(LCMOE_ERR_IO, "cannot stat %s: %s", path, strerror(errno));
    if (!S_ISREG(sb.st_mode)) return fail(LCMOE_ERR_IO, "%s is not a regular file", path);
    g->size = (size_t)sb.st_size;
    if (g->size < 24) return fail(LCMOE_ERR_CORRUPT, "%s: %zu bytes, shorter than a GGUF header", path, g->size);
    void *m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) return fail(LCMOE_ERR_IO, "cannot map %s: %s", path, strerror(errno));
    g->base = static_cast<const uint8_t *>(m);
    lcmoe_status st = parse(*g);
    if (st != LCMOE_OK) return st;
    *out = g.release();
    return LCMOE_OK;
}

void lcmoe_gguf_close(lcmoe_gguf *g) { delete g; }

lcmoe_status lcmoe_gguf_meta_int(const lcmoe_gguf *g, const char *key, int64_t *out) {
    clear_error();
    if (!g || !key || !out) return fail(LCMOE_ERR_INVALID_ARG, "g, key or out is NULL");
    const Value *v = g->find_meta(key);
    if (!v) return fail(LCMOE_ERR_NOT_FOUND, "metadata %s missing", key);
    if (!value_int(*v, out)) return fail(LCMOE_ERR_INVALID_ARG, "metadata %s is not an integer (type %u)", key, v->type);
    return LCMOE_OK;
}

const char *lcmoe_gguf_meta_str(const lcmoe_gguf *g, const char *key) {
    if (!g || !key) return nullptr;
    const Value *v = g->find_meta(key);
    return v && v->type == KV_STRING ? v->s.c_str() : nullptr;
}

lcmoe_status lcmoe_gguf_tensor(const lcmoe_gguf *g, const char *name, int32_t *type, int32_t *n_dims,
                               int64_t *dims, const uint8_t **data, uint64_t *bytes) {
    clear_error();
    if (!g || !name) return fail(LCMOE_ERR_INVALID_ARG, "g or name is NULL");
    const TensorInfo *t = g->find_tensor(name);
    if (!t) return fail(LCMOE_ERR_NOT_FOUND, "tensor %s missing", name);
    if (type) *type = (int32_t)t->type;
    if (n_dims) *n_dims = t->n_dims;
    if (dims)
        for (int i = 0; i < kMaxDims; i++) dims[i] = i < t->n_dims ? (int64_t)t->dims[i] : 1;
    if (data) *data = t->bytes ? g->data(*t) : nullptr;
    if (bytes) *bytes = t->bytes;
    return LCMOE_OK;
}

int32_t lcmoe_gguf_block_count(const lcmoe_gguf *g) {
    if (!g) return -1;
    int64_t v;
    if (meta_int(*g, g->arch() + ".block_count", &v) && v >= 0 && v <= INT32_MAX) return (int32_t)v;
    int64_t top = -1;
    for (const TensorInfo &t : g->tensors) {
        if (t.name.compare(0, 4, "blk.") != 0) continue;
        char *end = nullptr;
        const long long n = strtoll(t.name.c_str() + 4, &end, 10);
        if (end != t.name.c_str() + 4 && *end == '.' && n >= 0 && n < INT32_MAX) top = std::max<int64_t>(top, n);
    }
    return (int32_t)(top + 1);
}

int32_t lcmoe_gguf_is_moe_layer(const lcmoe_gguf *g, int32_t layer) {
    if (!g || layer < 0) return 0;
    return g->find_tensor("blk." + std::to_string(layer) + ".ffn_gate_inp.weight") != nullptr;
}

lcmoe_status lcmoe_gguf_moe_layer(lcmoe_gguf *g, int32_t layer, int32_t max_tokens, lcmoe_desc *desc,
                                  lcmoe_weights *w) {
    clear_error();
    if (!g || !desc || !w) return fail(LCMOE_ERR_INVALID_ARG, "g, desc or w is NULL");
    if (layer < 0) return fail(LCMOE_ERR_INVALID_ARG, "layer %d is negative", layer);
    return moe_layer(*g, layer, max_tokens, desc, w);
}

}  // extern "C"
