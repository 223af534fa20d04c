// dmoe_gguf.cpp — GGUF reader for the MoE tensors and hyper-parameters
// (C ABI in include/dmoe.h).
//
// Replaces, for the tensors this library consumes, the loader mechanics of
// src/diffuse-model.cpp: gguf_init_from_file (:70-73), the key helpers with
// the "diffuse." / "qwen2." / "llama." prefix search (:5-64), the MoE
// hyper-parameters (:143-158) and the per-layer tensor names (:164-196).
// The container layout is GGUF v2/v3 as tools/quantize_streaming.py:13-88
// parses it: magic "GGUF", u32 version, u64 tensor count, u64 key/value
// count; key/value pairs (u64-length string key, u32 value type, value; types
// 0..12, arrays as u32 element type + u64 count); tensor infos (name, u32
// n_dims, n_dims x i64 ne, u32 ggml type, u64 offset); tensor data from the
// first multiple of general.alignment (default 32) after the infos.
//
// The file is memory-mapped read-only; every field read is bounds-checked, so
// a truncated or malformed file is an error, never a read past the mapping.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/dmoe.h"

struct dmoe_gguf {
    const uint8_t *base = nullptr;       // the mapping
    size_t size = 0;
    uint32_t version = 0;
    uint32_t alignment = 32;
    size_t data_start = 0;
    struct Kv {
        uint32_t type;                   // GGUF value type
        size_t off;                      // offset of the value in the file
    };
    std::unordered_map<std::string, Kv> kv;
    struct Tinfo {
        int32_t type;
        int32_t n_dims;
        int64_t ne[4];
        uint64_t offset;                 // relative to data_start
        size_t nbytes;                   // 0: a type whose block size is unknown here
    };
    std::unordered_map<std::string, Tinfo> tensors;
    std::vector<std::string> tensor_order;
};

namespace {

// ggml block sizes and bytes per block of the types a GGUF file may hold
// (ggml_type ids; only the ones with a fixed block layout).
bool type_block(int32_t t, int64_t *elems, int64_t *bytes)
{
    switch (t) {
    case 0: *elems = 1; *bytes = 4; return true;        // F32
    case 1: *elems = 1; *bytes = 2; return true;        // F16
    case 2: *elems = 32; *bytes = 18; return true;      // Q4_0
    case 3: *elems = 32; *bytes = 20; return true;      // Q4_1
    case 6: *elems = 32; *bytes = 22; return true;      // Q5_0
    case 7: *elems = 32; *bytes = 24; return true;      // Q5_1
    case 8: *elems = 32; *bytes = 34; return true;      // Q8_0
    case 9: *elems = 32; *bytes = 36; return true;      // Q8_1
    case 10: *elems = 256; *bytes = 84; return true;    // Q2_K
    case 11: *elems = 256; *bytes = 110; return true;   // Q3_K
    case 12: *elems = 256; *bytes = 144; return true;   // Q4_K
    case 13: *elems = 256; *bytes = 176; return true;   // Q5_K
    case 14: *elems = 256; *bytes = 210; return true;   // Q6_K
    case 15: *elems = 256; *bytes = 292; return true;   // Q8_K
    case 24: *elems = 1; *bytes = 1; return true;       // I8
    case 25: *elems = 1; *bytes = 2; return true;       // I16
    case 26: *elems = 1; *bytes = 4; return true;       // I32
    case 27: *elems = 1; *bytes = 8; return true;       // I64
    case 28: *elems = 1; *bytes = 8; return true;       // F64
    case 30: *elems = 1; *bytes = 2; return true;       // BF16
    default: return false;
    }
}

int fail(char *err, size_t errlen, int code, const char *fmt, ...)
{
    if (err && errlen) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(err, errlen, fmt, ap);
        va_end(ap);
    }
    return code;
}

// Bounds-checked little-endian reader over the mapping.
struct Reader {
    const uint8_t *p;
    size_t size, pos = 0;
    bool ok = true;
    bool need(size_t n)
    {
        if (!ok || n > size - pos) ok = false;
        return ok;
    }
    template <class T> T get()
    {
        T v{};
        if (need(sizeof(T))) {
            memcpy(&v, p + pos, sizeof(T));
            pos += sizeof(T);
        }
        return v;
    }
    bool str(std::string *out)
    {
        const uint64_t n = get<uint64_t>();
        if (!need(n)) return false;
        if (out) out->assign((const char *)p + pos, (size_t)n);
        pos += (size_t)n;
        return true;
    }
};

size_t scalar_bytes(uint32_t t)
{
    switch (t) {
    case 0: case 1: case 7: return 1;      // u8, i8, bool
    case 2: case 3: return 2;              // u16, i16
    case 4: case 5: case 6: return 4;      // u32, i32, f32
    case 10: case 11: case 12: return 8;   // u64, i64, f64
    default: return 0;
    }
}

// Skips one value of type t (nesting depth bounded).
bool skip_value(Reader &r, uint32_t t, int depth)
{
    if (t == 8) return r.str(nullptr);
    if (t == 9) {
        if (depth > 4) return false;
        const uint32_t et = r.get<uint32_t>();
        const uint64_t n = r.get<uint64_t>();
        if (!r.ok) return false;
        const size_t sb = scalar_bytes(et);
        if (sb) return n <= (r.size - r.pos) / sb && r.need((size_t)n * sb) && ((r.pos += (size_t)n * sb), true);
        if (et != 8 && et != 9) return false;
        for (uint64_t i = 0; i < n; i++)
            if (!skip_value(r, et, depth + 1)) return false;
        return true;
    }
    const size_t sb = scalar_bytes(t);
    if (!sb || !r.need(sb)) return false;
    r.pos += sb;
    return true;
}

// Integer key/value as an unsigned 64-bit value (any integer type, non-negative).
bool kv_uint(const dmoe_gguf *g, const std::string &key, uint64_t *v)
{
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return false;
    const uint8_t *q = g->base + it->second.off;
    switch (it->second.type) {
    case 0: *v = q[0]; return true;
    case 1: { int8_t x; memcpy(&x, q, 1); if (x < 0) return false; *v = (uint64_t)x; return true; }
    case 2: { uint16_t x; memcpy(&x, q, 2); *v = x; return true; }
    case 3: { int16_t x; memcpy(&x, q, 2); if (x < 0) return false; *v = (uint64_t)x; return true; }
    case 4: { uint32_t x; memcpy(&x, q, 4); *v = x; return true; }
    case 5: { int32_t x; memcpy(&x, q, 4); if (x < 0) return false; *v = (uint64_t)x; return true; }
    case 7: *v = q[0] != 0; return true;
    case 10: { uint64_t x; memcpy(&x, q, 8); *v = x; return true; }
    case 11: { int64_t x; memcpy(&x, q, 8); if (x < 0) return false; *v = (uint64_t)x; return true; }
    default: return false;
    }
}

bool kv_float(const dmoe_gguf *g, const std::string &key, float *v)
{
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return false;
    const uint8_t *q = g->base + it->second.off;
    if (it->second.type == 6) { memcpy(v, q, 4); return true; }
    if (it->second.type == 12) { double d; memcpy(&d, q, 8); *v = (float)d; return true; }
    return false;
}

// The reference's prefix search: "diffuse.<suffix>", then "qwen2.", "llama."
// (src/diffuse-model.cpp:21-45).
const char *const kPrefixes[] = {"diffuse", "qwen2", "llama"};

int find_u32(const dmoe_gguf *g, const char *suffix, uint32_t *v)
{
    for (const char *pfx : kPrefixes) {
        const std::string key = std::string(pfx) + "." + suffix;
        if (!g->kv.count(key)) continue;
        uint64_t x = 0;
        if (!kv_uint(g, key, &x) || x > 0xFFFFFFFFull) return DMOE_ERR_FORMAT;
        *v = (uint32_t)x;
        return DMOE_OK;
    }
    return DMOE_ERR_NOT_FOUND;
}

int find_f32(const dmoe_gguf *g, const char *suffix, float *v)
{
    for (const char *pfx : kPrefixes) {
        const std::string key = std::string(pfx) + "." + suffix;
        if (!g->kv.count(key)) continue;
        return kv_float(g, key, v) ? DMOE_OK : DMOE_ERR_FORMAT;
    }
    return DMOE_ERR_NOT_FOUND;
}

// An optional key: *v = its value, or def when the key is absent.  A key
// that is present but not a non-negative integer below 2^32 is an error
// (DMOE_ERR_FORMAT), as a type mismatch is for the reference's
// gguf_get_val_u32, never a silent default.
int u32_or(const dmoe_gguf *g, const char *suffix, uint32_t def, uint32_t *v)
{
    const int rc = find_u32(g, suffix, v);
    if (rc == DMOE_ERR_NOT_FOUND) {
        *v = def;
        return DMOE_OK;
    }
    return rc;
}

int tensor_view(const dmoe_gguf *g, const std::string &name, dmoe_tensor *out)
{
    auto it = g->tensors.find(name);
    if (it == g->tensors.end()) return DMOE_ERR_NOT_FOUND;
    const dmoe_gguf::Tinfo &t = it->second;
    int64_t be = 0, bb = 0;
    if (!type_block(t.type, &be, &bb) || t.nbytes == 0) return DMOE_ERR_UNSUPPORTED_TYPE;
    dmoe_tensor v{};
    v.type = t.type;
    v.data = g->base + g->data_start + t.offset;
    for (int i = 0; i < 4; i++) v.ne[i] = i < t.n_dims ? t.ne[i] : 1;
    // ggml strides: nb[0] = bytes of one block, nb[1] = a row, then products
    v.nb[0] = (size_t)bb;
    v.nb[1] = (size_t)(v.ne[0] / be) * (size_t)bb;
    v.nb[2] = v.nb[1] * (size_t)v.ne[1];
    v.nb[3] = v.nb[2] * (size_t)v.ne[2];
    *out = v;
    return DMOE_OK;
}

std::string layer_name(const char *pattern, int il)
{
    char buf[160];
    snprintf(buf, sizeof(buf), pattern, il);
    return buf;
}

int parse(dmoe_gguf *g, char *err, size_t errlen)
{
    Reader r{g->base, g->size};
    if (!r.need(4) || memcmp(g->base, "GGUF", 4) != 0)
        return fail(err, errlen, DMOE_ERR_FORMAT, "not a GGUF file (magic)");
    r.pos = 4;
    g->version = r.get<uint32_t>();
    const uint64_t n_tensors = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
    if (!r.ok) return fail(err, errlen, DMOE_ERR_FORMAT, "truncated header");
    if (g->version < 2 || g->version > 3)
        return fail(err, errlen, DMOE_ERR_FORMAT, "GGUF version %u (2 or 3 supported)", g->version);
    // every key/value takes at least 12 bytes, every tensor info 24
    if (n_kv > g->size / 12 || n_tensors > g->size / 24)
        return fail(err, errlen, DMOE_ERR_FORMAT, "counts beyond the file size");
    for (uint64_t i = 0; i < n_kv; i++) {
        std::string key;
        if (!r.str(&key)) return fail(err, errlen, DMOE_ERR_FORMAT, "truncated key %llu", (unsigned long long)i);
        const uint32_t t = r.get<uint32_t>();
        const size_t at = r.pos;
        if (!r.ok || t > 12 || !skip_value(r, t, 0))
            return fail(err, errlen, DMOE_ERR_FORMAT, "bad value of key '%s'", key.c_str());
        g->kv[key] = dmoe_gguf::Kv{t, at};
    }
    uint64_t al = 32;
    if (g->kv.count("general.alignment") && (!kv_uint(g, "general.alignment", &al) || al == 0 || (al & (al - 1))))
        return fail(err, errlen, DMOE_ERR_FORMAT, "general.alignment is not a power of two");
    g->alignment = (uint32_t)al;
    for (uint64_t i = 0; i < n_tensors; i++) {
        std::string name;
        if (!r.str(&name)) return fail(err, errlen, DMOE_ERR_FORMAT, "truncated tensor info %llu", (unsigned long long)i);
        dmoe_gguf::Tinfo t{};
        const uint32_t nd = r.get<uint32_t>();
        if (!r.ok || nd < 1 || nd > 4)
            return fail(err, errlen, DMOE_ERR_FORMAT, "tensor '%s': %u dimensions", name.c_str(), nd);
        t.n_dims = (int32_t)nd;
        for (int d = 0; d < 4; d++) t.ne[d] = 1;
        for (uint32_t d = 0; d < nd; d++) t.ne[d] = r.get<int64_t>();
        t.type = (int32_t)r.get<uint32_t>();
        t.offset = r.get<uint64_t>();
        if (!r.ok) return fail(err, errlen, DMOE_ERR_FORMAT, "truncated tensor info '%s'", name.c_str());
        uint64_t n = 1;
        for (int d = 0; d < 4; d++) {
            if (t.ne[d] <= 0 || (uint64_t)t.ne[d] > (1ull << 40) / n)
                return fail(err, errlen, DMOE_ERR_FORMAT, "tensor '%s': bad shape", name.c_str());
            n *= (uint64_t)t.ne[d];
        }
        int64_t be = 0, bb = 0;
        if (type_block(t.type, &be, &bb)) {
            if (t.ne[0] % be)
                return fail(err, errlen, DMOE_ERR_FORMAT, "tensor '%s': ne0 not a whole number of blocks", name.c_str());
            t.nbytes = (size_t)(n / (uint64_t)be) * (size_t)bb;
        }
        if (t.offset % g->alignment)
            return fail(err, errlen, DMOE_ERR_FORMAT, "tensor '%s': misaligned offset", name.c_str());
        if (!g->tensors.emplace(name, t).second)
            return fail(err, errlen, DMOE_ERR_FORMAT, "duplicate tensor '%s'", name.c_str());
        g->tensor_order.push_back(name);
    }
    g->data_start = (r.pos + g->alignment - 1) / g->alignment * g->alignment;
    for (auto &kvp : g->tensors) {
        const dmoe_gguf::Tinfo &t = kvp.second;
        if (g->data_start > g->size || t.offset > g->size - g->data_start ||
            t.nbytes > g->size - g->data_start - t.offset)
            return fail(err, errlen, DMOE_ERR_FORMAT, "tensor '%s': data beyond the end of the file", kvp.first.c_str());
    }
    return DMOE_OK;
}

} // namespace

extern "C" {

int dmoe_gguf_open(const char *path, dmoe_gguf **out, char *err, size_t errlen)
{
    if (err && errlen) err[0] = 0;
    if (!path || !out) return fail(err, errlen, DMOE_ERR_INVALID_ARG, "path / out is NULL");
    *out = nullptr;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(err, errlen, DMOE_ERR_NOT_FOUND, "cannot open %s", path);
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 4) {
        close(fd);
        return fail(err, errlen, DMOE_ERR_FORMAT, "%s: not a GGUF file (size)", path);
    }
    void *m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) return fail(err, errlen, DMOE_ERR_OOM, "%s: mmap failed", path);
    dmoe_gguf *g = new (std::nothrow) dmoe_gguf();
    if (!g) {
        munmap(m, (size_t)st.st_size);
        return fail(err, errlen, DMOE_ERR_OOM, "host allocation failed");
    }
    g->base = (const uint8_t *)m;
    g->size = (size_t)st.st_size;
    const int rc = parse(g, err, errlen);
    if (rc) {
        dmoe_gguf_close(g);
        return rc;
    }
    *out = g;
    return DMOE_OK;
}

void dmoe_gguf_close(dmoe_gguf *g)
{
    if (!g) return;
    if (g->base) munmap((void *)g->base, g->size);
    delete g;
}

int dmoe_gguf_get_u32(const dmoe_gguf *g, const char *suffix, uint32_t *val)
{
    if (!g || !suffix || !val) return DMOE_ERR_INVALID_ARG;
    return find_u32(g, suffix, val);
}

int dmoe_gguf_get_f32(const dmoe_gguf *g, const char *suffix, float *val)
{
    if (!g || !suffix || !val) return DMOE_ERR_INVALID_ARG;
    return find_f32(g, suffix, val);
}

int dmoe_gguf_find_tensor(const dmoe_gguf *g, const char *name, dmoe_tensor *out)
{
    if (!g || !name || !out) return DMOE_ERR_INVALID_ARG;
    return tensor_view(g, name, out);
}

int dmoe_gguf_tensor_count(const dmoe_gguf *g)
{
    return g ? (int)g->tensor_order.size() : -1;
}

const char *dmoe_gguf_tensor_name(const dmoe_gguf *g, int i)
{
    if (!g || i < 0 || (size_t)i >= g->tensor_order.size()) return nullptr;
    return g->tensor_order[(size_t)i].c_str();
}

int dmoe_gguf_moe_hparams(const dmoe_gguf *g, dmoe_hparams *hp, int32_t *n_layer,
                          int32_t *first_k_dense)
{
    if (!g || !hp) return DMOE_ERR_INVALID_ARG;
    dmoe_hparams h{};
    uint32_t v = 0;
    int rc;
    // required (DIFFUSE_DIE in the reference when missing, :83-86)
    if ((rc = find_u32(g, "embedding_length", &v))) return rc;
    h.n_embd = (int32_t)v;
    uint32_t nl = 0;
    if ((rc = find_u32(g, "block_count", &nl))) return rc;
    // the MoE keys with the reference's defaults (:143-158)
    uint32_t ne = 0, nk = 0, ns = 0, nff = 0, norm = 0, cap = 0, block_length = 0, bs = 0;
    if ((rc = u32_or(g, "expert_count", 0, &ne)) || (rc = u32_or(g, "expert_used_count", 0, &nk)) ||
        (rc = u32_or(g, "expert_shared_count", 0, &ns)) ||
        (rc = u32_or(g, "expert_feed_forward_length", 0, &nff)) || (rc = u32_or(g, "norm_topk_prob", 1, &norm)) ||
        (rc = u32_or(g, "expert_capacity", 48, &cap)) || (rc = u32_or(g, "block_length", 0, &block_length)) ||
        (rc = u32_or(g, "moe_block_size", block_length ? block_length : 32, &bs)))
        return rc;
    // the counts and sizes feed int32 fields
    if (ne > INT32_MAX || nk > INT32_MAX || ns > INT32_MAX || nff > INT32_MAX || cap > INT32_MAX || bs > INT32_MAX)
        return DMOE_ERR_FORMAT;
    h.n_experts = (int32_t)ne;
    h.top_k = (int32_t)nk;
    h.n_shared = (int32_t)ns;
    h.moe_ff = (int32_t)nff;
    h.norm_topk_prob = norm != 0;
    h.capacity = (int32_t)cap;
    h.block_size = (int32_t)bs;
    float rs = 1.0f;
    if ((rc = find_f32(g, "routed_scaling_factor", &rs)) && rc != DMOE_ERR_NOT_FOUND) return rc;
    h.routed_scaling = rs;
    // shared_ff from the tensor, as the segment reads it (ne[1] of moe_shared_gate)
    h.shared_ff = 0;
    uint32_t fk = 0;
    if ((rc = u32_or(g, "first_k_dense_replace", 0, &fk))) return rc;
    if (h.n_shared > 0) {
        for (uint32_t il = fk; il < nl; il++) {
            dmoe_tensor t;
            if (tensor_view(g, layer_name("blk.%d.moe_shared_gate.weight", (int)il), &t) == DMOE_OK) {
                h.shared_ff = (int32_t)t.ne[1];
                break;
            }
        }
    }
    *hp = h;
    if (n_layer) *n_layer = (int32_t)nl;
    if (first_k_dense) *first_k_dense = (int32_t)fk;
    return DMOE_OK;
}

int dmoe_gguf_layer_desc(const dmoe_gguf *g, int32_t il, dmoe_layer_desc *desc)
{
    if (!g || !desc || il < 0) return DMOE_ERR_INVALID_ARG;
    dmoe_layer_desc d{};
    int rc;
    // src/diffuse-model.cpp:187-191 (required; the bias is optional, try_tensor)
    if ((rc = tensor_view(g, layer_name("blk.%d.moe_gate.weight", il), &d.gate_w))) return rc;
    rc = tensor_view(g, layer_name("blk.%d.moe_gate_bias.weight", il), &d.gate_bias);
    if (rc && rc != DMOE_ERR_NOT_FOUND) return rc;
    if ((rc = tensor_view(g, layer_name("blk.%d.moe_experts_gate.weight", il), &d.exp_gate))) return rc;
    if ((rc = tensor_view(g, layer_name("blk.%d.moe_experts_up.weight", il), &d.exp_up))) return rc;
    if ((rc = tensor_view(g, layer_name("blk.%d.moe_experts_down.weight", il), &d.exp_down))) return rc;
    // :192-196, present when the model has a shared expert
    uint32_t ns = 0;
    if ((rc = u32_or(g, "expert_shared_count", 0, &ns))) return rc;
    if (ns > 0) {
        if ((rc = tensor_view(g, layer_name("blk.%d.moe_shared_gate.weight", il), &d.sh_gate))) return rc;
        if ((rc = tensor_view(g, layer_name("blk.%d.moe_shared_up.weight", il), &d.sh_up))) return rc;
        if ((rc = tensor_view(g, layer_name("blk.%d.moe_shared_down.weight", il), &d.sh_down))) return rc;
    }
    *desc = d;
    return DMOE_OK;
}

int dmoe_gguf_dense_desc(const dmoe_gguf *g, int32_t il, dmoe_tensor *gate, dmoe_tensor *up,
                         dmoe_tensor *down, int32_t *n_ff)
{
    if (!g || !gate || !up || !down || il < 0) return DMOE_ERR_INVALID_ARG;
    int rc;
    // :183-185
    if ((rc = tensor_view(g, layer_name("blk.%d.ffn_gate.weight", il), gate))) return rc;
    if ((rc = tensor_view(g, layer_name("blk.%d.ffn_up.weight", il), up))) return rc;
    if ((rc = tensor_view(g, layer_name("blk.%d.ffn_down.weight", il), down))) return rc;
    if (n_ff) *n_ff = (int32_t)gate->ne[1];
    return DMOE_OK;
}

int dmoe_gguf_attn_hparams(const dmoe_gguf *g, dmoe_attn_hparams *ap)
{
    if (!g || !ap) return DMOE_ERR_INVALID_ARG;
    dmoe_attn_hparams a{};
    uint32_t v = 0;
    int rc;
    // required (:83-85)
    if ((rc = find_u32(g, "embedding_length", &v))) return rc;
    a.n_embd = (int32_t)v;
    if ((rc = find_u32(g, "attention.head_count", &v))) return rc;
    a.n_head = (int32_t)v;
    if ((rc = find_u32(g, "attention.head_count_kv", &v))) return rc;
    a.n_head_kv = (int32_t)v;
    if (a.n_head <= 0) return DMOE_ERR_FORMAT;
    // defaults as the reference's loader (:90-93, :148-150)
    uint32_t hd = 0, rd = 0, qkn = 0, bl = 0;
    if ((rc = u32_or(g, "head_dim", (uint32_t)(a.n_embd / a.n_head), &hd)) ||
        (rc = u32_or(g, "rotary_dim", hd, &rd)) || (rc = u32_or(g, "use_qk_norm", 0, &qkn)) ||
        (rc = u32_or(g, "block_length", 0, &bl)))
        return rc;
    if (hd > INT32_MAX || rd > INT32_MAX || bl > INT32_MAX) return DMOE_ERR_FORMAT;
    a.head_dim = (int32_t)hd;
    a.rotary_dim = (int32_t)rd;
    a.use_qk_norm = qkn != 0;
    a.block_length = (int32_t)bl;
    a.rope_base = 1000000.0f;
    if ((rc = find_f32(g, "rope.freq_base", &a.rope_base)) && rc != DMOE_ERR_NOT_FOUND) return rc;
    a.rms_eps = 1e-6f;
    if ((rc = find_f32(g, "attention.layer_norm_rms_epsilon", &a.rms_eps)) && rc != DMOE_ERR_NOT_FOUND)
        return rc;
    *ap = a;
    return DMOE_OK;
}

int dmoe_gguf_attn_desc(const dmoe_gguf *g, int32_t il, int32_t use_qk_norm, dmoe_attn_desc *desc)
{
    if (!g || !desc || il < 0) return DMOE_ERR_INVALID_ARG;
    dmoe_attn_desc d{};
    int rc;
    // :171-174
    if ((rc = tensor_view(g, layer_name("blk.%d.attn_norm.weight", il), &d.attn_norm))) return rc;
    if ((rc = tensor_view(g, layer_name("blk.%d.post_attn_norm.weight", il), &d.post_attn_norm))) return rc;
    if ((rc = tensor_view(g, layer_name("blk.%d.attn_qkv.weight", il), &d.qkv))) return rc;
    if ((rc = tensor_view(g, layer_name("blk.%d.attn_output.weight", il), &d.wo))) return rc;
    // :176-179, when the model uses QK norm
    if (use_qk_norm) {
        if ((rc = tensor_view(g, layer_name("blk.%d.attn_q_norm.weight", il), &d.q_norm))) return rc;
        if ((rc = tensor_view(g, layer_name("blk.%d.attn_k_norm.weight", il), &d.k_norm))) return rc;
    }
    *desc = d;
    return DMOE_OK;
}

} // extern "C"
