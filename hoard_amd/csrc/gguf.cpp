// GGUF reader for the MoE expert stage (include/hoard_gguf.h).
//
// Counterpart of the reference's load_model (src/run_moe_stream.cpp:119-186)
// and its qwen35 variant (src/run_qwen35.cpp:187-253), which read the file
// through ggml's gguf API.  The file format followed here is GGUF v2/v3:
//   u32 magic "GGUF", u32 version, u64 n_tensors, u64 n_kv,
//   n_kv x {string key, u32 value type, value}  (arrays: u32 type, u64 n, n values),
//   n_tensors x {string name, u32 n_dims, u64 ne[n_dims], u32 ggml type, u64 offset},
//   padding to general.alignment (default 32), then the tensor data, each
//   tensor at data_start + offset.
// Strings are a u64 length and the bytes.  The whole file is memory-mapped and
// every read is bounds-checked against its size.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "hoard_gguf.h"
#include "host_error.h"

using hoard::fail_fmt;

namespace {

enum : uint32_t {
    kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7,
    kString = 8, kArray = 9, kU64 = 10, kI64 = 11, kF64 = 12,
};

// ggml type ids used here and their (block elements, block bytes)
constexpr int kGgmlF32 = 0, kGgmlF16 = 1, kGgmlBF16 = 30;

bool type_block(int type, int *blk, int *bytes) {
    switch (type) {
    case 0: *blk = 1; *bytes = 4; return true;      // F32
    case 1: *blk = 1; *bytes = 2; return true;      // F16
    case 2: *blk = 32; *bytes = 18; return true;    // Q4_0
    case 3: *blk = 32; *bytes = 20; return true;    // Q4_1
    case 6: *blk = 32; *bytes = 22; return true;    // Q5_0
    case 7: *blk = 32; *bytes = 24; return true;    // Q5_1
    case 8: *blk = 32; *bytes = 34; return true;    // Q8_0
    case 9: *blk = 32; *bytes = 36; return true;    // Q8_1
    case 10: *blk = 256; *bytes = 84; return true;  // Q2_K
    case 11: *blk = 256; *bytes = 110; return true; // Q3_K
    case 12: *blk = 256; *bytes = 144; return true; // Q4_K
    case 13: *blk = 256; *bytes = 176; return true; // Q5_K
    case 14: *blk = 256; *bytes = 210; return true; // Q6_K
    case 15: *blk = 256; *bytes = 292; return true; // Q8_K
    case 24: *blk = 1; *bytes = 1; return true;     // I8
    case 25: *blk = 1; *bytes = 2; return true;     // I16
    case 26: *blk = 1; *bytes = 4; return true;     // I32
    case 27: *blk = 1; *bytes = 8; return true;     // I64
    case 28: *blk = 1; *bytes = 8; return true;     // F64
    case 30: *blk = 1; *bytes = 2; return true;     // BF16
    default: return false;
    }
}

struct Value {
    uint32_t type = 0;
    uint64_t u = 0;   // unsigned and bool values
    int64_t i = 0;    // signed values
    double f = 0.0;   // float values
    std::string s;    // strings
};

struct Tensor {
    int type = 0;
    int n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    uint64_t offset = 0;
    size_t nbytes = 0;  // 0 when the type's size is not known
};

struct Cursor {
    const uint8_t *p;
    size_t n, at = 0;
    bool ok = true;
    bool take(void *dst, size_t len) {
        if (!ok || len > n - at) return ok = false;
        std::memcpy(dst, p + at, len);
        at += len;
        return true;
    }
    template <class T>
    T get() {
        T v{};
        take(&v, sizeof v);
        return v;
    }
    bool str(std::string &s) {
        const uint64_t len = get<uint64_t>();
        if (!ok || len > n - at) return ok = false;
        s.assign(reinterpret_cast<const char *>(p + at), (size_t)len);
        at += (size_t)len;
        return true;
    }
    bool skip(size_t len) {
        if (!ok || len > n - at) return ok = false;
        at += len;
        return true;
    }
};

size_t scalar_bytes(uint32_t t) {
    switch (t) {
    case kU8: case kI8: case kBool: return 1;
    case kU16: case kI16: return 2;
    case kU32: case kI32: case kF32: return 4;
    case kU64: case kI64: case kF64: return 8;
    default: return 0;
    }
}

bool read_scalar(Cursor &c, uint32_t t, Value &v) {
    v.type = t;
    switch (t) {
    case kU8: v.u = c.get<uint8_t>(); break;
    case kI8: v.i = c.get<int8_t>(); break;
    case kBool: v.u = c.get<uint8_t>(); break;
    case kU16: v.u = c.get<uint16_t>(); break;
    case kI16: v.i = c.get<int16_t>(); break;
    case kU32: v.u = c.get<uint32_t>(); break;
    case kI32: v.i = c.get<int32_t>(); break;
    case kF32: v.f = c.get<float>(); break;
    case kU64: v.u = c.get<uint64_t>(); break;
    case kI64: v.i = c.get<int64_t>(); break;
    case kF64: v.f = c.get<double>(); break;
    case kString: return c.str(v.s);
    default: return c.ok = false;
    }
    if (t == kI8 || t == kI16 || t == kI32 || t == kI64) v.u = (uint64_t)v.i;
    else if (t != kF32 && t != kF64) v.i = (int64_t)v.u;
    return c.ok;
}

// Skips one array value (element type, count, elements); arrays may nest.
bool skip_array(Cursor &c, int depth) {
    const uint32_t et = c.get<uint32_t>();
    const uint64_t n = c.get<uint64_t>();
    if (!c.ok || depth > 8) return c.ok = false;
    if (et == kString) {
        for (uint64_t i = 0; i < n && c.ok; ++i) {
            const uint64_t len = c.get<uint64_t>();
            if (c.ok && len <= c.n - c.at) c.at += (size_t)len;
            else c.ok = false;
        }
        return c.ok;
    }
    if (et == kArray) {
        for (uint64_t i = 0; i < n && c.ok; ++i) skip_array(c, depth + 1);
        return c.ok;
    }
    const size_t sb = scalar_bytes(et);
    if (!sb || n > (c.n - c.at) / sb) return c.ok = false;
    return c.skip((size_t)(n * sb));
}

float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f, man = h & 0x3ff, bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {  // subnormal: normalise
            int e = -1;
            do {
                ++e;
                man <<= 1;
            } while ((man & 0x400) == 0);
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ff) << 13);
        }
    } else if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

}  // namespace

struct hoard_gguf {
    void *map = nullptr;
    size_t size = 0;
    const uint8_t *data = nullptr;  // tensor data start
    std::map<std::string, Value> kv;
    std::map<std::string, Tensor> tensors;
    std::string arch;
    std::vector<std::vector<float>> owned;  // f32 copies of f16 / bf16 tensors
    std::map<std::string, size_t> owned_of; // tensor name -> index into owned

    ~hoard_gguf() {
        if (map) munmap(map, size);
    }
    const Value *find(const std::string &k) const {
        auto it = kv.find(k);
        return it == kv.end() ? nullptr : &it->second;
    }
    int64_t get_int(const std::string &k, int64_t dflt) const {
        const Value *v = find(k);
        if (!v || v->type == kString || v->type == kArray || v->type == kF32 || v->type == kF64) return dflt;
        return v->i;
    }
    double get_float(const std::string &k, double dflt) const {
        const Value *v = find(k);
        if (!v) return dflt;
        if (v->type == kF32 || v->type == kF64) return v->f;
        if (v->type == kString || v->type == kArray) return dflt;
        return (double)v->i;
    }
    const Tensor *tensor(const std::string &name) const {
        auto it = tensors.find(name);
        return it == tensors.end() ? nullptr : &it->second;
    }
    const void *ptr(const Tensor &t) const { return data + t.offset; }
    // the tensor as f32: in place when stored so (4-byte aligned), else converted once
    const float *as_f32(const std::string &name, const Tensor &t) {
        if (t.type == kGgmlF32 && (reinterpret_cast<uintptr_t>(ptr(t)) & 3) == 0)
            return static_cast<const float *>(ptr(t));
        auto it = owned_of.find(name);
        if (it != owned_of.end()) return owned[it->second].data();
        const size_t n = (size_t)(t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3]);
        std::vector<float> f(n);
        const uint8_t *src = static_cast<const uint8_t *>(ptr(t));
        for (size_t i = 0; i < n; ++i) {
            uint16_t h;
            std::memcpy(&h, src + 2 * i, 2);
            if (t.type == kGgmlBF16) {
                const uint32_t bits = (uint32_t)h << 16;  // bf16 is the high half of an f32
                std::memcpy(&f[i], &bits, 4);
            } else if (t.type == kGgmlF16) {
                f[i] = half_to_float(h);
            } else {
                std::memcpy(&f[i], src + 4 * i, 4);
            }
        }
        owned.push_back(std::move(f));
        owned_of[name] = owned.size() - 1;
        return owned.back().data();
    }
};

namespace {

int parse(hoard_gguf *g, const char *path) {
    Cursor c{static_cast<const uint8_t *>(g->map), g->size};
    const uint32_t magic = c.get<uint32_t>(), version = c.get<uint32_t>();
    if (!c.ok || magic != 0x46554747u) return fail_fmt(HOARD_ERR_INVALID, "%s: not a GGUF file", path);
    if (version != 2 && version != 3)
        return fail_fmt(HOARD_ERR_UNSUPPORTED, "%s: GGUF version %u (2 and 3 are read)", path, version);
    const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
    if (!c.ok || n_tensors > (1u << 24) || n_kv > (1u << 24))
        return fail_fmt(HOARD_ERR_INVALID, "%s: implausible header (%llu tensors, %llu keys)", path,
                        (unsigned long long)n_tensors, (unsigned long long)n_kv);
    for (uint64_t k = 0; k < n_kv && c.ok; ++k) {
        std::string key;
        c.str(key);
        const uint32_t t = c.get<uint32_t>();
        Value v;
        if (t == kArray) {
            v.type = kArray;
            skip_array(c, 0);
        } else {
            read_scalar(c, t, v);
        }
        if (c.ok) g->kv[key] = std::move(v);
    }
    if (!c.ok) return fail_fmt(HOARD_ERR_INVALID, "%s: metadata runs past the end of the file", path);
    for (uint64_t k = 0; k < n_tensors && c.ok; ++k) {
        std::string name;
        c.str(name);
        Tensor t;
        const uint32_t nd = c.get<uint32_t>();
        if (!c.ok || nd == 0 || nd > 4) return fail_fmt(HOARD_ERR_INVALID, "%s: tensor %s has %u dims", path,
                                                          name.c_str(), nd);
        t.n_dims = (int)nd;
        for (uint32_t d = 0; d < nd; ++d) t.ne[d] = (int64_t)c.get<uint64_t>();
        t.type = (int)c.get<uint32_t>();
        t.offset = c.get<uint64_t>();
        int blk, bytes;
        if (c.ok && type_block(t.type, &blk, &bytes)) {
            bool good = t.ne[0] >= 0 && t.ne[0] % blk == 0;
            uint64_t n = (uint64_t)(t.ne[0] / blk) * (uint64_t)bytes;
            for (int d = 1; d < 4 && good; ++d) {
                if (t.ne[d] < 0 || (t.ne[d] && n > UINT64_MAX / (uint64_t)t.ne[d])) good = false;
                else n *= (uint64_t)t.ne[d];
            }
            if (!good) return fail_fmt(HOARD_ERR_INVALID, "%s: tensor %s has a bad shape", path, name.c_str());
            t.nbytes = (size_t)n;
        }
        if (c.ok) g->tensors[name] = t;
    }
    if (!c.ok) return fail_fmt(HOARD_ERR_INVALID, "%s: tensor infos run past the end of the file", path);
    int64_t align = g->get_int("general.alignment", 32);
    if (align <= 0 || (align & (align - 1))) align = 32;
    const size_t start = (c.at + (size_t)align - 1) & ~((size_t)align - 1);
    if (start > g->size) return fail_fmt(HOARD_ERR_INVALID, "%s: no tensor data", path);
    g->data = static_cast<const uint8_t *>(g->map) + start;
    const size_t avail = g->size - start;
    for (auto &kvp : g->tensors) {
        const Tensor &t = kvp.second;
        if (t.offset > avail || t.nbytes > avail - t.offset)
            return fail_fmt(HOARD_ERR_INVALID, "%s: tensor %s lies past the end of the file", path, kvp.first.c_str());
    }
    const Value *a = g->find("general.architecture");
    g->arch = a && a->type == kString ? a->s : "";
    return HOARD_OK;
}

bool shape_is(const Tensor &t, int64_t a, int64_t b, int64_t c) {
    return t.ne[0] == a && t.ne[1] == b && t.ne[2] == c && t.ne[3] == 1;
}

}  // namespace

extern "C" {

int hoard_gguf_open(const char *path, hoard_gguf **out) {
    if (!path || !out) return fail_fmt(HOARD_ERR_INVALID, "null argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return fail_fmt(HOARD_ERR_INVALID, "%s: cannot open", path);
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        close(fd);
        return fail_fmt(HOARD_ERR_INVALID, "%s: too short for a GGUF header", path);
    }
    void *m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) return fail_fmt(HOARD_ERR_OOM, "%s: mmap failed", path);
    hoard_gguf *g = new hoard_gguf;
    g->map = m;
    g->size = (size_t)st.st_size;
    const int rc = parse(g, path);
    if (rc) {
        delete g;
        return rc;
    }
    *out = g;
    return HOARD_OK;
}

void hoard_gguf_close(hoard_gguf *g) { delete g; }

const char *hoard_gguf_arch(const hoard_gguf *g) { return g ? g->arch.c_str() : ""; }

int hoard_gguf_moe_cfg(const hoard_gguf *g, hoard_moe_cfg *cfg) {
    if (!g || !cfg) return fail_fmt(HOARD_ERR_INVALID, "null argument");
    auto key = [&](const char *k) { return g->arch + "." + k; };
    hoard_moe_cfg c{};
    c.n_layer = (int32_t)g->get_int(key("block_count"), 0);
    c.n_embd = (int32_t)g->get_int(key("embedding_length"), 0);
    c.n_ff = (int32_t)g->get_int(key("expert_feed_forward_length"), g->get_int(key("feed_forward_length"), 0));
    c.n_expert = (int32_t)g->get_int(key("expert_count"), 0);
    c.n_used = (int32_t)g->get_int(key("expert_used_count"), 0);
    c.n_ff_shexp = (int32_t)g->get_int(key("expert_shared_feed_forward_length"), 0);
    if (c.n_ff_shexp == 0) {  // a shared expert the metadata does not size: take it from the tensor
        const Tensor *t = g->tensor("blk.0.ffn_gate_shexp.weight");
        if (t) c.n_ff_shexp = (int32_t)t->ne[1];
    }
    c.renorm = g->arch == "olmoe" ? 0 : 1;  // norm_topk_prob: OLMoE is the exception (src/run_moe_stream.cpp:149-150)
    c.pool_k = 0;
    c.max_tokens = 1;
    if (c.n_layer <= 0 || c.n_embd <= 0 || c.n_expert <= 0 || c.n_used <= 0 || c.n_ff <= 0)
        return fail_fmt(HOARD_ERR_INVALID, "GGUF (arch '%s') lacks the MoE hparams: layers %d, embd %d, experts %d/%d, ff %d",
                        g->arch.c_str(), c.n_layer, c.n_embd, c.n_used, c.n_expert, c.n_ff);
    *cfg = c;
    return HOARD_OK;
}

float hoard_gguf_rms_eps(const hoard_gguf *g) {
    if (!g) return 1e-5f;
    return (float)g->get_float(g->arch + ".attention.layer_norm_rms_epsilon", 1e-5);
}

int hoard_gguf_tensor(const hoard_gguf *g, const char *name, int32_t *type, int64_t ne[4], size_t *nbytes,
                      const void **data) {
    if (!g || !name) return fail_fmt(HOARD_ERR_INVALID, "null argument");
    const Tensor *t = g->tensor(name);
    if (!t) return fail_fmt(HOARD_ERR_INVALID, "no tensor %s", name);
    if (type) *type = t->type;
    if (ne)
        for (int d = 0; d < 4; ++d) ne[d] = t->ne[d];
    if (nbytes) *nbytes = t->nbytes;
    if (data) *data = g->ptr(*t);
    return HOARD_OK;
}

int hoard_gguf_layer_weights(hoard_gguf *g, int layer, hoard_layer_weights *w) {
    if (!g || !w) return fail_fmt(HOARD_ERR_INVALID, "null argument");
    hoard_moe_cfg c;
    if (int rc = hoard_gguf_moe_cfg(g, &c)) return rc;
    if (layer < 0 || layer >= c.n_layer) return fail_fmt(HOARD_ERR_INVALID, "layer %d outside 0..%d", layer, c.n_layer - 1);
    auto name = [&](const char *t) { return "blk." + std::to_string(layer) + "." + t + ".weight"; };
    auto need = [&](const char *t, const Tensor **out) {
        *out = g->tensor(name(t));
        if (!*out) return fail_fmt(HOARD_ERR_INVALID, "no tensor %s", name(t).c_str());
        if ((*out)->nbytes == 0) return fail_fmt(HOARD_ERR_UNSUPPORTED, "%s: ggml type %d", name(t).c_str(), (*out)->type);
        return HOARD_OK;
    };
    auto f32ish = [](const Tensor *t) { return t->type == kGgmlF32 || t->type == kGgmlF16 || t->type == kGgmlBF16; };
    hoard_layer_weights r{};
    const Tensor *tr, *tg, *tu, *td;
    if (int rc = need("ffn_gate_inp", &tr)) return rc;
    if (!f32ish(tr) || !shape_is(*tr, c.n_embd, c.n_expert, 1))
        return fail_fmt(HOARD_ERR_INVALID, "%s: want f32/f16/bf16 [%d, %d]", name("ffn_gate_inp").c_str(), c.n_embd,
                        c.n_expert);
    if (int rc = need("ffn_gate_exps", &tg)) return rc;
    if (int rc = need("ffn_up_exps", &tu)) return rc;
    if (int rc = need("ffn_down_exps", &td)) return rc;
    if (!shape_is(*tg, c.n_embd, c.n_ff, c.n_expert) || !shape_is(*tu, c.n_embd, c.n_ff, c.n_expert) ||
        !shape_is(*td, c.n_ff, c.n_embd, c.n_expert))
        return fail_fmt(HOARD_ERR_INVALID, "layer %d: expert tensors do not have the shapes [%d, %d, %d] / [%d, %d, %d]",
                        layer, c.n_embd, c.n_ff, c.n_expert, c.n_ff, c.n_embd, c.n_expert);
    r.router = g->as_f32(name("ffn_gate_inp"), *tr);
    r.gate_type = tg->type;
    r.up_type = tu->type;
    r.down_type = td->type;
    r.gate = g->ptr(*tg);
    r.up = g->ptr(*tu);
    r.down = g->ptr(*td);
    if (c.n_ff_shexp > 0) {
        const Tensor *sg, *su, *sd, *si;
        if (int rc = need("ffn_gate_shexp", &sg)) return rc;
        if (int rc = need("ffn_up_shexp", &su)) return rc;
        if (int rc = need("ffn_down_shexp", &sd)) return rc;
        if (int rc = need("ffn_gate_inp_shexp", &si)) return rc;
        if (!shape_is(*sg, c.n_embd, c.n_ff_shexp, 1) || !shape_is(*su, c.n_embd, c.n_ff_shexp, 1) ||
            !shape_is(*sd, c.n_ff_shexp, c.n_embd, 1) || !f32ish(si) ||
            !(shape_is(*si, c.n_embd, 1, 1)))
            return fail_fmt(HOARD_ERR_INVALID, "layer %d: shared-expert tensors do not have the shapes for ff %d", layer,
                            c.n_ff_shexp);
        r.sh_gate_type = sg->type;
        r.sh_up_type = su->type;
        r.sh_down_type = sd->type;
        r.sh_gate = g->ptr(*sg);
        r.sh_up = g->ptr(*su);
        r.sh_down = g->ptr(*sd);
        r.sh_gate_inp = g->as_f32(name("ffn_gate_inp_shexp"), *si);
    }
    *w = r;
    return HOARD_OK;
}

int hoard_gguf_store_layers(const hoard_gguf *g, hoard_store_layer *layers, int n_layer) {
    if (!g || !layers) return fail_fmt(HOARD_ERR_INVALID, "null argument");
    hoard_moe_cfg c;
    if (int rc = hoard_gguf_moe_cfg(g, &c)) return rc;
    if (n_layer != c.n_layer) return fail_fmt(HOARD_ERR_INVALID, "%d layers asked of a file of %d", n_layer, c.n_layer);
    const uint8_t *base = static_cast<const uint8_t *>(g->map);
    static const char *kParts[3] = {"ffn_gate_exps", "ffn_up_exps", "ffn_down_exps"};
    for (int l = 0; l < n_layer; ++l)
        for (int i = 0; i < 3; ++i) {
            const std::string name = "blk." + std::to_string(l) + "." + kParts[i] + ".weight";
            const Tensor *t = g->tensor(name);
            if (!t) return fail_fmt(HOARD_ERR_INVALID, "no tensor %s", name.c_str());
            if (t->nbytes == 0 || t->ne[2] != c.n_expert || t->nbytes % (size_t)c.n_expert)
                return fail_fmt(HOARD_ERR_INVALID, "%s is not %d experts of a known type", name.c_str(), c.n_expert);
            layers[l].off[i] = (uint64_t)(static_cast<const uint8_t *>(g->ptr(*t)) - base);
            layers[l].stride[i] = (uint64_t)(t->nbytes / (size_t)c.n_expert);
        }
    return HOARD_OK;
}

}  // extern "C"
