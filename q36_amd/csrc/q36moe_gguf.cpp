// GGUF v3 ingest of the MoE tensors (host C++).
//
// Replaces the path gguf_open (gguf.c) -> bind_moe (q36_model.c:54-77) ->
// upload() (q36_engine.cu:196-228) for the expert weights: the file is
// mapped read-only, the header, metadata and tensor directory are parsed
// (the data is never copied), and the MXFP4 expert tensors of a block go
// straight to q36moe_weights_upload, which repacks them into the MFMA
// fragment layout.
//
// File layout (GGUF v3, little endian):
//   "GGUF" | u32 version | u64 n_tensors | u64 n_kv
//   n_kv x  { string key | u32 type | value }
//   n_tensors x { string name | u32 n_dims | u64 dims[n_dims] | u32 ggml_type | u64 offset }
//   padding to `general.alignment` (default 32) | tensor data (offsets relative to here)
// string = u64 length + bytes (no terminator); array value = u32 element type
// + u64 count + elements; dims[0] is the innermost (contiguous) extent.
#include "q36moe.h"

#include <cerrno>
#include <cstdlib>
#include <cstring>
#include <fcntl.h>
#include <new>
#include <string>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include <unordered_map>
#include <vector>

namespace {

enum : uint32_t {
    V_U8 = 0, V_I8 = 1, V_U16 = 2, V_I16 = 3, V_U32 = 4, V_I32 = 5, V_F32 = 6, V_BOOL = 7,
    V_STR = 8, V_ARR = 9, V_U64 = 10, V_I64 = 11, V_F64 = 12,
};

enum : uint32_t { T_F32 = 0, T_F16 = 1, T_Q8_0 = 8, T_Q5_K = 13, T_Q6_K = 14, T_BF16 = 30, T_MXFP4 = 39 };

// bytes per block and elements per block of the tensor types the q36 files use
bool type_block(uint32_t t, uint64_t *bytes, uint64_t *elems) {
    switch (t) {
        case T_F32: *bytes = 4; *elems = 1; return true;
        case T_F16: case T_BF16: *bytes = 2; *elems = 1; return true;
        case T_Q8_0: *bytes = 34; *elems = 32; return true;
        case T_Q5_K: *bytes = 176; *elems = 256; return true;
        case T_Q6_K: *bytes = 210; *elems = 256; return true;
        case T_MXFP4: *bytes = 17; *elems = 32; return true;
        default: return false;
    }
}

size_t scalar_size(uint32_t t) {
    switch (t) {
        case V_U8: case V_I8: case V_BOOL: return 1;
        case V_U16: case V_I16: return 2;
        case V_U32: case V_I32: case V_F32: return 4;
        case V_U64: case V_I64: case V_F64: return 8;
        default: return 0;
    }
}

struct Reader {
    const uint8_t *p, *end;
    bool get(void *dst, size_t n) {
        if ((size_t)(end - p) < n) return false;
        if (dst) memcpy(dst, p, n);
        p += n;
        return true;
    }
    bool u32(uint32_t *v) { return get(v, 4); }
    bool u64(uint64_t *v) { return get(v, 8); }
    bool str(std::string *s) {
        uint64_t n;
        if (!u64(&n) || (uint64_t)(end - p) < n) return false;
        if (s) s->assign(reinterpret_cast<const char *>(p), (size_t)n);
        p += n;
        return true;
    }
};

struct Kv {
    uint32_t type;
    const uint8_t *value;   // scalar payload (for scalar types)
};

struct Tensor {
    std::string name;
    uint32_t n_dims, type;
    uint64_t dims[4];
    uint64_t offset;        // within the data section
    uint64_t nbytes;        // 0 for types without a known block size
};

}  // namespace

struct q36moe_gguf {
    int fd = -1;
    void *map = MAP_FAILED;
    size_t size = 0;
    uint32_t version = 0, alignment = 32;
    uint64_t data_off = 0;
    std::unordered_map<std::string, Kv> kv;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> by_name;
};

namespace {

int parse(q36moe_gguf *g) {
    Reader r{static_cast<const uint8_t *>(g->map), static_cast<const uint8_t *>(g->map) + g->size};
    char magic[4];
    uint64_t n_tensors, n_kv;
    if (!r.get(magic, 4) || memcmp(magic, "GGUF", 4) != 0) return Q36MOE_EINVAL;
    if (!r.u32(&g->version) || g->version != 3) return Q36MOE_EINVAL;
    if (!r.u64(&n_tensors) || !r.u64(&n_kv)) return Q36MOE_EINVAL;
    // every kv and tensor record takes at least 12 bytes: bound the counts
    // by the file size before reserving anything
    if (n_kv > g->size / 12 || n_tensors > g->size / 12) return Q36MOE_EINVAL;
    for (uint64_t i = 0; i < n_kv; i++) {
        std::string key;
        uint32_t t;
        if (!r.str(&key) || !r.u32(&t)) return Q36MOE_EINVAL;
        Kv v{t, r.p};
        if (t == V_STR) {
            if (!r.str(nullptr)) return Q36MOE_EINVAL;
        } else if (t == V_ARR) {
            uint32_t et;
            uint64_t n;
            if (!r.u32(&et) || !r.u64(&n)) return Q36MOE_EINVAL;
            if (et == V_STR) {
                for (uint64_t j = 0; j < n; j++)
                    if (!r.str(nullptr)) return Q36MOE_EINVAL;
            } else {
                const size_t es = scalar_size(et);
                if (es == 0 || n > (uint64_t)(r.end - r.p) / es || !r.get(nullptr, es * n)) return Q36MOE_EINVAL;
            }
        } else {
            const size_t es = scalar_size(t);
            if (es == 0 || !r.get(nullptr, es)) return Q36MOE_EINVAL;
        }
        g->kv[key] = v;
    }
    g->tensors.resize(n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
        Tensor &t = g->tensors[i];
        if (!r.str(&t.name) || !r.u32(&t.n_dims) || t.n_dims < 1 || t.n_dims > 4) return Q36MOE_EINVAL;
        for (uint32_t d = 0; d < 4; d++) t.dims[d] = 1;
        for (uint32_t d = 0; d < t.n_dims; d++)
            if (!r.u64(&t.dims[d])) return Q36MOE_EINVAL;
        if (!r.u32(&t.type) || !r.u64(&t.offset)) return Q36MOE_EINVAL;
        if (!g->by_name.emplace(t.name, i).second) return Q36MOE_EINVAL;   // duplicate name
    }
    auto al = g->kv.find("general.alignment");
    if (al != g->kv.end()) {
        if (al->second.type != V_U32) return Q36MOE_EINVAL;
        uint32_t a;
        memcpy(&a, al->second.value, 4);
        if (a == 0) return Q36MOE_EINVAL;
        g->alignment = a;
    }
    const uint64_t here = (uint64_t)(r.p - static_cast<const uint8_t *>(g->map));
    g->data_off = (here + g->alignment - 1) / g->alignment * g->alignment;
    for (Tensor &t : g->tensors) {
        uint64_t bb, be, n = 1;
        for (uint32_t d = 0; d < t.n_dims; d++) {
            if (t.dims[d] && n > UINT64_MAX / t.dims[d]) return Q36MOE_EINVAL;
            n *= t.dims[d];
        }
        t.nbytes = type_block(t.type, &bb, &be) ? n / be * bb : 0;
        if (type_block(t.type, &bb, &be) && n % be) return Q36MOE_EINVAL;
        if (t.offset > g->size || g->data_off > g->size - t.offset ||
            t.nbytes > g->size - g->data_off - t.offset)
            return Q36MOE_EINVAL;   // runs past the end of the file
    }
    return Q36MOE_OK;
}

const Tensor *find(const q36moe_gguf *g, const std::string &name) {
    auto it = g->by_name.find(name);
    return it == g->by_name.end() ? nullptr : &g->tensors[it->second];
}

const uint8_t *data_of(const q36moe_gguf *g, const Tensor *t) {
    return static_cast<const uint8_t *>(g->map) + g->data_off + t->offset;
}

std::string blk(int layer, const char *suffix) { return "blk." + std::to_string(layer) + "." + suffix; }

// bf16 -> f32 is exact (the upper half of the f32 pattern)
float bf16_to_f32(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

}  // namespace

extern "C" {

int q36moe_gguf_open(const char *path, q36moe_gguf **out) {
    if (!path || !out) return Q36MOE_EINVAL;
    *out = nullptr;
    q36moe_gguf *g = new (std::nothrow) q36moe_gguf();
    if (!g) return Q36MOE_ENOMEM;
    g->fd = open(path, O_RDONLY | O_CLOEXEC);
    struct stat st;
    if (g->fd < 0 || fstat(g->fd, &st) != 0 || st.st_size <= 0) {
        q36moe_gguf_close(g);
        return Q36MOE_EIO;
    }
    g->size = (size_t)st.st_size;
    g->map = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (g->map == MAP_FAILED) {
        q36moe_gguf_close(g);
        return Q36MOE_EIO;
    }
    // the experts are read once, front to back, by the upload
    (void)madvise(g->map, g->size, MADV_SEQUENTIAL);
    int rc;
    try {
        rc = parse(g);
    } catch (const std::bad_alloc &) {
        rc = Q36MOE_ENOMEM;
    }
    if (rc) {
        q36moe_gguf_close(g);
        return rc;
    }
    *out = g;
    return Q36MOE_OK;
}

void q36moe_gguf_close(q36moe_gguf *g) {
    if (!g) return;
    if (g->map != MAP_FAILED) munmap(g->map, g->size);
    if (g->fd >= 0) close(g->fd);
    delete g;
}

int q36moe_gguf_info(const q36moe_gguf *g, uint32_t *version, uint64_t *n_tensors, uint64_t *n_kv,
                     uint32_t *alignment, uint64_t *data_offset) {
    if (!g) return Q36MOE_EINVAL;
    if (version) *version = g->version;
    if (n_tensors) *n_tensors = g->tensors.size();
    if (n_kv) *n_kv = g->kv.size();
    if (alignment) *alignment = g->alignment;
    if (data_offset) *data_offset = g->data_off;
    return Q36MOE_OK;
}

int q36moe_gguf_tensor(const q36moe_gguf *g, const char *name, uint32_t *ggml_type, uint32_t *n_dims,
                       uint64_t *dims, uint64_t *file_offset, const void **data, uint64_t *nbytes) {
    if (!g || !name) return Q36MOE_EINVAL;
    const Tensor *t = find(g, name);
    if (!t) return Q36MOE_ENOENT;
    if (ggml_type) *ggml_type = t->type;
    if (n_dims) *n_dims = t->n_dims;
    if (dims)
        for (int d = 0; d < 4; d++) dims[d] = t->dims[d];
    if (file_offset) *file_offset = g->data_off + t->offset;
    if (data) *data = data_of(g, t);
    if (nbytes) *nbytes = t->nbytes;
    return Q36MOE_OK;
}

int q36moe_gguf_u32(const q36moe_gguf *g, const char *key, uint32_t *out) {
    if (!g || !key || !out) return Q36MOE_EINVAL;
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return Q36MOE_ENOENT;
    if (it->second.type != V_U32) return Q36MOE_EINVAL;
    memcpy(out, it->second.value, 4);
    return Q36MOE_OK;
}

int q36moe_weights_from_gguf(const q36moe_gguf *g, int layer, int with_shared, q36moe_weights **out) {
    if (!g || !out || layer < 0) return Q36MOE_EINVAL;
    *out = nullptr;
    const Tensor *gt = find(g, blk(layer, "ffn_gate_exps.weight"));
    const Tensor *ut = find(g, blk(layer, "ffn_up_exps.weight"));
    const Tensor *dt = find(g, blk(layer, "ffn_down_exps.weight"));
    if (!gt || !ut || !dt) return Q36MOE_ENOENT;
    // gate/up MXFP4; down MXFP4 or one of the reference's requantised
    // fallback types (Q5_K / Q6_K experts of real files, and Q8_0)
    if (gt->type != T_MXFP4 || ut->type != T_MXFP4) return Q36MOE_EINVAL;
    if (dt->type != T_MXFP4 && dt->type != T_Q5_K && dt->type != T_Q6_K && dt->type != T_Q8_0)
        return Q36MOE_EINVAL;
    // ggml order: gate/up [d_model][d_ff][E], down [d_ff][d_model][E]
    if (gt->n_dims != 3 || ut->n_dims != 3 || dt->n_dims != 3) return Q36MOE_EINVAL;
    const uint64_t D = gt->dims[0], FF = gt->dims[1], E = gt->dims[2];
    if (ut->dims[0] != D || ut->dims[1] != FF || ut->dims[2] != E || dt->dims[0] != FF ||
        dt->dims[1] != D || dt->dims[2] != E || D > (1u << 20) || FF > (1u << 20) || E > (1u << 20))
        return Q36MOE_EINVAL;
    const uint8_t *sg = nullptr, *su = nullptr, *sd = nullptr;
    int ff_sh = 0, sh_type = (int)T_MXFP4;
    if (with_shared) {
        const Tensor *a = find(g, blk(layer, "ffn_gate_shexp.weight"));
        const Tensor *b = find(g, blk(layer, "ffn_up_shexp.weight"));
        const Tensor *c = find(g, blk(layer, "ffn_down_shexp.weight"));
        if (!a || !b || !c) return Q36MOE_ENOENT;
        // one type for all three; MXFP4 or one of the split-Q8 sources
        if (a->type != b->type || a->type != c->type) return Q36MOE_EINVAL;
        if (a->type != T_MXFP4 && a->type != T_Q8_0 && a->type != T_Q5_K && a->type != T_Q6_K)
            return Q36MOE_EINVAL;
        sh_type = (int)a->type;
        if (a->dims[0] != D || a->dims[1] != FF || b->dims[0] != D || b->dims[1] != FF || c->dims[0] != FF ||
            c->dims[1] != D || a->dims[2] != 1 || b->dims[2] != 1 || c->dims[2] != 1)
            return Q36MOE_EINVAL;
        sg = data_of(g, a);
        su = data_of(g, b);
        sd = data_of(g, c);
        ff_sh = (int)FF;
    }
    return q36moe_weights_upload_typed(data_of(g, gt), data_of(g, ut), data_of(g, dt), (int)dt->type, sg, su,
                                       sd, sh_type, (int)E, (int)D, (int)FF, ff_sh, out);
}

int q36moe_router_from_gguf(const q36moe_gguf *g, int layer, float *dst, size_t dst_floats, int *n_rows,
                            int *d_model) {
    if (!g || !dst || layer < 0) return Q36MOE_EINVAL;
    const Tensor *r = find(g, blk(layer, "ffn_gate_inp.weight"));
    if (!r) return Q36MOE_ENOENT;
    const Tensor *s = find(g, blk(layer, "ffn_gate_inp_shexp.weight"));
    if (r->n_dims != 2 || (r->type != T_F32 && r->type != T_BF16)) return Q36MOE_EINVAL;
    const uint64_t D = r->dims[0], E = r->dims[1];
    if (s && (s->type != T_F32 && s->type != T_BF16)) return Q36MOE_EINVAL;
    if (s && s->dims[0] * s->dims[1] * s->dims[2] * s->dims[3] != D) return Q36MOE_EINVAL;
    const uint64_t rows = E + (s ? 1 : 0);
    if (D > (1u << 20) || E > (1u << 20) || rows * D > dst_floats) return Q36MOE_EINVAL;
    auto widen = [&](const Tensor *t, float *o, uint64_t n) {
        const uint8_t *p = data_of(g, t);
        if (t->type == T_F32) {
            memcpy(o, p, n * 4);
        } else {
            for (uint64_t i = 0; i < n; i++) {
                uint16_t h;
                memcpy(&h, p + 2 * i, 2);
                o[i] = bf16_to_f32(h);
            }
        }
    };
    widen(r, dst, E * D);
    if (s) widen(s, dst + E * D, D);
    if (n_rows) *n_rows = (int)rows;
    if (d_model) *d_model = (int)D;
    return Q36MOE_OK;
}

}  // extern "C"
