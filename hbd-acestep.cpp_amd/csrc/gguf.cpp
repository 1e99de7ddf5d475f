// GGUF reader and load-time weight preparation.
//
// Replaces the reference's weight loader (gguf-weights.h:74-354): gf_load
// (mmap, header parse through ggml's gguf_init_from_file, and a check that
// every tensor lies inside the file), gf_load_tensor / gf_load_tensor_f32 (raw
// bytes, or F16/BF16 widened to F32 for the small tensors), gf_load_qkv_fused /
// gf_load_pair_fused (row concatenation of projections that share ne0 and
// type) and the gf_get_u32/f32/str/bool metadata getters (gguf-weights.h:356-390).
// ggml's GGUF parser is not in the reference checkout; this one follows the
// published GGUF format (versions 2 and 3, little-endian):
//   magic "GGUF", u32 version, u64 tensor count, u64 KV count,
//   KV: string key, u32 value type, value (u8 i8 u16 i16 u32 i32 f32 bool
//       string array u64 i64 f64 = types 0..12; array = u32 element type,
//       u64 count, elements; string = u64 length, bytes),
//   tensor info: string name, u32 n_dims, u64 ne[n_dims], u32 ggml type,
//       u64 offset (from the data section, a multiple of the alignment),
//   data section at the header end rounded up to general.alignment (u32,
//   default 32).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "launch.h"

namespace {

enum : uint32_t {
    GT_U8 = 0, GT_I8, GT_U16, GT_I16, GT_U32, GT_I32, GT_F32, GT_BOOL, GT_STR, GT_ARR, GT_U64, GT_I64, GT_F64,
};

// block size and bytes per block of the ggml types a GGUF tensor may hold
bool type_geom(uint32_t t, int64_t & blk, int64_t & bytes) {
    switch (t) {
        case 0: blk = 1; bytes = 4; return true;      // F32
        case 1: blk = 1; bytes = 2; return true;      // F16
        case 2: blk = 32; bytes = 18; return true;    // Q4_0
        case 3: blk = 32; bytes = 20; return true;    // Q4_1
        case 6: blk = 32; bytes = 22; return true;    // Q5_0
        case 7: blk = 32; bytes = 24; return true;    // Q5_1
        case 8: blk = 32; bytes = 34; return true;    // Q8_0
        case 9: blk = 32; bytes = 36; return true;    // Q8_1
        case 10: blk = 256; bytes = 84; return true;  // Q2_K
        case 11: blk = 256; bytes = 110; return true; // Q3_K
        case 12: blk = 256; bytes = 144; return true; // Q4_K
        case 13: blk = 256; bytes = 176; return true; // Q5_K
        case 14: blk = 256; bytes = 210; return true; // Q6_K
        case 15: blk = 256; bytes = 292; return true; // Q8_K
        case 24: blk = 1; bytes = 1; return true;     // I8
        case 25: blk = 1; bytes = 2; return true;     // I16
        case 26: blk = 1; bytes = 4; return true;     // I32
        case 27: blk = 1; bytes = 8; return true;     // I64
        case 28: blk = 1; bytes = 8; return true;     // F64
        case 30: blk = 1; bytes = 2; return true;     // BF16
        default: return false;
    }
}

size_t scalar_size(uint32_t t) {
    switch (t) {
        case GT_U8: case GT_I8: case GT_BOOL: return 1;
        case GT_U16: case GT_I16: return 2;
        case GT_U32: case GT_I32: case GT_F32: return 4;
        case GT_U64: case GT_I64: case GT_F64: return 8;
        default: return 0;
    }
}

struct Cursor {
    const uint8_t * p;
    size_t          n, at = 0;
    bool            ok = true;
    bool need(size_t k) {
        if (!ok || k > n - at) {
            ok = false;
        }
        return ok;
    }
    template <typename T> T get() {
        T v{};
        if (need(sizeof(T))) {
            memcpy(&v, p + at, sizeof(T));
            at += sizeof(T);
        }
        return v;
    }
    // a GGUF string: returns its position and length
    bool str(size_t & pos, uint64_t & len) {
        len = get<uint64_t>();
        if (!ok || !need(len)) {
            return false;
        }
        pos = at;
        at += len;
        return true;
    }
    bool skip_value(uint32_t type, int depth = 0) {
        if (type == GT_STR) {
            size_t   pos;
            uint64_t len;
            return str(pos, len);
        }
        if (type == GT_ARR) {
            if (depth > 0) {
                ok = false;  // nested arrays are not GGUF
                return false;
            }
            const uint32_t et = get<uint32_t>();
            const uint64_t cnt = get<uint64_t>();
            if (!ok) {
                return false;
            }
            if (et == GT_STR) {
                for (uint64_t i = 0; i < cnt && ok; ++i) {
                    skip_value(GT_STR, depth + 1);
                }
                return ok;
            }
            const size_t es = scalar_size(et);
            if (es == 0 || cnt > (n - at) / es) {
                ok = false;
                return false;
            }
            at += cnt * es;
            return true;
        }
        const size_t es = scalar_size(type);
        if (es == 0) {
            ok = false;
            return false;
        }
        if (need(es)) {
            at += es;
        }
        return ok;
    }
};

}  // namespace

struct mi_gguf {
    int       fd   = -1;
    uint8_t * map  = nullptr;
    size_t    size = 0;
    uint32_t  version = 0;
    size_t    alignment = 32, data_offset = 0;
    struct KV {
        std::string key;
        uint32_t    type;
        size_t      at;  // value position in the mapping (after the type)
    };
    struct TI {
        std::string name;
        uint32_t    type;
        int32_t     n_dims;
        int64_t     ne[4];
        uint64_t    offset, nbytes;
    };
    std::vector<KV>                          kv;
    std::vector<TI>                          ti;
    std::unordered_map<std::string, int64_t> kidx, tidx;
    std::vector<std::string>                 strs;  // string values, NUL-terminated copies
    std::unordered_map<int64_t, size_t>      kstr;  // KV index -> strs index
};

namespace {

void gguf_free(mi_gguf * g) {
    if (!g) {
        return;
    }
    if (g->map) {
        munmap(g->map, g->size);
    }
    if (g->fd >= 0) {
        close(g->fd);
    }
    delete g;
}

int gguf_parse(mi_gguf * g) {
    Cursor c{ g->map, g->size };
    const uint32_t magic = c.get<uint32_t>();
    if (!c.ok || magic != 0x46554747u) {  // "GGUF"
        return MI_ERR_FILE;
    }
    g->version = c.get<uint32_t>();
    if (g->version != 2 && g->version != 3) {
        return MI_ERR_FILE;
    }
    const uint64_t nt = c.get<uint64_t>(), nk = c.get<uint64_t>();
    if (!c.ok || nt > g->size / 24 || nk > g->size / 12) {
        return MI_ERR_FILE;
    }
    for (uint64_t i = 0; i < nk; ++i) {
        size_t   pos;
        uint64_t len;
        if (!c.str(pos, len)) {
            return MI_ERR_FILE;
        }
        mi_gguf::KV e{ std::string((const char *) g->map + pos, len), c.get<uint32_t>(), 0 };
        e.at = c.at;
        if (!c.ok || !c.skip_value(e.type)) {
            return MI_ERR_FILE;
        }
        if (g->kidx.count(e.key)) {
            return MI_ERR_FILE;  // duplicate key
        }
        const int64_t ki = (int64_t) g->kv.size();
        g->kidx[e.key] = ki;
        if (e.type == GT_STR) {
            uint64_t sl;
            memcpy(&sl, g->map + e.at, 8);
            g->kstr[ki] = g->strs.size();
            g->strs.emplace_back((const char *) g->map + e.at + 8, sl);
        }
        if (e.key == "general.alignment") {
            if (e.type != GT_U32) {
                return MI_ERR_FILE;
            }
            uint32_t a;
            memcpy(&a, g->map + e.at, 4);
            if (a == 0 || (a & (a - 1)) != 0) {
                return MI_ERR_FILE;
            }
            g->alignment = a;
        }
        g->kv.push_back(std::move(e));
    }
    for (uint64_t i = 0; i < nt; ++i) {
        size_t   pos;
        uint64_t len;
        if (!c.str(pos, len)) {
            return MI_ERR_FILE;
        }
        mi_gguf::TI t{};
        t.name   = std::string((const char *) g->map + pos, len);
        t.n_dims = (int32_t) c.get<uint32_t>();
        if (!c.ok || t.n_dims < 1 || t.n_dims > 4) {
            return MI_ERR_FILE;
        }
        for (int d = 0; d < 4; ++d) {
            t.ne[d] = 1;
        }
        for (int d = 0; d < t.n_dims; ++d) {
            const uint64_t v = c.get<uint64_t>();
            if (v > (uint64_t) INT64_MAX / 2) {
                return MI_ERR_FILE;
            }
            t.ne[d] = (int64_t) v;
        }
        t.type   = c.get<uint32_t>();
        t.offset = c.get<uint64_t>();
        if (!c.ok) {
            return MI_ERR_FILE;
        }
        int64_t blk, bytes;
        if (!type_geom(t.type, blk, bytes)) {
            return MI_ERR_TYPE;  // a ggml type this reader has no block size for
        }
        if (t.ne[0] % blk != 0) {
            return MI_ERR_FILE;
        }
        // element count and byte count with every product checked: a
        // wrapped product would describe a huge tensor over a small region
        int64_t nel = t.ne[0], nb = 0;
        for (int d = 1; d < 4; ++d) {
            if (__builtin_mul_overflow(nel, t.ne[d], &nel)) {
                return MI_ERR_FILE;
            }
        }
        if (__builtin_mul_overflow(nel / blk, bytes, &nb) || (uint64_t) nb > g->size) {
            return MI_ERR_FILE;
        }
        t.nbytes = (uint64_t) nb;
        if (g->tidx.count(t.name)) {
            return MI_ERR_FILE;  // duplicate tensor name
        }
        g->tidx[t.name] = (int64_t) g->ti.size();
        g->ti.push_back(std::move(t));
    }
    g->data_offset = (c.at + g->alignment - 1) / g->alignment * g->alignment;
    // every tensor aligned and inside the file (gguf-weights.h:130-148)
    for (const auto & t : g->ti) {
        if (t.offset % g->alignment != 0) {
            return MI_ERR_FILE;
        }
        if (t.offset > g->size || g->data_offset > g->size - t.offset ||
            t.nbytes > g->size - g->data_offset - t.offset) {
            return MI_ERR_FILE;
        }
    }
    return MI_OK;
}

const mi_gguf::KV * kv_of(const mi_gguf * g, const char * key) {
    if (!g || !key) {
        return nullptr;
    }
    const auto it = g->kidx.find(key);
    return it == g->kidx.end() ? nullptr : &g->kv[(size_t) it->second];
}

const mi_gguf::TI * ti_of(const mi_gguf * g, const char * name) {
    if (!g || !name) {
        return nullptr;
    }
    const auto it = g->tidx.find(name);
    return it == g->tidx.end() ? nullptr : &g->ti[(size_t) it->second];
}

float h2f(uint16_t h) {
    const uint32_t s = (uint32_t) (h >> 15) << 31;
    uint32_t       e = (h >> 10) & 31, m = h & 1023, u;
    if (e == 0) {
        if (m == 0) {
            u = s;
        } else {  // subnormal: normalize
            e = 113;
            while ((m & 1024) == 0) {
                m <<= 1;
                --e;
            }
            u = s | (e << 23) | ((m & 1023) << 13);
        }
    } else if (e == 31) {
        u = s | 0x7F800000u | (m << 13);
    } else {
        u = s | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

int copy_to_device(void * dst, const void * src, size_t n, hipStream_t s) {
    if (n == 0) {
        return MI_OK;
    }
    if (hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess) {
        return MI_ERR_HIP;
    }
    return MI_OK;
}

}  // namespace

extern "C" {

int mi_gguf_open(const char * path, mi_gguf ** out) {
    if (!path || !out) {
        return MI_ERR_NULL;
    }
    *out       = nullptr;
    mi_gguf * g = new mi_gguf();
    g->fd      = open(path, O_RDONLY);
    struct stat sb;
    if (g->fd < 0 || fstat(g->fd, &sb) != 0 || sb.st_size < 24) {
        gguf_free(g);
        return MI_ERR_FILE;
    }
    g->size = (size_t) sb.st_size;
    void * m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) {
        gguf_free(g);
        return MI_ERR_FILE;
    }
    g->map       = (uint8_t *) m;
    const int rc = gguf_parse(g);
    if (rc != MI_OK) {
        gguf_free(g);
        return rc;
    }
    *out = g;
    return MI_OK;
}

void mi_gguf_close(mi_gguf * g) {
    gguf_free(g);
}

int64_t mi_gguf_n_tensors(const mi_gguf * g) {
    return g ? (int64_t) g->ti.size() : -1;
}

int64_t mi_gguf_find_tensor(const mi_gguf * g, const char * name) {
    if (!g || !name) {
        return -1;
    }
    const auto it = g->tidx.find(name);
    return it == g->tidx.end() ? -1 : it->second;
}

int mi_gguf_get_tensor(const mi_gguf * g, int64_t idx, mi_gguf_tensor * t) {
    if (!g || !t) {
        return MI_ERR_NULL;
    }
    if (idx < 0 || idx >= (int64_t) g->ti.size()) {
        return MI_ERR_PARAM;
    }
    const auto & s = g->ti[(size_t) idx];
    t->name        = s.name.c_str();
    t->type        = (int32_t) s.type;
    t->n_dims      = s.n_dims;
    for (int d = 0; d < 4; ++d) {
        t->ne[d] = s.ne[d];
    }
    t->nbytes = s.nbytes;
    t->data   = g->map + g->data_offset + s.offset;
    return MI_OK;
}

int64_t mi_gguf_n_kv(const mi_gguf * g) {
    return g ? (int64_t) g->kv.size() : -1;
}

int64_t mi_gguf_find_key(const mi_gguf * g, const char * key) {
    if (!g || !key) {
        return -1;
    }
    const auto it = g->kidx.find(key);
    return it == g->kidx.end() ? -1 : it->second;
}

int mi_gguf_get_key(const mi_gguf * g, int64_t idx, const char ** key, int32_t * type) {
    if (!g || !key || !type) {
        return MI_ERR_NULL;
    }
    if (idx < 0 || idx >= (int64_t) g->kv.size()) {
        return MI_ERR_PARAM;
    }
    *key  = g->kv[(size_t) idx].key.c_str();
    *type = (int32_t) g->kv[(size_t) idx].type;
    return MI_OK;
}

// typed getters: MI_ERR_PARAM if the key is absent, MI_ERR_TYPE if it holds another type
int mi_gguf_get_u32(const mi_gguf * g, const char * key, uint32_t * v) {
    const mi_gguf::KV * e = kv_of(g, key);
    if (!v) {
        return MI_ERR_NULL;
    }
    if (!e) {
        return MI_ERR_PARAM;
    }
    if (e->type != GT_U32) {
        return MI_ERR_TYPE;
    }
    memcpy(v, g->map + e->at, 4);
    return MI_OK;
}

int mi_gguf_get_f32(const mi_gguf * g, const char * key, float * v) {
    const mi_gguf::KV * e = kv_of(g, key);
    if (!v) {
        return MI_ERR_NULL;
    }
    if (!e) {
        return MI_ERR_PARAM;
    }
    if (e->type != GT_F32) {
        return MI_ERR_TYPE;
    }
    memcpy(v, g->map + e->at, 4);
    return MI_OK;
}

int mi_gguf_get_bool(const mi_gguf * g, const char * key, int * v) {
    const mi_gguf::KV * e = kv_of(g, key);
    if (!v) {
        return MI_ERR_NULL;
    }
    if (!e) {
        return MI_ERR_PARAM;
    }
    if (e->type != GT_BOOL) {
        return MI_ERR_TYPE;
    }
    *v = g->map[e->at] != 0;
    return MI_OK;
}

int mi_gguf_get_str(const mi_gguf * g, const char * key, const char ** v) {
    const mi_gguf::KV * e = kv_of(g, key);
    if (!v) {
        return MI_ERR_NULL;
    }
    if (!e) {
        return MI_ERR_PARAM;
    }
    if (e->type != GT_STR) {
        return MI_ERR_TYPE;
    }
    *v = g->strs[g->kstr.at(g->kidx.at(key))].c_str();
    return MI_OK;
}

int mi_gguf_upload(const mi_gguf * g, const char * name, int to_f32, void * dst, size_t dst_bytes,
                   mi_stream stream) {
    if (!g || !name) {
        return MI_ERR_NULL;
    }
    const mi_gguf::TI * t = ti_of(g, name);
    if (!t) {
        return MI_ERR_PARAM;
    }
    const uint8_t * src = g->map + g->data_offset + t->offset;
    hipStream_t     s   = (hipStream_t) stream;
    if (!to_f32 || t->type == 0) {
        if (t->nbytes > 0 && (!dst || dst_bytes < t->nbytes)) {
            return MI_ERR_PARAM;
        }
        return copy_to_device(dst, src, t->nbytes, s);
    }
    if (t->type != 1 && t->type != 30) {
        return MI_ERR_TYPE;  // F32 widening is for F16 and BF16 sources
    }
    const size_t n = t->nbytes / 2;
    if (n > 0 && (!dst || dst_bytes < n * 4)) {
        return MI_ERR_PARAM;
    }
    std::vector<float> buf(n);
    for (size_t i = 0; i < n; ++i) {
        uint16_t h;
        memcpy(&h, src + 2 * i, 2);
        if (t->type == 30) {
            const uint32_t u = (uint32_t) h << 16;
            memcpy(&buf[i], &u, 4);
        } else {
            buf[i] = h2f(h);
        }
    }
    return copy_to_device(dst, buf.data(), n * 4, s);
}

int mi_gguf_upload_rows(const mi_gguf * g, const char * const * names, int n, void * dst, size_t dst_bytes,
                        int64_t * ne1_out, mi_stream stream) {
    if (!g || !names) {
        return MI_ERR_NULL;
    }
    if (n < 1) {
        return MI_ERR_PARAM;
    }
    std::vector<const mi_gguf::TI *> ts((size_t) n);
    size_t                           total = 0;
    int64_t                          ne1   = 0;
    for (int i = 0; i < n; ++i) {
        ts[(size_t) i] = ti_of(g, names[i]);
        if (!ts[(size_t) i]) {
            return MI_ERR_PARAM;
        }
        const auto & t = *ts[(size_t) i];
        if (t.n_dims > 2) {
            return MI_ERR_SHAPE;
        }
        if (t.ne[0] != ts[0]->ne[0]) {
            return MI_ERR_SHAPE;
        }
        if (t.type != ts[0]->type) {
            return MI_ERR_UNSUPPORTED;  // the reference then loads the projections separately
        }
        total += t.nbytes;
        ne1 += t.ne[1];
    }
    if (total > 0 && (!dst || dst_bytes < total)) {
        return MI_ERR_PARAM;
    }
    size_t at = 0;
    for (int i = 0; i < n; ++i) {
        const auto & t  = *ts[(size_t) i];
        const int    rc = copy_to_device((char *) dst + at, g->map + g->data_offset + t.offset, t.nbytes,
                                         (hipStream_t) stream);
        if (rc != MI_OK) {
            return rc;
        }
        at += t.nbytes;
    }
    if (ne1_out) {
        *ne1_out = ne1;
    }
    return MI_OK;
}

}  // extern "C"
