// abi.cpp -- the extern "C" entry points declared in include/mi_ops.h.
//
// Every entry validates its descriptors on the host (types, shapes, strides,
// alignment, scalar parameters) with the shape rules of the ggml op it
// replaces, returns a negative mi_status instead of asserting, and only then
// launches on the caller's stream. Nothing here allocates or synchronizes.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <mutex>
#include <vector>

#include "launch.h"

namespace mi {

int num_cus() {
    static std::atomic<int> cache[64];
    int                     dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        return 256;
    }
    int v = cache[dev].load(std::memory_order_relaxed);
    if (v == 0) {
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) {
            v = 256;
        }
        cache[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

namespace {
thread_local bool t_dry_run = false;
}

bool dry_run() {
    return t_dry_run;
}

void set_dry_run(bool on) {
    t_dry_run = on;
}

}  // namespace mi

using namespace mi;

namespace {

constexpr int64_t kMaxRows = (int64_t) 1 << 31;

// Common descriptor checks. `inner` requires nb[0] == element (block) size.
int check(const mi_tensor * t, bool inner = true) {
    if (!t) {
        return MI_ERR_NULL;
    }
    if (t->reserved != 0) {
        return MI_ERR_PARAM;
    }
    const int es = type_size(t->type);
    if (es == 0) {
        return MI_ERR_TYPE;
    }
    for (int d = 0; d < 4; ++d) {
        if (t->ne[d] < 0) {
            return MI_ERR_SHAPE;
        }
    }
    if (t->type == MI_TYPE_Q8_0 && t->ne[0] % 32 != 0) {
        return MI_ERR_SHAPE;
    }
    // the row count, element count and byte extent must each fit in int64:
    // nrows() / nelements() and the launchers multiply the ne[] unchecked
    int64_t rows = 1, elems = 0;
    if (__builtin_mul_overflow(t->ne[1], t->ne[2], &rows) || __builtin_mul_overflow(rows, t->ne[3], &rows) ||
        __builtin_mul_overflow(rows, t->ne[0], &elems)) {
        return MI_ERR_UNSUPPORTED;
    }
    if (elems > 0) {
        // last addressed byte: sum of (ne[d] - 1) * nb[d] plus one element
        uint64_t ext = (uint64_t) es;
        for (int d = 0; d < 4; ++d) {
            const uint64_t n = (uint64_t) (d == 0 ? t->ne[0] / blck_size(t->type) : t->ne[d]) - 1;
            uint64_t       part = 0;
            if (__builtin_mul_overflow(n, t->nb[d], &part) || __builtin_add_overflow(ext, part, &ext)) {
                return MI_ERR_UNSUPPORTED;
            }
        }
        if (ext > (uint64_t) INT64_MAX) {
            return MI_ERR_UNSUPPORTED;
        }
    }
    if (nelements(*t) > 0 && !t->data) {
        return MI_ERR_NULL;
    }
    const size_t al = t->type == MI_TYPE_Q8_0 ? 2 : (size_t) es;
    if (!aligned(t->data, al)) {
        return MI_ERR_ALIGN;
    }
    if (inner && t->ne[0] > 1 && t->nb[0] != (uint64_t) es) {
        return MI_ERR_STRIDE;
    }
    for (int d = 1; d < 4; ++d) {
        if (t->nb[d] % al != 0) {
            return MI_ERR_ALIGN;
        }
    }
    if (t->ne[0] >= kMaxRows || nrows(*t) >= kMaxRows) {
        return MI_ERR_UNSUPPORTED;
    }
    return MI_OK;
}

int check_act(const mi_tensor * t) {
    const int rc = check(t);
    if (rc != MI_OK) {
        return rc;
    }
    return is_act(t->type) ? MI_OK : MI_ERR_TYPE;
}

// F32 [n] vector (a contiguous ggml 1-D tensor, or [n,1,1,1] view)
int check_vec(const mi_tensor * v, int64_t n) {
    const int rc = check(v);
    if (rc != MI_OK) {
        return rc;
    }
    if (v->type != MI_TYPE_F32) {
        return MI_ERR_TYPE;
    }
    if (v->ne[0] != n || v->ne[1] != 1 || v->ne[2] != 1 || v->ne[3] != 1) {
        return MI_ERR_SHAPE;
    }
    return MI_OK;
}

// rows uniformly strided by nb[1] (ggml_is_contiguous_1 style flattening)
bool uniform_rows(const mi_tensor & t) {
    return (t.ne[2] <= 1 || t.nb[2] == t.nb[1] * (uint64_t) t.ne[1]) &&
           (t.ne[3] <= 1 || t.nb[3] == t.nb[2] * (uint64_t) t.ne[2]);
}

bool can_repeat(const mi_tensor & b, const mi_tensor & a) {
    for (int d = 0; d < 4; ++d) {
        if (b.ne[d] == 0 || a.ne[d] % b.ne[d] != 0) {
            return false;
        }
    }
    return true;
}

int finish(int rc) {
    if (rc != MI_OK || dry_run()) {
        return rc;  // a validate-only call leaves the HIP error state alone
    }
    return hipGetLastError() == hipSuccess ? MI_OK : MI_ERR_HIP;
}

#define MI_TRY(expr)              \
    do {                          \
        const int _rc = (expr);   \
        if (_rc != MI_OK) {       \
            return _rc;           \
        }                         \
    } while (0)

HeadSeg make_seg(const mi_tensor & x, const mi_tensor & y, const mi_tensor * w) {
    HeadSeg s;
    s.x     = (const char *) x.data;
    s.y     = (char *) y.data;
    s.heads = (uint32_t) x.ne[1];
    s.xs1   = (int64_t) x.nb[1];
    s.xs2   = (int64_t) x.nb[2];
    s.xs3   = (int64_t) x.nb[3];
    s.ys1   = (int64_t) y.nb[1];
    s.ys2   = (int64_t) y.nb[2];
    s.ys3   = (int64_t) y.nb[3];
    s.w     = w ? (const float *) w->data : nullptr;
    return s;
}

int binary_entry(int op, const mi_tensor * a, const mi_tensor * b, bool clamp, float lo, float hi,
                 const mi_tensor * y, mi_stream stream) {
    MI_TRY(check_act(a));
    MI_TRY(check_act(y));
    if (!same_shape(*a, *y)) {
        return MI_ERR_SHAPE;
    }
    hipStream_t s = (hipStream_t) stream;
    if (!b) {
        return finish(launch_binary(op, *a, nullptr, nullptr, nullptr, clamp, lo, hi, *y, s));
    }
    MI_TRY(check_act(b));
    if (same_shape(*a, *b)) {
        return finish(launch_binary(op, *a, b, nullptr, nullptr, clamp, lo, hi, *y, s));
    }
    if (check_vec(b, a->ne[0]) == MI_OK) {
        return finish(launch_binary(op, *a, nullptr, (const float *) b->data, nullptr, clamp, lo, hi, *y, s));
    }
    if (!can_repeat(*b, *a)) {
        return MI_ERR_SHAPE;
    }
    return finish(launch_binary_bcast(op, *a, *b, clamp, lo, hi, *y, s));
}

}  // namespace

extern "C" {

int mi_abi_version(void) {
    return MI_OPS_ABI_VERSION;
}

const char * mi_status_str(int status) {
    switch (status) {
        case MI_OK:
            return "ok";
        case MI_ERR_NULL:
            return "null tensor or data pointer";
        case MI_ERR_TYPE:
            return "unsupported type";
        case MI_ERR_SHAPE:
            return "inconsistent shapes";
        case MI_ERR_STRIDE:
            return "unsupported stride";
        case MI_ERR_ALIGN:
            return "misaligned pointer or stride";
        case MI_ERR_PARAM:
            return "invalid parameter";
        case MI_ERR_UNSUPPORTED:
            return "unsupported configuration";
        case MI_ERR_HIP:
            return "HIP runtime error";
        case MI_ERR_FILE:
            return "file missing, unreadable, truncated or not GGUF";
        case MI_ERR_SCRATCH:
            return "needs more scratch than the library's static buffer holds";
        default:
            return "unknown status";
    }
}

int mi_rms_norm(const mi_tensor * x, const mi_tensor * w, float eps, const mi_tensor * y, mi_stream stream) {
    MI_TRY(check_act(x));
    MI_TRY(check_act(y));
    if (!same_shape(*x, *y)) {
        return MI_ERR_SHAPE;
    }
    if (w) {
        MI_TRY(check_vec(w, x->ne[0]));
    }
    if (!(eps >= 0.0f) || std::isinf(eps)) {
        return MI_ERR_PARAM;
    }
    hipStream_t s = (hipStream_t) stream;
    if (x->ne[0] == 64 || x->ne[0] == 128 || x->ne[0] == 256) {
        // head-sized rows: whole rows per lane group when the view allows it,
        // else the per-head kernel's sub-wave groups
        const int rc = launch_rms_norm_short(*x, w ? (const float *) w->data : nullptr, eps, *y, s);
        if (rc != MI_ERR_UNSUPPORTED) {
            return finish(rc);
        }
        HeadArgs a;
        a.seg[0] = make_seg(*x, *y, w);
        a.nseg   = 1;
        a.ntok   = (uint32_t) (x->ne[2] * x->ne[3]);
        a.ne2    = (uint32_t) x->ne[2];
        a.pos    = nullptr;
        a.theta_scale = a.freq_scale = a.mscale = 1.0f;
        a.eps    = eps;
        a.ne0    = (int) x->ne[0];
        a.n_dims = (int) x->ne[0];
        a.norm   = 1;
        if (x->ne[1] * x->ne[2] * x->ne[3] >= kMaxRows || x->ne[1] * 4 >= kMaxRows) {
            return MI_ERR_UNSUPPORTED;
        }
        return finish(launch_heads(a, x->type, y->type, s));
    }
    return finish(launch_rms_norm(*x, w ? (const float *) w->data : nullptr, nullptr, nullptr, eps, *y, s));
}

int mi_rms_norm_modulate(const mi_tensor * x, const mi_tensor * w, const mi_tensor * scale, const mi_tensor * shift,
                         float eps, const mi_tensor * y, mi_stream stream) {
    MI_TRY(check_act(x));
    MI_TRY(check_act(y));
    if (!same_shape(*x, *y)) {
        return MI_ERR_SHAPE;
    }
    MI_TRY(check_vec(w, x->ne[0]));
    MI_TRY(check_vec(scale, x->ne[0]));
    MI_TRY(check_vec(shift, x->ne[0]));
    if (!(eps >= 0.0f) || std::isinf(eps)) {
        return MI_ERR_PARAM;
    }
    return finish(launch_rms_norm(*x, (const float *) w->data, (const float *) scale->data,
                                  (const float *) shift->data, eps, *y, (hipStream_t) stream));
}

int mi_add_rms_norm(const mi_tensor * residual, const mi_tensor * x, const mi_tensor * gate, int clamp, float lo,
                    float hi, const mi_tensor * w, const mi_tensor * scale, const mi_tensor * shift, float eps,
                    const mi_tensor * y_sum, const mi_tensor * y_norm, mi_stream stream) {
    MI_TRY(check_act(residual));
    MI_TRY(check_act(x));
    MI_TRY(check_act(y_sum));
    MI_TRY(check_act(y_norm));
    if (!same_shape(*residual, *x) || !same_shape(*residual, *y_sum) || !same_shape(*residual, *y_norm)) {
        return MI_ERR_SHAPE;
    }
    if (x->type != residual->type || y_sum->type != residual->type || y_norm->type != residual->type) {
        return MI_ERR_TYPE;
    }
    const int64_t n = residual->ne[0];
    if (gate) {
        MI_TRY(check_vec(gate, n));
    }
    if (w) {
        MI_TRY(check_vec(w, n));
    }
    if ((scale == nullptr) != (shift == nullptr) || (scale && !w)) {
        return MI_ERR_NULL;
    }
    if (scale) {
        MI_TRY(check_vec(scale, n));
        MI_TRY(check_vec(shift, n));
    }
    if (!(eps >= 0.0f) || std::isinf(eps) || (clamp && (std::isnan(lo) || std::isnan(hi)))) {
        return MI_ERR_PARAM;
    }
    if (y_norm->data == residual->data || y_norm->data == x->data || y_norm->data == y_sum->data) {
        return MI_ERR_PARAM;  // y_norm must not alias an input or y_sum
    }
    AddNorm add;
    add.x2    = x;
    add.gate  = gate ? (const float *) gate->data : nullptr;
    add.clamp = clamp ? 1 : 0;
    add.lo    = lo;
    add.hi    = hi;
    add.ysum  = y_sum;
    return finish(launch_rms_norm(*residual, w ? (const float *) w->data : nullptr,
                                  scale ? (const float *) scale->data : nullptr,
                                  shift ? (const float *) shift->data : nullptr, eps, *y_norm, (hipStream_t) stream,
                                  &add));
}

static int rope_common(const mi_tensor * q, const mi_tensor * q_w, const mi_tensor * q_out, const mi_tensor * k,
                       const mi_tensor * k_w, const mi_tensor * k_out, const mi_tensor * pos, float eps, int n_dims,
                       float freq_base, float freq_scale, float attn_factor, bool norm, bool rope,
                       mi_stream stream) {
    MI_TRY(check_act(q));
    MI_TRY(check_act(q_out));
    if (!same_shape(*q, *q_out)) {
        return MI_ERR_SHAPE;
    }
    if ((k == nullptr) != (k_out == nullptr)) {
        return MI_ERR_NULL;
    }
    if (k) {
        MI_TRY(check_act(k));
        MI_TRY(check_act(k_out));
        if (!same_shape(*k, *k_out) || k->ne[0] != q->ne[0] || k->ne[2] != q->ne[2] || k->ne[3] != q->ne[3]) {
            return MI_ERR_SHAPE;
        }
        if (k->type != q->type || k_out->type != q_out->type) {
            return MI_ERR_TYPE;  // one launch serves both: same in/out types
        }
    }
    const int64_t D = q->ne[0];
    if (norm) {
        if (q_w) {
            MI_TRY(check_vec(q_w, D));
        }
        if (k && k_w) {
            MI_TRY(check_vec(k_w, D));
        }
        if (!(eps >= 0.0f) || std::isinf(eps)) {
            return MI_ERR_PARAM;
        }
    }
    if (rope) {
        MI_TRY(check(pos));
        if (pos->type != MI_TYPE_I32) {
            return MI_ERR_TYPE;
        }
        if (pos->ne[0] != q->ne[2] || pos->ne[1] != 1 || pos->ne[2] != 1 || pos->ne[3] != 1) {
            return MI_ERR_SHAPE;
        }
        if (n_dims <= 0 || n_dims % 2 != 0 || n_dims > D) {
            return MI_ERR_PARAM;
        }
        if (!(freq_base > 0.0f) || !std::isfinite(freq_scale) || !std::isfinite(attn_factor)) {
            return MI_ERR_PARAM;
        }
    }
    if (q->ne[2] * q->ne[3] >= kMaxRows || q->ne[1] * 256 >= kMaxRows || (k && k->ne[1] * 256 >= kMaxRows)) {
        return MI_ERR_UNSUPPORTED;
    }
    HeadArgs a;
    a.seg[0] = make_seg(*q, *q_out, norm ? q_w : nullptr);
    a.nseg   = 1;
    if (k) {
        a.seg[1] = make_seg(*k, *k_out, norm ? k_w : nullptr);
        a.nseg   = 2;
    }
    a.ntok        = (uint32_t) (q->ne[2] * q->ne[3]);
    a.ne2         = (uint32_t) q->ne[2];
    a.pos         = rope ? (const int32_t *) pos->data : nullptr;
    // ggml-cpu derives theta_scale on the host CPU with libm powf
    a.theta_scale = rope ? powf(freq_base, -2.0f / (float) n_dims) : 1.0f;
    a.freq_scale  = freq_scale;
    a.mscale      = attn_factor;
    a.eps         = eps;
    a.ne0         = (int) D;
    a.n_dims      = rope ? n_dims : (int) D;
    a.norm        = norm ? 1 : 0;
    return finish(launch_heads(a, q->type, q_out->type, (hipStream_t) stream));
}

int mi_rope_ext(const mi_tensor * x, const mi_tensor * pos, int n_dims, int mode, float freq_base, float freq_scale,
                float ext_factor, float attn_factor, const mi_tensor * y, mi_stream stream) {
    if (mode != 2 || ext_factor != 0.0f) {
        return MI_ERR_UNSUPPORTED;
    }
    return rope_common(x, nullptr, y, nullptr, nullptr, nullptr, pos, 0.0f, n_dims, freq_base, freq_scale,
                       attn_factor, false, true, stream);
}

int mi_qk_norm_rope(const mi_tensor * q, const mi_tensor * q_w, const mi_tensor * q_out, const mi_tensor * k,
                    const mi_tensor * k_w, const mi_tensor * k_out, const mi_tensor * pos, float eps, int n_dims,
                    float freq_base, float freq_scale, float attn_factor, mi_stream stream) {
    const bool norm = q_w != nullptr;
    if (k && ((k_w != nullptr) != norm)) {
        return MI_ERR_PARAM;
    }
    return rope_common(q, q_w, q_out, k, k_w, k_out, pos, eps, n_dims, freq_base, freq_scale, attn_factor, norm,
                       true, stream);
}

static int swiglu_common(const mi_tensor * g, const mi_tensor * u, const char * gp, const char * up, int64_t n,
                         const mi_tensor * y, mi_stream stream) {
    MI_TRY(check_act(y));
    if (y->ne[0] != n || y->ne[1] != g->ne[1] || y->ne[2] != g->ne[2] || y->ne[3] != g->ne[3]) {
        return MI_ERR_SHAPE;
    }
    if (!uniform_rows(*g) || !uniform_rows(*u) || !uniform_rows(*y)) {
        return MI_ERR_STRIDE;
    }
    const int64_t rows = nrows(*g);
    return finish(launch_swiglu(gp, up, (int64_t) g->nb[1], (int64_t) u->nb[1], g->type, (char *) y->data,
                                (int64_t) y->nb[1], y->type, rows, n, true, (hipStream_t) stream));
}

int mi_swiglu(const mi_tensor * gu, int swapped, const mi_tensor * y, mi_stream stream) {
    MI_TRY(check_act(gu));
    if (gu->ne[0] % 2 != 0) {
        return MI_ERR_SHAPE;
    }
    const int64_t n  = gu->ne[0] / 2;
    const size_t  hb = (size_t) n * type_size(gu->type);
    const char *  b  = (const char *) gu->data;
    return swiglu_common(gu, gu, swapped ? b + hb : b, swapped ? b : b + hb, n, y, stream);
}

int mi_swiglu_split(const mi_tensor * g, const mi_tensor * u, const mi_tensor * y, mi_stream stream) {
    MI_TRY(check_act(g));
    MI_TRY(check_act(u));
    if (!same_shape(*g, *u)) {
        return MI_ERR_SHAPE;
    }
    if (g->type != u->type) {
        return MI_ERR_TYPE;
    }
    return swiglu_common(g, u, (const char *) g->data, (const char *) u->data, g->ne[0], y, stream);
}

int mi_add(const mi_tensor * a, const mi_tensor * b, const mi_tensor * y, mi_stream stream) {
    if (!b) {
        return MI_ERR_NULL;
    }
    return binary_entry(OP_ADD, a, b, false, 0.0f, 0.0f, y, stream);
}

int mi_mul(const mi_tensor * a, const mi_tensor * b, const mi_tensor * y, mi_stream stream) {
    if (!b) {
        return MI_ERR_NULL;
    }
    return binary_entry(OP_MUL, a, b, false, 0.0f, 0.0f, y, stream);
}

int mi_add_clamp(const mi_tensor * a, const mi_tensor * b, float lo, float hi, const mi_tensor * y,
                 mi_stream stream) {
    if (std::isnan(lo) || std::isnan(hi)) {
        return MI_ERR_PARAM;
    }
    return binary_entry(b ? OP_ADD : OP_NONE, a, b, true, lo, hi, y, stream);
}

int mi_gated_add(const mi_tensor * residual, const mi_tensor * x, const mi_tensor * gate, const mi_tensor * y,
                 mi_stream stream) {
    MI_TRY(check_act(residual));
    MI_TRY(check_act(x));
    MI_TRY(check_act(y));
    if (!same_shape(*residual, *x) || !same_shape(*residual, *y)) {
        return MI_ERR_SHAPE;
    }
    MI_TRY(check_vec(gate, residual->ne[0]));
    return finish(launch_binary(OP_GATED, *residual, x, (const float *) gate->data, nullptr, false, 0.0f, 0.0f, *y,
                                (hipStream_t) stream));
}

int mi_modulate(const mi_tensor * x, const mi_tensor * scale, const mi_tensor * shift, const mi_tensor * y,
                mi_stream stream) {
    MI_TRY(check_act(x));
    MI_TRY(check_act(y));
    if (!same_shape(*x, *y)) {
        return MI_ERR_SHAPE;
    }
    MI_TRY(check_vec(scale, x->ne[0]));
    MI_TRY(check_vec(shift, x->ne[0]));
    return finish(launch_binary(OP_MOD, *x, nullptr, (const float *) scale->data, (const float *) shift->data, false,
                                0.0f, 0.0f, *y, (hipStream_t) stream));
}

int mi_get_rows(const mi_tensor * table, const mi_tensor * ids, const mi_tensor * y, int32_t * d_err,
                mi_stream stream) {
    MI_TRY(check(table));
    MI_TRY(check(ids, false));
    MI_TRY(check(y));
    if (table->type != MI_TYPE_Q8_0 && !is_act(table->type)) {
        return MI_ERR_TYPE;
    }
    if (ids->type != MI_TYPE_I32 || (y->type != MI_TYPE_F32 && y->type != MI_TYPE_BF16)) {
        return MI_ERR_TYPE;
    }
    if (table->ne[2] != 1 || table->ne[3] != 1 || ids->ne[1] != 1 || ids->ne[2] != 1 || ids->ne[3] != 1) {
        return MI_ERR_UNSUPPORTED;  // batched tables (ne02/ne03 > 1) are not used by the reference
    }
    if (y->ne[0] != table->ne[0] || y->ne[1] != ids->ne[0] || y->ne[2] != 1 || y->ne[3] != 1) {
        return MI_ERR_SHAPE;
    }
    if (!aligned(d_err, 4) || ids->nb[0] % 4 != 0) {
        return MI_ERR_ALIGN;
    }
    const int64_t ids_stride = ids->ne[0] > 1 ? (int64_t) (ids->nb[0] / 4) : 1;
    return finish(launch_get_rows(*table, (const int32_t *) ids->data, ids->ne[0], ids_stride, *y, d_err,
                                  (hipStream_t) stream));
}

static RowCopy plain_copy(const mi_tensor & src, const mi_tensor & dst) {
    RowCopy r{};
    r.src  = (const char *) src.data;
    r.sr   = make_rows3(src);
    r.rows = (uint32_t) nrows(src);
    r.ne0  = (int) src.ne[0];
    r.dst  = (char *) dst.data;
    r.dr   = make_rows3(dst);
    r.kv   = 0;
    return r;
}

int mi_cpy_q8_0(const mi_tensor * src, const mi_tensor * dst, int rounding, mi_stream stream) {
    MI_TRY(check_act(src));
    MI_TRY(check(dst));
    if (dst->type != MI_TYPE_Q8_0 && !is_act(dst->type)) {
        return MI_ERR_TYPE;
    }
    if (!same_shape(*src, *dst)) {
        return MI_ERR_SHAPE;
    }
    if (rounding != MI_Q8_0_CPU_X86 && rounding != MI_Q8_0_REF) {
        return MI_ERR_PARAM;
    }
    const RowCopy k = plain_copy(*src, *dst);
    return finish(launch_row_copy(k, nullptr, src->type, dst->type, rounding, (hipStream_t) stream));
}

int mi_cpy(const mi_tensor * src, const mi_tensor * dst, mi_stream stream) {
    return mi_cpy_q8_0(src, dst, MI_Q8_0_CPU_X86, stream);
}

static int kv_desc(const mi_tensor * x, const mi_tensor * cache, const mi_tensor * pos0, const mi_tensor * sets,
                   int32_t * d_err, RowCopy & r) {
    MI_TRY(check_act(x));
    MI_TRY(check(cache));
    if (cache->type != MI_TYPE_Q8_0 && !is_act(cache->type)) {
        return MI_ERR_TYPE;
    }
    if (cache->ne[0] != x->ne[0] || cache->ne[2] != x->ne[1]) {
        return MI_ERR_SHAPE;
    }
    r      = RowCopy{};
    r.src  = (const char *) x->data;
    r.sr   = make_rows3(*x);
    r.rows = (uint32_t) nrows(*x);
    r.ne0  = (int) x->ne[0];
    r.dst  = (char *) cache->data;
    r.kv   = 1;
    r.ne1  = (uint32_t) x->ne[1];
    r.ne2  = (uint32_t) x->ne[2];
    r.d1   = FastDiv(r.ne1);
    r.d2   = FastDiv(r.ne2);
    r.pos0 = (const int32_t *) pos0->data;
    r.sets = sets ? (const int32_t *) sets->data : nullptr;
    r.cnb1 = (int64_t) cache->nb[1];
    r.cnb2 = (int64_t) cache->nb[2];
    r.cnb3 = (int64_t) cache->nb[3];
    r.max_seq = cache->ne[1];
    r.n_sets  = cache->ne[3];
    r.d_err   = d_err;
    return MI_OK;
}

int mi_kv_store(const mi_tensor * k, const mi_tensor * k_cache, const mi_tensor * v, const mi_tensor * v_cache,
                const mi_tensor * pos0, const mi_tensor * sets, int rounding, int32_t * d_err, mi_stream stream) {
    if (!k || !k_cache || !pos0) {
        return MI_ERR_NULL;
    }
    if ((v == nullptr) != (v_cache == nullptr)) {
        return MI_ERR_NULL;
    }
    MI_TRY(check(pos0));
    if (pos0->type != MI_TYPE_I32) {
        return MI_ERR_TYPE;
    }
    if (pos0->ne[0] != k->ne[3] || pos0->ne[1] != 1 || pos0->ne[2] != 1 || pos0->ne[3] != 1) {
        return MI_ERR_SHAPE;
    }
    if (sets) {
        MI_TRY(check(sets));
        if (sets->type != MI_TYPE_I32) {
            return MI_ERR_TYPE;
        }
        if (sets->ne[0] != k->ne[3] || sets->ne[1] != 1 || sets->ne[2] != 1 || sets->ne[3] != 1) {
            return MI_ERR_SHAPE;
        }
    }
    if (rounding != MI_Q8_0_CPU_X86 && rounding != MI_Q8_0_REF) {
        return MI_ERR_PARAM;
    }
    if (!aligned(d_err, 4)) {
        return MI_ERR_ALIGN;
    }
    RowCopy rk, rv;
    MI_TRY(kv_desc(k, k_cache, pos0, sets, d_err, rk));
    if (v) {
        MI_TRY(kv_desc(v, v_cache, pos0, sets, d_err, rv));
        if (!same_shape(*k, *v) || !same_shape(*k_cache, *v_cache) || k->type != v->type ||
            k_cache->type != v_cache->type) {
            return MI_ERR_SHAPE;
        }
    }
    return finish(launch_row_copy(rk, v ? &rv : nullptr, k->type, k_cache->type, rounding, (hipStream_t) stream));
}

int mi_qk_norm_rope_kv_store(const mi_tensor * q, const mi_tensor * q_w, const mi_tensor * q_out, const mi_tensor * k,
                             const mi_tensor * k_w, const mi_tensor * v, const mi_tensor * pos, float eps, int n_dims,
                             float freq_base, float freq_scale, float attn_factor, int clamp_v,
                             const mi_tensor * k_cache, const mi_tensor * v_cache, const mi_tensor * pos0,
                             const mi_tensor * sets, int rounding, int32_t * d_err, mi_stream stream) {
    if (!q || !q_out || !k || !v || !pos || !k_cache || !v_cache || !pos0) {
        return MI_ERR_NULL;
    }
    const bool norm = q_w != nullptr;
    if ((k_w != nullptr) != norm) {
        return MI_ERR_PARAM;
    }
    // Q, K as mi_qk_norm_rope (K's output shape is K's own)
    MI_TRY(check_act(q));
    MI_TRY(check_act(q_out));
    MI_TRY(check_act(k));
    MI_TRY(check_act(v));
    if (!same_shape(*q, *q_out) || k->ne[0] != q->ne[0] || k->ne[2] != q->ne[2] || k->ne[3] != q->ne[3] ||
        !same_shape(*k, *v)) {
        return MI_ERR_SHAPE;
    }
    if (k->type != q->type || v->type != q->type || q_out->type != q->type) {
        return MI_ERR_TYPE;
    }
    const int64_t D = q->ne[0];
    if (norm) {
        MI_TRY(check_vec(q_w, D));
        MI_TRY(check_vec(k_w, D));
        if (!(eps >= 0.0f) || std::isinf(eps)) {
            return MI_ERR_PARAM;
        }
    }
    MI_TRY(check(pos));
    if (pos->type != MI_TYPE_I32) {
        return MI_ERR_TYPE;
    }
    if (pos->ne[0] != q->ne[2] || pos->ne[1] != 1 || pos->ne[2] != 1 || pos->ne[3] != 1) {
        return MI_ERR_SHAPE;
    }
    if (n_dims <= 0 || n_dims % 2 != 0 || n_dims > D) {
        return MI_ERR_PARAM;
    }
    if (!(freq_base > 0.0f) || !std::isfinite(freq_scale) || !std::isfinite(attn_factor)) {
        return MI_ERR_PARAM;
    }
    if (q->ne[2] * q->ne[3] >= kMaxRows || q->ne[1] * 256 >= kMaxRows || k->ne[1] * 256 >= kMaxRows) {
        return MI_ERR_UNSUPPORTED;
    }
    // the caches and the sequences as mi_kv_store: token t of the flat
    // [ne2 * ne3] order belongs to sequence t / T, T = tokens / B
    MI_TRY(check(k_cache));
    MI_TRY(check(v_cache));
    if (k_cache->type != MI_TYPE_Q8_0 && !is_act(k_cache->type)) {
        return MI_ERR_TYPE;
    }
    if (!same_shape(*k_cache, *v_cache) || k_cache->type != v_cache->type || k_cache->nb[1] != v_cache->nb[1] ||
        k_cache->nb[2] != v_cache->nb[2] || k_cache->nb[3] != v_cache->nb[3]) {
        return MI_ERR_SHAPE;
    }
    if (k_cache->ne[0] != D || k_cache->ne[2] != k->ne[1]) {
        return MI_ERR_SHAPE;
    }
    MI_TRY(check(pos0));
    if (pos0->type != MI_TYPE_I32) {
        return MI_ERR_TYPE;
    }
    const int64_t n_tok = q->ne[2] * q->ne[3];
    const int64_t B     = pos0->ne[0];
    if (pos0->ne[1] != 1 || pos0->ne[2] != 1 || pos0->ne[3] != 1 || B <= 0 || n_tok % B != 0) {
        return MI_ERR_SHAPE;
    }
    if (sets) {
        MI_TRY(check(sets));
        if (sets->type != MI_TYPE_I32) {
            return MI_ERR_TYPE;
        }
        if (sets->ne[0] != B || sets->ne[1] != 1 || sets->ne[2] != 1 || sets->ne[3] != 1) {
            return MI_ERR_SHAPE;
        }
    }
    if (rounding != MI_Q8_0_CPU_X86 && rounding != MI_Q8_0_REF) {
        return MI_ERR_PARAM;
    }
    if (!aligned(d_err, 4)) {
        return MI_ERR_ALIGN;
    }
    HeadArgs a;
    a.seg[0]      = make_seg(*q, *q_out, norm ? q_w : nullptr);
    a.seg[1]      = make_seg(*k, *k, norm ? k_w : nullptr);  // K's destination is the cache
    a.nseg        = 2;
    a.ntok        = (uint32_t) n_tok;
    a.ne2         = (uint32_t) q->ne[2];
    a.pos         = (const int32_t *) pos->data;
    a.theta_scale = powf(freq_base, -2.0f / (float) n_dims);  // the host libm powf, as ggml-cpu
    a.freq_scale  = freq_scale;
    a.mscale      = attn_factor;
    a.eps         = eps;
    a.ne0         = (int) D;
    a.n_dims      = n_dims;
    a.norm        = norm ? 1 : 0;
    HeadKV kv;
    kv.v       = (const char *) v->data;
    kv.vs1     = (int64_t) v->nb[1];
    kv.vs2     = (int64_t) v->nb[2];
    kv.vs3     = (int64_t) v->nb[3];
    kv.kc      = (char *) k_cache->data;
    kv.vc      = (char *) v_cache->data;
    kv.cnb1    = (int64_t) k_cache->nb[1];
    kv.cnb2    = (int64_t) k_cache->nb[2];
    kv.cnb3    = (int64_t) k_cache->nb[3];
    kv.max_seq = k_cache->ne[1];
    kv.n_sets  = k_cache->ne[3];
    kv.pos0    = (const int32_t *) pos0->data;
    kv.sets    = sets ? (const int32_t *) sets->data : nullptr;
    kv.T       = (uint32_t) (n_tok / B);
    kv.dT      = FastDiv(kv.T);
    kv.clamp_v = clamp_v != 0;
    kv.d_err   = d_err;
    return finish(launch_heads_kv(a, kv, q->type, k_cache->type, rounding, (hipStream_t) stream));
}

// ggml_flash_attn_ext shape rules; fills the launcher's descriptor (without data pointers' workspace)
static int fa_desc(const mi_tensor * q, const mi_tensor * k, const mi_tensor * v, const mi_tensor * mask,
                   const mi_tensor * y, FaArgs & a) {
    MI_TRY(check(q));
    MI_TRY(check(k));
    MI_TRY(check(v));
    if (!is_act(q->type)) {
        return MI_ERR_TYPE;
    }
    const int kt = k->type;
    if (kt != v->type || (kt != MI_TYPE_F16 && kt != MI_TYPE_BF16 && kt != MI_TYPE_Q8_0 && kt != MI_TYPE_F32)) {
        return MI_ERR_TYPE;
    }
    const int64_t D = q->ne[0];
    if (k->ne[0] != D || v->ne[0] != D || k->ne[1] != v->ne[1] || k->ne[2] != v->ne[2] || k->ne[3] != v->ne[3]) {
        return MI_ERR_SHAPE;
    }
    if (k->ne[2] == 0 || k->ne[3] == 0 || q->ne[2] % k->ne[2] != 0 || q->ne[3] % k->ne[3] != 0) {
        return MI_ERR_SHAPE;
    }
    if (D != 64 && D != 128 && D != 256) {
        return MI_ERR_UNSUPPORTED;
    }
    if (kt == MI_TYPE_F32 && D > 128) {
        return MI_ERR_UNSUPPORTED;
    }
    // K/V rows are read in 16-byte chunks (Q8_0, 34-byte blocks: 8-byte when D is a
    // multiple of 128, else 4-byte)
    const size_t cb = kt == MI_TYPE_Q8_0 ? (D % 128 == 0 ? 8 : 4) : 16;
    for (const mi_tensor * t : { k, v }) {
        if (!aligned(t->data, cb) || t->nb[1] % cb != 0 || t->nb[2] % cb != 0 || t->nb[3] % cb != 0) {
            return MI_ERR_ALIGN;
        }
    }
    if (q->nb[1] % type_size(q->type) != 0 || q->nb[2] % type_size(q->type) != 0) {
        return MI_ERR_ALIGN;
    }
    a      = FaArgs{};
    a.q    = (const char *) q->data;
    a.q1   = (int64_t) q->nb[1];
    a.q2   = (int64_t) q->nb[2];
    a.q3   = (int64_t) q->nb[3];
    a.tq   = q->type;
    a.qvec = aligned(q->data, 16) && q->nb[1] % 16 == 0 && q->nb[2] % 16 == 0 && q->nb[3] % 16 == 0;
    a.k    = (const char *) k->data;
    a.k1   = (int64_t) k->nb[1];
    a.k2   = (int64_t) k->nb[2];
    a.k3   = (int64_t) k->nb[3];
    a.v    = (const char *) v->data;
    a.v1   = (int64_t) v->nb[1];
    a.v2   = (int64_t) v->nb[2];
    a.v3   = (int64_t) v->nb[3];
    a.n_q  = (int) q->ne[1];
    a.n_kv = (int) k->ne[1];
    a.nh   = (int) q->ne[2];
    a.nkv  = (int) k->ne[2];
    a.nb   = (int) q->ne[3];
    a.rk   = (int) (q->ne[2] / k->ne[2]);
    a.rk3  = (int) (q->ne[3] / k->ne[3]);
    a.kt   = kt;
    if (mask) {
        MI_TRY(check(mask));
        if (mask->type != MI_TYPE_F16) {
            return MI_ERR_TYPE;
        }
        if (mask->ne[0] != k->ne[1] || mask->ne[1] < q->ne[1] || mask->ne[2] == 0 || mask->ne[3] == 0 ||
            q->ne[2] % mask->ne[2] != 0 || q->ne[3] % mask->ne[3] != 0) {
            return MI_ERR_SHAPE;
        }
        a.mask = (const char *) mask->data;
        a.m1   = (int64_t) mask->nb[1];
        a.m2   = (int64_t) mask->nb[2];
        a.m3   = (int64_t) mask->nb[3];
        a.mne2 = (int) mask->ne[2];
        a.mne3 = (int) mask->ne[3];
        a.mvec = aligned(mask->data, 8) && a.m1 % 8 == 0 && a.m2 % 8 == 0 && a.m3 % 8 == 0;
    } else {
        a.mne2 = 1;
        a.mne3 = 1;
    }
    if (y) {
        MI_TRY(check(y));
        if (y->type != MI_TYPE_F32) {
            return MI_ERR_TYPE;
        }
        if (y->ne[0] != D || y->ne[1] != q->ne[2] || y->ne[2] != q->ne[1] || y->ne[3] != q->ne[3]) {
            return MI_ERR_SHAPE;
        }
        a.y    = (char *) y->data;
        a.y1   = (int64_t) y->nb[1];
        a.y2   = (int64_t) y->nb[2];
        a.y3   = (int64_t) y->nb[3];
        a.yvec = aligned(y->data, 16) && a.y1 % 16 == 0 && a.y2 % 16 == 0 && a.y3 % 16 == 0;
    }
    flash_attn_plan(a, (int) D);
    if (a.splits == 0) {
        return MI_ERR_UNSUPPORTED;  // a key range beyond 1024 splits of 256 keys
    }
    return MI_OK;
}

int mi_flash_attn_ext_workspace(const mi_tensor * q, const mi_tensor * k, const mi_tensor * v, size_t * bytes) {
    if (!bytes) {
        return MI_ERR_NULL;
    }
    FaArgs a;
    MI_TRY(fa_desc(q, k, v, nullptr, nullptr, a));
    *bytes = flash_attn_workspace(a, (int) q->ne[0]);
    return MI_OK;
}

int mi_flash_attn_ext(const mi_tensor * q, const mi_tensor * k, const mi_tensor * v, const mi_tensor * mask,
                      float scale, float max_bias, float logit_softcap, const mi_tensor * y, void * workspace,
                      size_t workspace_bytes, mi_stream stream) {
    if (!y) {
        return MI_ERR_NULL;
    }
    if (max_bias != 0.0f || logit_softcap != 0.0f) {
        return MI_ERR_UNSUPPORTED;
    }
    if (!std::isfinite(scale)) {
        return MI_ERR_PARAM;
    }
    FaArgs a;
    MI_TRY(fa_desc(q, k, v, mask, y, a));
    a.scale         = scale;
    const size_t need = flash_attn_workspace(a, (int) q->ne[0]);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
        return MI_ERR_PARAM;
    }
    if (!aligned(workspace, 16)) {
        return MI_ERR_ALIGN;
    }
    a.ws    = (float *) workspace;
    a.msum  = a.mfma && a.mask ? (uint8_t *) workspace : nullptr;
    a.fpart = a.mfma && a.tsplit > 0 ? (float *) ((char *) workspace + flash_attn_part_offset(a)) : nullptr;
    return finish(launch_flash_attn(a, k->type, (int) q->ne[0], (hipStream_t) stream));
}

int mi_q8_0_repack_bytes(int64_t k, int64_t n, size_t * bytes) {
    if (!bytes) {
        return MI_ERR_NULL;
    }
    if (k <= 0 || k % 32 != 0 || n < 0) {
        return MI_ERR_SHAPE;
    }
    if (k >= kMaxRows || n >= kMaxRows) {
        return MI_ERR_UNSUPPORTED;
    }
    *bytes = (size_t) ((n + 63) / 64) * (size_t) (k / 32) * 2176;
    return MI_OK;
}

int mi_q8_0_repack(const mi_tensor * w, void * dst, size_t dst_bytes, mi_stream stream) {
    MI_TRY(check(w));
    if (w->type != MI_TYPE_Q8_0) {
        return MI_ERR_TYPE;
    }
    if (w->ne[2] != 1 || w->ne[3] != 1) {
        return MI_ERR_SHAPE;
    }
    size_t need = 0;
    MI_TRY(mi_q8_0_repack_bytes(w->ne[0], w->ne[1], &need));
    if (need > 0 && (!dst || dst_bytes < need)) {
        return MI_ERR_PARAM;
    }
    if (!aligned(dst, 16)) {
        return MI_ERR_ALIGN;
    }
    return finish(launch_q8_0_repack((const char *) w->data, (int64_t) w->nb[1], (uint32_t) w->ne[0],
                                     (uint32_t) w->ne[1], (char *) dst, (hipStream_t) stream));
}

// ggml_mul_mat(w, x) operands: w R64 [k, n], x F32 [k, m] (rows folded over ne1..ne3), y F32 [n, m]
static int mm_desc(const void * w, int64_t k, int64_t n, const mi_tensor * x, const mi_tensor * y, MmvArgs & a) {
    size_t wb = 0;
    MI_TRY(mi_q8_0_repack_bytes(k, n, &wb));
    MI_TRY(check(x));
    if (x->type != MI_TYPE_F32) {
        return MI_ERR_TYPE;
    }
    if (x->ne[0] != k || !uniform_rows(*x)) {
        return MI_ERR_SHAPE;
    }
    const int64_t m = nrows(*x);
    (void) wb;
    a        = MmvArgs{};
    a.w      = (const char *) w;
    a.k      = (uint32_t) k;
    a.n      = (uint32_t) n;
    a.nbk    = (uint32_t) (k / 32);
    a.m      = (uint32_t) m;
    a.x      = (const char *) x->data;
    a.x1     = (int64_t) x->nb[1];
    a.xvec   = aligned(x->data, 16) && (m <= 1 || x->nb[1] % 16 == 0);
    if (y) {
        MI_TRY(check(y));
        if (y->type != MI_TYPE_F32) {
            return MI_ERR_TYPE;
        }
        if (y->ne[0] != n || nrows(*y) != m || !uniform_rows(*y)) {
            return MI_ERR_SHAPE;
        }
        a.y  = (char *) y->data;
        a.y1 = (int64_t) y->nb[1];
    }
    mul_mat_q8_0_plan(a, num_cus());
    return MI_OK;
}

int mi_mul_mat_q8_0_workspace(int64_t k, int64_t n, const mi_tensor * x, size_t * bytes) {
    if (!bytes) {
        return MI_ERR_NULL;
    }
    MmvArgs a;
    MI_TRY(mm_desc(nullptr, k, n, x, nullptr, a));
    *bytes = a.m == 0 || a.n == 0 ? 0 : mul_mat_q8_0_workspace(a);
    return MI_OK;
}

int mi_mul_mat_q8_0(const void * w, int64_t k, int64_t n, const mi_tensor * x, const mi_tensor * y,
                    void * workspace, size_t workspace_bytes, mi_stream stream) {
    if (!y) {
        return MI_ERR_NULL;
    }
    MmvArgs a;
    MI_TRY(mm_desc(w, k, n, x, y, a));
    if (a.m == 0 || a.n == 0) {
        return MI_OK;
    }
    if (!w) {
        return MI_ERR_NULL;
    }
    if (!aligned(w, 16)) {
        return MI_ERR_ALIGN;
    }
    if (!workspace || workspace_bytes < mul_mat_q8_0_workspace(a)) {
        return MI_ERR_PARAM;
    }
    if (!aligned(workspace, 256)) {
        return MI_ERR_ALIGN;
    }
    mul_mat_q8_0_bind(a, (char *) workspace);
    return finish(launch_mul_mat_q8_0(a, (hipStream_t) stream));
}

// Scratch of mi_mul_mat_q8_0_noalloc: one static array per GPU, loaded with the
// library's code object. Host code never uses this name as an address (on the
// host it is only a stand-in for the symbol): each device's address comes from
// hipGetSymbolAddress, once per device, with that device current.
static __device__ __align__(256) char scratch[MI_MUL_MAT_NOALLOC_SCRATCH_BYTES];

static int noalloc_scratch(void ** out) {
    constexpr int            MAX_DEV = 64;
    static std::atomic<void *> addr[MAX_DEV];
    static std::mutex          mu;
    int                        dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEV) {
        return MI_ERR_HIP;
    }
    void * p = addr[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(mu);
        p = addr[dev].load(std::memory_order_relaxed);
        if (!p) {
            if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
                (void) hipGetLastError();
                return MI_ERR_HIP;
            }
            addr[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return MI_OK;
}

int mi_mul_mat_q8_0_noalloc(const void * w, int64_t k, int64_t n, const mi_tensor * x, const mi_tensor * y,
                            mi_stream stream) {
    if (!y) {
        return MI_ERR_NULL;
    }
    MmvArgs a;
    MI_TRY(mm_desc(w, k, n, x, y, a));
    if (a.m == 0 || a.n == 0) {
        return MI_OK;
    }
    if (!w) {
        return MI_ERR_NULL;
    }
    if (!aligned(w, 16)) {
        return MI_ERR_ALIGN;
    }
    if (mul_mat_q8_0_workspace(a) > MI_MUL_MAT_NOALLOC_SCRATCH_BYTES) {
        return MI_ERR_SCRATCH;
    }
    void * ws = nullptr;
    MI_TRY(noalloc_scratch(&ws));
    mul_mat_q8_0_bind(a, (char *) ws);
    return finish(launch_mul_mat_q8_0(a, (hipStream_t) stream));
}

// gu F32 [2k, m] -> the descriptor of the SwiGLU input x [k, m] (the gate half's
// view) with g / u pointed at the two halves
static int mm_glu_desc(const void * w, int64_t k, int64_t n, const mi_tensor * gu, int swapped, const mi_tensor * y,
                       MmvArgs & a) {
    if (!gu) {
        return MI_ERR_NULL;
    }
    MI_TRY(check(gu));
    if (gu->type != MI_TYPE_F32) {
        return MI_ERR_TYPE;
    }
    if (k <= 0 || gu->ne[0] != 2 * k) {
        return MI_ERR_SHAPE;
    }
    mi_tensor x = *gu;
    x.ne[0]     = k;
    MI_TRY(mm_desc(w, k, n, &x, y, a));
    const char * lo = (const char *) gu->data;
    const char * hi = lo + k * 4;
    a.glu           = 1;
    a.g             = swapped ? hi : lo;
    a.u             = swapped ? lo : hi;
    a.gu1           = (int64_t) gu->nb[1];
    a.xvec          = aligned(lo, 16) && aligned(hi, 16) && (a.m <= 1 || gu->nb[1] % 16 == 0);
    return MI_OK;
}

int mi_mul_mat_q8_0_swiglu_workspace(int64_t k, int64_t n, const mi_tensor * gu, size_t * bytes) {
    if (!bytes) {
        return MI_ERR_NULL;
    }
    MmvArgs a;
    MI_TRY(mm_glu_desc(nullptr, k, n, gu, 0, nullptr, a));
    *bytes = a.m == 0 || a.n == 0 ? 0 : mul_mat_q8_0_workspace(a);
    return MI_OK;
}

int mi_mul_mat_q8_0_swiglu(const void * w, int64_t k, int64_t n, const mi_tensor * gu, int swapped,
                           const mi_tensor * y, void * workspace, size_t workspace_bytes, mi_stream stream) {
    if (!y) {
        return MI_ERR_NULL;
    }
    MmvArgs a;
    MI_TRY(mm_glu_desc(w, k, n, gu, swapped, y, a));
    if (a.m == 0 || a.n == 0) {
        return MI_OK;
    }
    if (!w) {
        return MI_ERR_NULL;
    }
    if (!aligned(w, 16)) {
        return MI_ERR_ALIGN;
    }
    if (!workspace || workspace_bytes < mul_mat_q8_0_workspace(a)) {
        return MI_ERR_PARAM;
    }
    if (!aligned(workspace, 256)) {
        return MI_ERR_ALIGN;
    }
    mul_mat_q8_0_bind(a, (char *) workspace);
    return finish(launch_mul_mat_q8_0(a, (hipStream_t) stream));
}

// an F32 vector of k contiguous elements (the norm weight, a gate, a modulate scale or shift)
static int mm_vec(const mi_tensor * v, int64_t k) {
    MI_TRY(check(v));
    if (v->type != MI_TYPE_F32) {
        return MI_ERR_TYPE;
    }
    if (v->ne[0] != k || nrows(*v) != 1 || v->nb[0] != 4) {
        return MI_ERR_SHAPE;
    }
    return MI_OK;
}

static int mm_swiglu_res(const void * w, int64_t k, int64_t n, const mi_tensor * gu, int swapped, const mi_tensor * r,
                         const mi_tensor * gate, int clamp, float lo, float hi, const mi_tensor * y, void * workspace,
                         size_t workspace_bytes, mi_stream stream) {
    if (!y || !r) {
        return MI_ERR_NULL;
    }
    MmvArgs a;
    MI_TRY(mm_glu_desc(w, k, n, gu, swapped, y, a));
    if (gate) {
        MI_TRY(mm_vec(gate, n));
        a.rgate = (const float *) gate->data;
    }
    MI_TRY(check(r));
    if (r->type != MI_TYPE_F32) {
        return MI_ERR_TYPE;
    }
    if (!same_shape(*r, *y) || !uniform_rows(*r) || r->nb[0] != 4) {
        return MI_ERR_SHAPE;
    }
    if (clamp && !(lo <= hi)) {
        return MI_ERR_PARAM;
    }
    if (a.m == 0 || a.n == 0) {
        return MI_OK;
    }
    if (!w) {
        return MI_ERR_NULL;
    }
    if (!aligned(w, 16)) {
        return MI_ERR_ALIGN;
    }
    if (!workspace || workspace_bytes < mul_mat_q8_0_workspace(a)) {
        return MI_ERR_PARAM;
    }
    if (!aligned(workspace, 256)) {
        return MI_ERR_ALIGN;
    }
    a.res    = (const char *) r->data;
    a.res1   = (int64_t) r->nb[1];
    a.rclamp = clamp != 0;
    a.rlo    = lo;
    a.rhi    = hi;
    mul_mat_q8_0_bind(a, (char *) workspace);
    return finish(launch_mul_mat_q8_0(a, (hipStream_t) stream));
}

int mi_mul_mat_q8_0_swiglu_add(const void * w, int64_t k, int64_t n, const mi_tensor * gu, int swapped,
                               const mi_tensor * r, int clamp, float lo, float hi, const mi_tensor * y, void * workspace,
                               size_t workspace_bytes, mi_stream stream) {
    return mm_swiglu_res(w, k, n, gu, swapped, r, nullptr, clamp, lo, hi, y, workspace, workspace_bytes, stream);
}

int mi_mul_mat_q8_0_swiglu_gated_add(const void * w, int64_t k, int64_t n, const mi_tensor * gu, int swapped,
                                     const mi_tensor * r, const mi_tensor * gate, const mi_tensor * y, void * workspace,
                                     size_t workspace_bytes, mi_stream stream) {
    if (!gate) {
        return MI_ERR_NULL;
    }
    return mm_swiglu_res(w, k, n, gu, swapped, r, gate, 0, 0.0f, 0.0f, y, workspace, workspace_bytes, stream);
}


static int mm_norm(const void * w, int64_t k, int64_t n, const mi_tensor * x, const mi_tensor * b,
                   const mi_tensor * norm_w, float eps, const mi_tensor * sum, const mi_tensor * y, void * workspace,
                   size_t workspace_bytes, mi_stream stream, const mi_tensor * gate = nullptr,
                   const mi_tensor * scale = nullptr, const mi_tensor * shift = nullptr) {
    if (!y || !norm_w) {
        return MI_ERR_NULL;
    }
    if ((scale == nullptr) != (shift == nullptr) || (gate && !b)) {
        return MI_ERR_NULL;
    }
    MmvArgs a;
    MI_TRY(mm_desc(w, k, n, x, y, a));
    if (gate) {
        MI_TRY(mm_vec(gate, k));
        a.gate = (const float *) gate->data;
    }
    if (scale) {
        MI_TRY(mm_vec(scale, k));
        MI_TRY(mm_vec(shift, k));
        a.msc = (const float *) scale->data;
        a.msh = (const float *) shift->data;
    }
    if (b) {  // the residual addend and the sum: F32 rows of x's shape, uniformly strided
        if (!sum) {
            return MI_ERR_NULL;
        }
        MI_TRY(check(b));
        MI_TRY(check(sum));
        if (b->type != MI_TYPE_F32 || sum->type != MI_TYPE_F32) {
            return MI_ERR_TYPE;
        }
        if (!same_shape(*b, *x) || !same_shape(*sum, *x) || !uniform_rows(*b) || !uniform_rows(*sum) ||
            b->nb[0] != 4 || sum->nb[0] != 4) {
            return MI_ERR_SHAPE;
        }
        // the second pass forms a + b again from the inputs: sum must not overlap them
        auto span_overlap = [&](const mi_tensor & p, const mi_tensor & q) {
            const char * p0 = (const char *) p.data;
            const char * q0 = (const char *) q.data;
            const char * p1 = p0 + (size_t) (a.m - 1) * p.nb[1] + (size_t) k * 4;
            const char * q1 = q0 + (size_t) (a.m - 1) * q.nb[1] + (size_t) k * 4;
            return p0 < q1 && q0 < p1;
        };
        if (a.m > 0 && (span_overlap(*sum, *x) || span_overlap(*sum, *b))) {
            return MI_ERR_PARAM;
        }
        a.ab   = (const char *) b->data;
        a.ab1  = (int64_t) b->nb[1];
        a.sum  = (char *) sum->data;
        a.sum1 = (int64_t) sum->nb[1];
        a.xvec = a.xvec && aligned(b->data, 16) && (a.m <= 1 || b->nb[1] % 16 == 0);
    }
    MI_TRY(mm_vec(norm_w, k));
    if (!(eps >= 0.0f)) {
        return MI_ERR_PARAM;
    }
    if (a.m == 0 || a.n == 0) {
        return MI_OK;
    }
    if (!w) {
        return MI_ERR_NULL;
    }
    if (!aligned(w, 16)) {
        return MI_ERR_ALIGN;
    }
    if (!workspace || workspace_bytes < mul_mat_q8_0_workspace(a)) {
        return MI_ERR_PARAM;
    }
    if (!aligned(workspace, 256)) {
        return MI_ERR_ALIGN;
    }
    a.nw  = (const float *) norm_w->data;
    a.eps = eps;
    mul_mat_q8_0_bind(a, (char *) workspace);
    return finish(launch_mul_mat_q8_0(a, (hipStream_t) stream));
}

int mi_mul_mat_q8_0_rms_norm(const void * w, int64_t k, int64_t n, const mi_tensor * x, const mi_tensor * norm_w,
                             float eps, const mi_tensor * y, void * workspace, size_t workspace_bytes,
                             mi_stream stream) {
    return mm_norm(w, k, n, x, nullptr, norm_w, eps, nullptr, y, workspace, workspace_bytes, stream);
}

int mi_mul_mat_q8_0_add_rms_norm(const void * w, int64_t k, int64_t n, const mi_tensor * a, const mi_tensor * b,
                                 const mi_tensor * norm_w, float eps, const mi_tensor * sum, const mi_tensor * y,
                                 void * workspace, size_t workspace_bytes, mi_stream stream) {
    if (!b) {
        return MI_ERR_NULL;
    }
    return mm_norm(w, k, n, a, b, norm_w, eps, sum, y, workspace, workspace_bytes, stream);
}

int mi_mul_mat_q8_0_adaln(const void * w, int64_t k, int64_t n, const mi_tensor * a, const mi_tensor * b,
                          const mi_tensor * gate, const mi_tensor * norm_w, const mi_tensor * scale,
                          const mi_tensor * shift, float eps, const mi_tensor * sum, const mi_tensor * y,
                          void * workspace, size_t workspace_bytes, mi_stream stream) {
    return mm_norm(w, k, n, a, b, norm_w, eps, b ? sum : nullptr, y, workspace, workspace_bytes, stream, gate, scale,
                   shift);
}

// F32 [oc, t, n] contiguous, the velocity/latent layout of the sampler
static int lat_check(const mi_tensor * x, const mi_tensor * ref) {
    MI_TRY(check(x));
    if (x->type != MI_TYPE_F32) {
        return MI_ERR_TYPE;
    }
    if (ref && !same_shape(*x, *ref)) {
        return MI_ERR_SHAPE;
    }
    if (x->ne[3] != 1) {
        return MI_ERR_SHAPE;
    }
    if (x->nb[1] != (uint64_t) x->ne[0] * 4 || x->nb[2] != x->nb[1] * (uint64_t) x->ne[1]) {
        return MI_ERR_STRIDE;
    }
    return MI_OK;
}

int mi_apg_buffer_bytes(const mi_tensor * cond, size_t * bytes) {
    if (!bytes) {
        return MI_ERR_NULL;
    }
    MI_TRY(lat_check(cond, nullptr));
    *bytes = (size_t) nelements(*cond) * sizeof(double);
    return MI_OK;
}

int mi_apg_forward(const mi_tensor * cond, const mi_tensor * uncond, float guidance_scale, float momentum,
                   float norm_threshold, void * momentum_buf, size_t momentum_bytes, int first, const mi_tensor * out,
                   mi_stream stream) {
    MI_TRY(lat_check(cond, nullptr));
    MI_TRY(lat_check(uncond, cond));
    MI_TRY(lat_check(out, cond));
    if (!std::isfinite(guidance_scale) || !std::isfinite(momentum) || !std::isfinite(norm_threshold)) {
        return MI_ERR_PARAM;
    }
    if (cond->ne[0] > 1024) {
        return MI_ERR_UNSUPPORTED;  // channels per workgroup
    }
    const size_t need = (size_t) nelements(*cond) * sizeof(double);
    if (need > 0 && (!momentum_buf || momentum_bytes < need)) {
        return MI_ERR_PARAM;
    }
    if (!aligned(momentum_buf, 8)) {
        return MI_ERR_ALIGN;
    }
    ApgArgs a;
    a.cond      = (const float *) cond->data;
    a.uncond    = (const float *) uncond->data;
    a.out       = (float *) out->data;
    a.ra        = (double *) momentum_buf;
    a.oc        = (uint32_t) cond->ne[0];
    a.t         = (uint32_t) cond->ne[1];
    a.n         = (uint32_t) cond->ne[2];
    a.first     = first != 0;
    a.scale     = guidance_scale;
    a.threshold = norm_threshold;
    a.momentum  = (double) momentum;
    return finish(launch_apg(a, (hipStream_t) stream));
}

int mi_flow_step(int solver, const mi_tensor * vt, const mi_tensor * xt, float t_curr, float t_next, int history,
                 const mi_tensor * prev, const mi_tensor * prev2, mi_stream stream) {
    MI_TRY(lat_check(vt, nullptr));
    MI_TRY(lat_check(xt, vt));
    if (solver != MI_SOLVER_EULER && solver != MI_SOLVER_DPM3M) {
        return MI_ERR_PARAM;
    }
    if (!std::isfinite(t_curr) || !std::isfinite(t_next) || history < 0 || history > 2) {
        return MI_ERR_PARAM;
    }
    FlowArgs a{};
    if (solver == MI_SOLVER_DPM3M) {
        MI_TRY(lat_check(prev, vt));
        MI_TRY(lat_check(prev2, vt));
        a.prev  = (float *) prev->data;
        a.prev2 = (float *) prev2->data;
    }
    a.xt     = (float *) xt->data;
    a.vt     = (const float *) vt->data;
    a.n      = (uint64_t) nelements(*vt);
    a.solver = solver == MI_SOLVER_EULER ? 0 : 1;
    a.hist   = history;
    a.t_curr = t_curr;
    a.t_next = t_next;
    return finish(launch_flow_step(a, (hipStream_t) stream));
}

int mi_flow_final(const mi_tensor * xt, const mi_tensor * vt, float t, const mi_tensor * out, mi_stream stream) {
    MI_TRY(lat_check(vt, nullptr));
    MI_TRY(lat_check(xt, vt));
    MI_TRY(lat_check(out, vt));
    if (!std::isfinite(t)) {
        return MI_ERR_PARAM;
    }
    FlowArgs a{};
    a.xt     = (float *) xt->data;
    a.vt     = (const float *) vt->data;
    a.out    = (float *) out->data;
    a.n      = (uint64_t) nelements(*vt);
    a.solver = 2;
    a.t_curr = t;
    return finish(launch_flow_step(a, (hipStream_t) stream));
}

int mi_flow_step_sde(const mi_tensor * vt, const mi_tensor * xt, const mi_tensor * noise, float t_curr, float t_next,
                     mi_stream stream) {
    MI_TRY(lat_check(vt, nullptr));
    MI_TRY(lat_check(xt, vt));
    MI_TRY(lat_check(noise, vt));
    if (!std::isfinite(t_curr) || !std::isfinite(t_next)) {
        return MI_ERR_PARAM;
    }
    FlowArgs a{};
    a.xt     = (float *) xt->data;
    a.vt     = (const float *) vt->data;
    a.noise  = (const float *) noise->data;
    a.n      = (uint64_t) nelements(*vt);
    a.solver = 3;
    a.t_curr = t_curr;
    a.t_next = t_next;
    return finish(launch_flow_step(a, (hipStream_t) stream));
}

int mi_stork4_workspace(const mi_tensor * xt, size_t * bytes) {
    if (!bytes) {
        return MI_ERR_NULL;
    }
    MI_TRY(lat_check(xt, nullptr));
    *bytes = STORK_WS_XNEXT + (size_t) nelements(*xt) * sizeof(float);
    return MI_OK;
}

// _rock4_mdegr (solver-stork.h:140-159): the tabulated degree for s, its row
// in the finishing tables, and its offset in the recurrence table
static void rock4_degree(const mi_rock4_tables & t, int s, int & mdeg, int & mz, int & mr) {
    int mp1 = 1;
    for (int i = 0; i < t.ms_len; i++) {
        if (t.ms[i] >= s) {
            mdeg = t.ms[i];
            mz   = i;
            mr   = mp1 - 1;
            return;
        }
        mp1 += t.ms[i] * 2 - 1;
    }
    mz   = t.ms_len - 1;
    mdeg = t.ms[mz];
    mr   = mp1 - 1;
}

// The fp32 scalar chain of one sub-stepping attempt (solver-stork.h:179-264),
// in the reference's order; false when the tables are too short for it.
static bool rock4_plan(const mi_rock4_tables & t, int s, float t_curr, float t_next, StorkPlan & p) {
    const int smax = t.ms[t.ms_len - 1];
    if (s > smax) {
        s = smax;
    }
    int mdeg = 0, mz = 0, mr = 0;
    rock4_degree(t, s, mdeg, mz, mr);
    if (mdeg < 1 || mdeg > STORK_MAX_DEG || mr < 0 || (int64_t) mr + 2 * (int64_t) (mdeg - 2) + 2 >= t.recf_len ||
        mr >= t.recf_len) {
        return false;
    }
    const float dt = t_curr - t_next;
    p.mdeg         = mdeg;
    float ci1 = t_curr, ci2 = t_curr, ci3 = t_curr;
    for (int j = 1; j <= mdeg; j++) {
        if (j == 1) {
            p.t1_first = -dt * (float) t.recf[mr];
            ci1        = t_curr + p.t1_first;
            ci2        = ci1;
        } else {
            float * c   = p.sub[j - 2];
            c[3]        = ci1 - t_curr;
            c[0]        = -dt * (float) t.recf[mr + 2 * (j - 2) + 1];
            c[2]        = -(float) t.recf[mr + 2 * (j - 2) + 2];
            c[1]        = 1.0f - c[2];
            const float nw = c[0] + c[1] * ci2 + c[2] * ci3;
            ci3            = ci2;
            ci2            = nw;
            ci1            = nw;
        }
    }
    const double * fa = t.fpa + 6 * mz;
    const double * fb = t.fpb + 4 * mz;
    const float    a0 = -dt * (float) fa[0];
    p.fin_diff[0]     = ci1 - t_curr;
    float c2f         = ci1 + a0;
    const float a1 = -dt * (float) fa[1], a2 = -dt * (float) fa[2];
    p.fin_diff[1]  = c2f - t_curr;
    c2f            = ci1 + a1 + a2;
    const float a3 = -dt * (float) fa[3], a4 = -dt * (float) fa[4], a5 = -dt * (float) fa[5];
    p.fin_diff[2]  = c2f - t_curr;
    c2f            = ci1 + a3 + a4 + a5;
    p.fin_diff[3]  = c2f - t_curr;
    for (int k = 0; k < 4; ++k) {
        p.fpb[k] = -dt * (float) fb[k];
    }
    return true;
}

int mi_stork4_step(const mi_tensor * vt, const mi_tensor * xt, float t_curr, float t_next, int history, float h_prev,
                   float h_prev2, const mi_tensor * prev, const mi_tensor * prev2, int substeps,
                   const mi_rock4_tables * tables, void * workspace, size_t workspace_bytes, mi_stream stream) {
    MI_TRY(lat_check(vt, nullptr));
    MI_TRY(lat_check(xt, vt));
    MI_TRY(lat_check(prev, vt));
    MI_TRY(lat_check(prev2, vt));
    if (!tables || !tables->ms || !tables->fpa || !tables->fpb || !tables->recf) {
        return MI_ERR_NULL;
    }
    if (!std::isfinite(t_curr) || !std::isfinite(t_next) || !std::isfinite(h_prev) || !std::isfinite(h_prev2) ||
        history < 0) {
        return MI_ERR_PARAM;
    }
    const mi_rock4_tables & tb = *tables;
    if (tb.ms_len < 1 || tb.recf_len < 1) {
        return MI_ERR_PARAM;
    }
    for (int i = 0; i < tb.ms_len; ++i) {
        if (tb.ms[i] < 1 || (i > 0 && tb.ms[i] <= tb.ms[i - 1])) {
            return MI_ERR_PARAM;
        }
    }
    if (tb.ms[tb.ms_len - 1] > STORK_MAX_DEG) {
        return MI_ERR_UNSUPPORTED;
    }
    const size_t n = (size_t) nelements(*vt);
    if (!workspace || workspace_bytes < STORK_WS_XNEXT + n * sizeof(float)) {
        return MI_ERR_PARAM;
    }
    if (!aligned(workspace, 256)) {
        return MI_ERR_ALIGN;
    }
    StorkArgs a{};
    a.xt     = (float *) xt->data;
    a.vt     = (const float *) vt->data;
    a.prev   = (float *) prev->data;
    a.prev2  = (float *) prev2->data;
    a.status = (uint32_t *) workspace;
    a.part   = (double *) ((char *) workspace + STORK_WS_STATUS);
    a.xnext  = (float *) ((char *) workspace + STORK_WS_XNEXT);
    a.n      = (uint64_t) n;
    a.hist   = history > 2 ? 2 : history;
    a.h1     = h_prev;
    a.h2     = h_prev2;
    a.dt     = t_curr - t_next;
    // The derivative order the step sizes allow (solver-stork.h:75-111); the
    // guards on the velocities' sums of squares run on the device.
    a.max_order = 0;
    if (a.hist >= 1 && h_prev != 0.0f) {
        a.max_order = 1;
        if (a.hist >= 2 && h_prev2 != 0.0f) {
            const double h1 = (double) h_prev, h2 = (double) h_prev2, den = h1 * h2 * (h1 + h2);
            if (!(std::fabs(den) < 1e-30)) {
                a.max_order = 2;
                a.c2        = 2.0 / den;
            }
        }
    }
    // The halving sequence of sub-step counts (solver-stork.h:302-309); counts
    // that map to the degree of the attempt before give its result again and
    // are skipped.
    std::vector<StorkPlan> plans;
    if (a.hist > 0) {
        int s = substeps >= 2 ? substeps : 2;
        while (s >= 2) {
            StorkPlan p;
            if (!rock4_plan(tb, s, t_curr, t_next, p)) {
                return MI_ERR_PARAM;
            }
            if (plans.empty() || plans.back().mdeg != p.mdeg) {
                if ((int) plans.size() == STORK_MAX_ATTEMPTS) {
                    return MI_ERR_UNSUPPORTED;
                }
                p.attempt                = (int32_t) plans.size();
                a.att_deg[plans.size()] = p.mdeg;
                plans.push_back(p);
            }
            s /= 2;
        }
    }
    a.n_attempts = (int) plans.size();
    return finish(launch_stork4(a, plans.data(), (hipStream_t) stream));
}

int mi_dcw(int mode, const mi_tensor * xt, const mi_tensor * vt, float t_curr, float t_next, float scaler,
           float high_scaler, mi_stream stream) {
    MI_TRY(lat_check(vt, nullptr));
    MI_TRY(lat_check(xt, vt));
    if (mode < MI_DCW_LOW || mode > MI_DCW_PIX) {
        return MI_ERR_PARAM;
    }
    if (!std::isfinite(t_curr) || !std::isfinite(t_next) || !std::isfinite(scaler) || !std::isfinite(high_scaler)) {
        return MI_ERR_PARAM;
    }
    if (xt->ne[0] > UINT32_MAX || xt->ne[1] > UINT32_MAX || xt->ne[2] > UINT32_MAX) {
        return MI_ERR_UNSUPPORTED;
    }
    // the per-mode effective scalers (dit-sampler.h:641-644)
    const float s_low = t_curr * scaler, s_high = (1.0f - t_curr) * scaler;
    const float s_dh = (1.0f - t_curr) * high_scaler;
    DcwArgs     a{};
    a.xt     = (float *) xt->data;
    a.vt     = (const float *) vt->data;
    a.oc     = (uint32_t) xt->ne[0];
    a.t      = (uint32_t) xt->ne[1];
    a.n      = (uint32_t) xt->ne[2];
    a.t_next = t_next;
    a.pix    = mode == MI_DCW_PIX;
    a.lo_s   = mode == MI_DCW_LOW || mode == MI_DCW_DOUBLE ? s_low : mode == MI_DCW_PIX ? scaler : 0.0f;
    a.hi_s   = mode == MI_DCW_HIGH ? s_high : mode == MI_DCW_DOUBLE ? s_dh : 0.0f;
    if (a.lo_s == 0.0f && a.hi_s == 0.0f) {
        return MI_OK;  // the reference returns before the transform
    }
    return finish(launch_dcw(a, (hipStream_t) stream));
}

int mi_scale(const mi_tensor * x, float s, const mi_tensor * y, mi_stream stream) {
    MI_TRY(check_act(x));
    MI_TRY(check_act(y));
    if (!same_shape(*x, *y)) {
        return MI_ERR_SHAPE;
    }
    return finish(launch_scale(*x, s, *y, (hipStream_t) stream));
}

int mi_timestep_embedding(const mi_tensor * t, int dim, int max_period, const mi_tensor * y, mi_stream stream) {
    MI_TRY(check(t));
    MI_TRY(check(y));
    if (t->type != MI_TYPE_F32 || y->type != MI_TYPE_F32) {
        return MI_ERR_TYPE;
    }
    if (dim <= 0 || max_period <= 0) {
        return MI_ERR_PARAM;
    }
    if (t->ne[1] != 1 || t->ne[2] != 1 || t->ne[3] != 1 || y->ne[0] != dim || y->ne[1] != t->ne[0] ||
        y->ne[2] != 1 || y->ne[3] != 1) {
        return MI_ERR_SHAPE;
    }
    return finish(launch_timestep_embedding((const float *) t->data, t->ne[0], 1, dim, max_period, (char *) y->data,
                                            (int64_t) y->nb[1], (hipStream_t) stream));
}

}  // extern "C"
