// getrows.hip -- ggml_get_rows: embedding lookup with on-the-fly dequant.
//
// Reference sites: qwen3-enc.h:390, 465; qwen3-lm.h:464, 626 (token
// embedding; the table is Q8_0 in Q8_0 GGUFs, tools/quantize.cpp:62).
// Q8_0 dequant (dequantize_row_q8_0): y[32b + j] = (float)qs[j] * fp16(d_b).
// The int8 x fp16 product has at most 8 + 11 significant bits, so the fp32
// result is exact: the output is bit-identical to ggml-cpu.
//
// Q8_0 path: one wave per id; each lane produces 8 consecutive outputs (two
// 16-byte stores, so the wave's stores are fully coalesced). Its 8 quants sit
// at byte 34b + 2 + 8k of the row, which is only 2-byte aligned, so they are
// read as four 16-bit loads (always in bounds: no over-read past a block).
// F16/BF16/F32 tables: 16-byte row vectors converted to f32.
// An id outside [0, n_rows) writes a zero row and bumps *d_err.
#include "launch.h"

namespace mi {

struct GetRowsArgs {
    const char *    table;
    int64_t         tnb1;      // table row stride (bytes)
    int64_t         n_rows;
    const int32_t * ids;
    int64_t         ids_stride;  // elements
    uint32_t        n_ids;
    int             n;           // ne0 (elements per row)
    char *          y;
    int64_t         ynb1;
    int32_t *       d_err;
};

__device__ __forceinline__ float i8f(uint32_t w, int k) {
    return (float) (int32_t) __builtin_amdgcn_sbfe(w, 8 * k, 8);
}

template <int TO>
__global__ void __launch_bounds__(256) k_get_rows_q8_0(const GetRowsArgs a) {
    constexpr int EO   = TT<TO>::ES;
    const int     lane = threadIdx.x & 63;
    const int     wpb  = blockDim.x >> 6;
    const int     n8   = a.n >> 3;  // groups of 8 outputs
    for (uint32_t i = blockIdx.x * wpb + (threadIdx.x >> 6); i < a.n_ids; i += gridDim.x * wpb) {
        const int64_t r   = a.ids[(int64_t) i * a.ids_stride];
        char *        yp  = a.y + (int64_t) i * a.ynb1;
        const bool    bad = r < 0 || r >= a.n_rows;
        if (bad && lane == 0 && a.d_err) {
            atomicAdd(a.d_err, 1);
        }
        const char * row = a.table + (bad ? 0 : r) * a.tnb1;
        for (int m = lane; m < n8; m += 64) {
            float f[8];
            if (!bad) {
                const int       b  = m >> 2;
                const char *    bp = row + (size_t) b * 34;
                const uint16_t  dh = *(const uint16_t *) bp;
                const uint16_t * qp = (const uint16_t *) (bp + 2 + (m & 3) * 8);
                const uint32_t  w0 = (uint32_t) qp[0] | ((uint32_t) qp[1] << 16);
                const uint32_t  w1 = (uint32_t) qp[2] | ((uint32_t) qp[3] << 16);
                const float     d  = (float) __builtin_bit_cast(_Float16, dh);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    f[k]     = i8f(w0, k) * d;
                    f[k + 4] = i8f(w1, k) * d;
                }
            } else {
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    f[k] = 0.0f;
                }
            }
            store_vec<TO, 8>(yp + (size_t) m * 8 * EO, f);
        }
    }
}

template <int TT_, int TO>
__global__ void __launch_bounds__(256) k_get_rows_vec(const GetRowsArgs a) {
    constexpr int VI   = TT<TT_>::VEC;
    constexpr int EO   = TT<TO>::ES;
    const int     lane = threadIdx.x & 63;
    const int     wpb  = blockDim.x >> 6;
    const int     nv   = a.n / VI;
    for (uint32_t i = blockIdx.x * wpb + (threadIdx.x >> 6); i < a.n_ids; i += gridDim.x * wpb) {
        const int64_t r   = a.ids[(int64_t) i * a.ids_stride];
        char *        yp  = a.y + (int64_t) i * a.ynb1;
        const bool    bad = r < 0 || r >= a.n_rows;
        if (bad && lane == 0 && a.d_err) {
            atomicAdd(a.d_err, 1);
        }
        const char * row = a.table + (bad ? 0 : r) * a.tnb1;
        for (int m = lane; m < nv; m += 64) {
            float f[VI];
            if (!bad) {
                unpack16<TT_>(ld16(row + (size_t) m * 16), f);
            } else {
#pragma unroll
                for (int k = 0; k < VI; ++k) {
                    f[k] = 0.0f;
                }
            }
            store_vec<TO, VI>(yp + (size_t) m * VI * EO, f);
        }
    }
}

// Generic: any n, element-aligned table rows, scalar.
template <int TO>
__global__ void __launch_bounds__(256) k_get_rows_generic(const GetRowsArgs a, int ttype) {
    constexpr int EO   = TT<TO>::ES;
    const int     lane = threadIdx.x & 63;
    const int     wpb  = blockDim.x >> 6;
    for (uint32_t i = blockIdx.x * wpb + (threadIdx.x >> 6); i < a.n_ids; i += gridDim.x * wpb) {
        const int64_t r   = a.ids[(int64_t) i * a.ids_stride];
        char *        yp  = a.y + (int64_t) i * a.ynb1;
        const bool    bad = r < 0 || r >= a.n_rows;
        if (bad && lane == 0 && a.d_err) {
            atomicAdd(a.d_err, 1);
        }
        const char * row = a.table + (bad ? 0 : r) * a.tnb1;
        for (int j = lane; j < a.n; j += 64) {
            float v = 0.0f;
            if (!bad) {
                switch (ttype) {
                    case MI_TYPE_Q8_0: {
                        const char *   bp = row + (size_t) (j >> 5) * 34;
                        const uint16_t dh = *(const uint16_t *) bp;
                        v = (float) (int8_t) bp[2 + (j & 31)] * (float) __builtin_bit_cast(_Float16, dh);
                        break;
                    }
                    case MI_TYPE_F32:
                        v = load_elem<MI_TYPE_F32>(row + (size_t) j * 4);
                        break;
                    case MI_TYPE_BF16:
                        v = load_elem<MI_TYPE_BF16>(row + (size_t) j * 2);
                        break;
                    default:
                        v = load_elem<MI_TYPE_F16>(row + (size_t) j * 2);
                        break;
                }
            }
            store_elem<TO>(yp + (size_t) j * EO, v);
        }
    }
}

template <int TO>
static int launch_to(const GetRowsArgs & a, int ttype, bool fast, hipStream_t s) {
    uint32_t       grid = (a.n_ids + 3) / 4;
    const uint32_t cap  = (uint32_t) num_cus() * 16;
    grid                = grid > cap ? cap : grid;
    if (fast) {
        switch (ttype) {
            case MI_TYPE_Q8_0:
                hipLaunchKernelGGL((k_get_rows_q8_0<TO>), dim3(grid), dim3(256), 0, s, a);
                return MI_OK;
            case MI_TYPE_F32:
                hipLaunchKernelGGL((k_get_rows_vec<MI_TYPE_F32, TO>), dim3(grid), dim3(256), 0, s, a);
                return MI_OK;
            case MI_TYPE_BF16:
                hipLaunchKernelGGL((k_get_rows_vec<MI_TYPE_BF16, TO>), dim3(grid), dim3(256), 0, s, a);
                return MI_OK;
            default:
                hipLaunchKernelGGL((k_get_rows_vec<MI_TYPE_F16, TO>), dim3(grid), dim3(256), 0, s, a);
                return MI_OK;
        }
    }
    hipLaunchKernelGGL((k_get_rows_generic<TO>), dim3(grid), dim3(256), 0, s, a, ttype);
    return MI_OK;
}

int launch_get_rows(const mi_tensor & table, const int32_t * ids, int64_t n_ids, int64_t ids_stride,
                    const mi_tensor & y, int32_t * d_err, hipStream_t s) {
    if (n_ids == 0 || table.ne[0] == 0) {
        return MI_OK;
    }
    GetRowsArgs a;
    a.table      = (const char *) table.data;
    a.tnb1       = (int64_t) table.nb[1];
    a.n_rows     = table.ne[1];
    a.ids        = ids;
    a.ids_stride = ids_stride;
    a.n_ids      = (uint32_t) n_ids;
    a.n          = (int) table.ne[0];
    a.y          = (char *) y.data;
    a.ynb1       = (int64_t) y.nb[1];
    a.d_err      = d_err;

    const int es_out = type_size(y.type);
    bool      fast;
    if (table.type == MI_TYPE_Q8_0) {
        // 8 outputs per lane; 16-bit aligned quants; output 16-byte stores
        fast = a.n % 8 == 0 && aligned(table.data, 2) && a.tnb1 % 2 == 0 && aligned(y.data, 16) &&
               (a.ynb1 % 16 == 0) && (8 * es_out) % 16 == 0;
    } else {
        const int VI = 16 / type_size(table.type);
        fast         = a.n % VI == 0 && aligned(table.data, 16) && a.tnb1 % 16 == 0 && aligned(y.data, 16) &&
               a.ynb1 % 16 == 0 && (VI * es_out) % 8 == 0;
    }
    if (y.type == MI_TYPE_F32) {
        return launch_to<MI_TYPE_F32>(a, table.type, fast, s);
    }
    return launch_to<MI_TYPE_BF16>(a, table.type, fast, s);
}

}  // namespace mi
