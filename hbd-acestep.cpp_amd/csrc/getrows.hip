// getrows.hip -- ggml_get_rows: embedding lookup with on-the-fly dequant.
//
// Reference sites: qwen3-enc.h:390, 465; qwen3-lm.h:464, 626 (token
// embedding; the table is Q8_0 in Q8_0 GGUFs, tools/quantize.cpp:62).
// Q8_0 dequant (dequantize_row_q8_0): y[32b + j] = (float)qs[j] * fp16(d_b).
// The int8 x fp16 product has at most 8 + 11 significant bits, so the fp32
// result is exact: the output is bit-identical to ggml-cpu.
//
// Q8_0 path: rows shorter than 64 16-byte output vectors (KV-cache heads) go
// through a flat kernel, one output vector per thread-step. Longer rows: one
// wave per id; each lane produces one 16-byte output vector (4 F32 or 8 BF16
// outputs) per step, so every store instruction writes 1 KB contiguous. When
// the row is a whole number of 16-byte chunks (ne0 % 256 == 0: every Qwen3
// hidden size) the wave first stages the row in LDS with coalesced 16-byte
// loads, so a row costs one memory round trip; otherwise a lane's quants,
// only 2-byte aligned (block b starts at byte 34b), are read as 16-bit loads.
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
    constexpr int OPS  = 16 / EO;  // outputs per 16-byte store: wave-contiguous store instructions
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
        for (int o = lane * OPS; o < a.n; o += 64 * OPS) {
            float f[OPS];
            if (!bad) {
                const char *     bp = row + (size_t) (o >> 5) * 34;
                const uint16_t * qp = (const uint16_t *) (bp + 2 + (o & 31));
                const float      d  = (float) __builtin_bit_cast(_Float16, *(const uint16_t *) bp);
#pragma unroll
                for (int h = 0; h < OPS / 4; ++h) {
                    const uint32_t w = (uint32_t) qp[2 * h] | ((uint32_t) qp[2 * h + 1] << 16);
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        f[4 * h + k] = i8f(w, k) * d;
                    }
                }
            } else {
#pragma unroll
                for (int k = 0; k < OPS; ++k) {
                    f[k] = 0.0f;
                }
            }
            store_vec<TO, OPS>(yp + (size_t) o * EO, f);
        }
    }
}

// Q8_0 rows whose byte length is a multiple of 16 (ne0 % 256 == 0) in a
// 16-byte aligned table: the wave copies its row into LDS with coalesced
// 16-byte loads, all issued at once, then each lane decodes groups of 8 outputs
// from LDS and writes them with 16-byte stores. A wave walks ids a grid stride
// apart, and the next id's row loads are issued (into the registers just copied
// to LDS) before this id's outputs are written, so their memory latency runs
// under the stores. LDS per wave: the row's nc 16-byte chunks (nc <= 9*64,
// ne0 <= 8192).
#ifndef MI_GR_LDS_WG_PER_CU
#define MI_GR_LDS_WG_PER_CU 16  // grid cap of the LDS kernel, in workgroups per CU
#endif
// MAXC: 64-lane load rounds per row, ceil(nc / 64) (the registers that carry the
// next row stay live through the stores, so only the rounds the row needs)
template <int TO, int MAXC>
__global__ void __launch_bounds__(256) k_get_rows_q8_0_lds(const GetRowsArgs a, int nc) {
    extern __shared__ uint4 stage_all[];
    constexpr int    EO   = TT<TO>::ES;
    constexpr int    OPS  = 16 / EO;  // outputs per 16-byte store: 4 (F32) or 8 (BF16)
    const int        lane = threadIdx.x & 63;
    const uint32_t   wv   = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint4 *          stage = stage_all + wv * nc;
    const uint16_t * s16   = (const uint16_t *) stage;
    const uint32_t   step  = gridDim.x * 4;
    uint4            v[MAXC];
    // the row of id `id`; its loads are issued into v when it is valid. The id
    // (wave-uniform) comes through the scalar path: waiting for it does not
    // wait for the previous row's stores, which the vector memory counter
    // also tracks.
    auto fetch = [&](uint32_t id) -> int64_t {
        const int64_t r = ld_scalar_i32(a.ids, (int64_t) id * a.ids_stride);
        if (r >= 0 && r < a.n_rows) {
            const char * row = a.table + r * a.tnb1;
#pragma unroll
            for (int k = 0; k < MAXC; ++k) {
                const int c = lane + 64 * k;
                if (c < nc) {
                    v[k] = ld16(row + (size_t) c * 16);
                }
            }
        }
        return r;
    };
    uint32_t i = blockIdx.x * 4 + wv;
    int64_t  r = i < a.n_ids ? fetch(i) : -1;
    for (; i < a.n_ids; i += step) {
        char *     yp  = a.y + (int64_t) i * a.ynb1;
        const bool bad = r < 0 || r >= a.n_rows;
        if (!bad) {
#pragma unroll
            for (int k = 0; k < MAXC; ++k) {
                const int c = lane + 64 * k;
                if (c < nc) {
                    stage[c] = v[k];
                }
            }
        }
        const uint32_t in = i + step;
        const int64_t  rn = in < a.n_ids ? fetch(in) : -1;  // in flight during this id's stores
        if (bad) {
            if (lane == 0 && a.d_err) {
                atomicAdd(a.d_err, 1);
            }
            float z[OPS] = {};
            for (int o = lane * OPS; o < a.n; o += 64 * OPS) {
                store_vec<TO, OPS>(yp + (size_t) o * EO, z);
            }
        } else {
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            __builtin_amdgcn_wave_barrier();
            // OPS outputs (one 16-byte store) per lane per step: each store
            // instruction writes 1 KB contiguous, whole cache lines
            for (int o = lane * OPS; o < a.n; o += 64 * OPS) {
                const uint16_t * bp = s16 + (o >> 5) * 17;  // a 34-byte block is 17 halfwords
                const uint16_t * qp = bp + 1 + ((o & 31) >> 1);
                const float      d  = (float) __builtin_bit_cast(_Float16, bp[0]);
                float            f[OPS];
#pragma unroll
                for (int h = 0; h < OPS / 4; ++h) {
                    const uint32_t w = (uint32_t) qp[2 * h] | ((uint32_t) qp[2 * h + 1] << 16);
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        f[4 * h + k] = i8f(w, k) * d;
                    }
                }
                store_vec<TO, OPS>(yp + (size_t) o * EO, f);
            }
        }
        // the next id overwrites this wave's LDS rows
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
        r = rn;
    }
}

template <int TT_, int TO>
__global__ void __launch_bounds__(256) k_get_rows_vec(const GetRowsArgs a) {
    constexpr int ET   = TT<TT_>::ES;
    constexpr int EO   = TT<TO>::ES;
    constexpr int OPS  = 16 / (ET > EO ? ET : EO);  // elements per lane step: 16-byte loads or stores
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
        for (int o = lane * OPS; o < a.n; o += 64 * OPS) {
            float f[OPS];
            if (bad) {
#pragma unroll
                for (int k = 0; k < OPS; ++k) {
                    f[k] = 0.0f;
                }
            } else if constexpr (OPS * ET == 16) {
                unpack16<TT_>(ld16(row + (size_t) o * ET), f);
            } else {  // 4 half-width elements widened to F32
                const uint2 w = *(const uint2 *) (row + (size_t) o * ET);
                f[0]          = TT_ == MI_TYPE_BF16 ? bf16_lo(w.x) : f16_lo(w.x);
                f[1]          = TT_ == MI_TYPE_BF16 ? bf16_hi(w.x) : f16_hi(w.x);
                f[2]          = TT_ == MI_TYPE_BF16 ? bf16_lo(w.y) : f16_lo(w.y);
                f[3]          = TT_ == MI_TYPE_BF16 ? bf16_hi(w.y) : f16_hi(w.y);
            }
            store_vec<TO, OPS>(yp + (size_t) o * EO, f);
        }
    }
}

// Flat Q8_0 path, for rows shorter than one wave-wide store (KV-cache heads):
// the output is a stream of 16-byte chunks (OPS outputs of one row) and each
// thread produces U of them, 256 chunks apart, so every store instruction
// still writes 1 KB contiguous. A thread finds each chunk's id and column by
// division, reads the id (shared by the row's threads, a cache hit after the
// first), then the block scale and its OPS quants (16-bit loads: a block is
// 34 bytes, so quants are only 2-byte aligned), and writes one 16-byte
// vector. All U chunks' loads are issued before the first store. A wave per
// row would leave most lanes idle on such rows. An invalid id writes zeros
// (its loads read row 0, which the host guarantees exists); its first
// chunk's thread bumps *d_err.
template <int TO, int U>
__global__ void __launch_bounds__(256) k_get_rows_q8_0_flat(const GetRowsArgs a, FastDiv per_row, uint32_t nchunks) {
    constexpr int  EO  = TT<TO>::ES;
    constexpr int  OPS = 16 / EO;
    const uint32_t c0  = blockIdx.x * (256 * U) + threadIdx.x;
    uint32_t       i[U];
    int            o[U];
    int64_t        r[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t c = c0 + 256 * u < nchunks ? c0 + 256 * u : nchunks - 1;  // clamped: loads stay in bounds
        i[u]             = per_row.div(c);
        o[u]             = (int) (c - i[u] * per_row.d) * OPS;
        r[u]             = a.ids[(int64_t) i[u] * a.ids_stride];
    }
    uint16_t dh[U], q[U][OPS / 2];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const bool       ok = r[u] >= 0 && r[u] < a.n_rows;
        const char *     bp = a.table + (ok ? r[u] : 0) * a.tnb1 + (int64_t) (o[u] >> 5) * 34;
        const uint16_t * qp = (const uint16_t *) (bp + 2 + (o[u] & 31));
        dh[u]               = *(const uint16_t *) bp;
#pragma unroll
        for (int h = 0; h < OPS / 2; ++h) {
            q[u][h] = qp[h];
        }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        if (c0 + 256 * u >= nchunks) {
            break;
        }
        float f[OPS];
        if (r[u] < 0 || r[u] >= a.n_rows) {
            if (o[u] == 0 && a.d_err) {
                atomicAdd(a.d_err, 1);
            }
#pragma unroll
            for (int k = 0; k < OPS; ++k) {
                f[k] = 0.0f;
            }
        } else {
            const float d = (float) __builtin_bit_cast(_Float16, dh[u]);
#pragma unroll
            for (int h = 0; h < OPS / 4; ++h) {
                const uint32_t w = (uint32_t) q[u][2 * h] | ((uint32_t) q[u][2 * h + 1] << 16);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    f[4 * h + k] = i8f(w, k) * d;
                }
            }
        }
        store_vec<TO, OPS>(a.y + (int64_t) i[u] * a.ynb1 + (int64_t) o[u] * EO, f);
    }
}

#ifndef MI_GR_FLAT_U
#define MI_GR_FLAT_U 4  // output chunks per thread in the flat kernel
#endif

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
static int launch_to(const GetRowsArgs & a, int ttype, bool fast, bool lds, hipStream_t s) {
    uint32_t       grid = (a.n_ids + 3) / 4;
    const uint32_t cap  = (uint32_t) num_cus() * 16;
    grid                = grid > cap ? cap : grid;
    if (fast) {
        switch (ttype) {
            case MI_TYPE_Q8_0: {
                constexpr int  OPS     = 16 / TT<TO>::ES;
                const uint64_t nchunks = (uint64_t) a.n_ids * (uint64_t) (a.n / OPS);
                // rows shorter than one wave-wide store; an invalid id loads from row 0
                if (a.n / OPS < 64 && a.n_rows > 0 && nchunks < (1ull << 31)) {
                    constexpr uint32_t per_wg = 256 * MI_GR_FLAT_U;
                    MI_LAUNCH((k_get_rows_q8_0_flat<TO, MI_GR_FLAT_U>),
                                       dim3((uint32_t) ((nchunks + per_wg - 1) / per_wg)), dim3(256), 0, s, a,
                                       FastDiv((uint32_t) (a.n / OPS)), (uint32_t) nchunks);
                    return MI_OK;
                }
                if (lds) {
                    const int      nc   = a.n / 32 * 34 / 16;
                    const uint32_t gcap = (uint32_t) num_cus() * MI_GR_LDS_WG_PER_CU;
                    const dim3     g(grid > gcap ? gcap : grid);
                    const size_t   lb = (size_t) 4 * nc * 16;
                    switch ((nc + 63) / 64) {  // nc <= 9 * 64 (ne0 <= 8192)
                        case 1: MI_LAUNCH((k_get_rows_q8_0_lds<TO, 1>), g, dim3(256), lb, s, a, nc); break;
                        case 2: MI_LAUNCH((k_get_rows_q8_0_lds<TO, 2>), g, dim3(256), lb, s, a, nc); break;
                        case 3: MI_LAUNCH((k_get_rows_q8_0_lds<TO, 3>), g, dim3(256), lb, s, a, nc); break;
                        case 4: MI_LAUNCH((k_get_rows_q8_0_lds<TO, 4>), g, dim3(256), lb, s, a, nc); break;
                        case 5: MI_LAUNCH((k_get_rows_q8_0_lds<TO, 5>), g, dim3(256), lb, s, a, nc); break;
                        case 6: MI_LAUNCH((k_get_rows_q8_0_lds<TO, 6>), g, dim3(256), lb, s, a, nc); break;
                        case 7: MI_LAUNCH((k_get_rows_q8_0_lds<TO, 7>), g, dim3(256), lb, s, a, nc); break;
                        case 8: MI_LAUNCH((k_get_rows_q8_0_lds<TO, 8>), g, dim3(256), lb, s, a, nc); break;
                        default: MI_LAUNCH((k_get_rows_q8_0_lds<TO, 9>), g, dim3(256), lb, s, a, nc); break;
                    }
                } else {
                    MI_LAUNCH((k_get_rows_q8_0<TO>), dim3(grid), dim3(256), 0, s, a);
                }
                return MI_OK;
            }
            case MI_TYPE_F32:
                MI_LAUNCH((k_get_rows_vec<MI_TYPE_F32, TO>), dim3(grid), dim3(256), 0, s, a);
                return MI_OK;
            case MI_TYPE_BF16:
                MI_LAUNCH((k_get_rows_vec<MI_TYPE_BF16, TO>), dim3(grid), dim3(256), 0, s, a);
                return MI_OK;
            default:
                MI_LAUNCH((k_get_rows_vec<MI_TYPE_F16, TO>), dim3(grid), dim3(256), 0, s, a);
                return MI_OK;
        }
    }
    MI_LAUNCH((k_get_rows_generic<TO>), dim3(grid), dim3(256), 0, s, a, ttype);
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
    bool      fast, lds = false;
    if (table.type == MI_TYPE_Q8_0) {
        // 8 outputs per lane; 16-bit aligned quants; output 16-byte stores
        fast = a.n % 8 == 0 && aligned(table.data, 2) && a.tnb1 % 2 == 0 && aligned(y.data, 16) &&
               (a.ynb1 % 16 == 0) && (8 * es_out) % 16 == 0;
        // whole rows through LDS: rows of 16-byte multiples (ne0 % 256 == 0), 16-byte aligned
        lds = fast && a.n % 256 == 0 && a.n <= 8192 && aligned(table.data, 16) && a.tnb1 % 16 == 0;
    } else {
        const int VI = 16 / type_size(table.type);
        fast         = a.n % VI == 0 && aligned(table.data, 16) && a.tnb1 % 16 == 0 && aligned(y.data, 16) &&
               a.ynb1 % 16 == 0 && (VI * es_out) % 8 == 0;
    }
    if (y.type == MI_TYPE_F32) {
        return launch_to<MI_TYPE_F32>(a, table.type, fast, lds, s);
    }
    return launch_to<MI_TYPE_BF16>(a, table.type, fast, lds, s);
}

}  // namespace mi
