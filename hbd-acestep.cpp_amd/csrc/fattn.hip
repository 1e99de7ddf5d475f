// fattn.hip -- ggml_flash_attn_ext(q, k, v, mask, scale, max_bias = 0,
// logit_softcap = 0) with GGML_PREC_F32: the DiT self/cross attention
// (dit-graph.h:227-231, 348-349) and the batched LM decode over the KV cache
// (qwen3-lm.h:706-723, reading a 256-bucketed length, qwen3-lm.h:582-596).
//
// Semantics kept from ggml-cpu's flash attention:
//   - each q row is first converted to K's vec_dot type: fp16 for F16 K, bf16
//     for BF16 K, Q8_0 (the x86 from_float: id = 127/amax, round half to even,
//     saturate; fp16 scale) for Q8_0 K; the Q8_0 dot product is then an exact
//     integer sum per block scaled by d_k*d_q;
//   - s = dot * scale + mask; a key whose mask is -inf is skipped, and the
//     bytes of one masked for every row of the wave are discarded (replaced by
//     zeros before any arithmetic), so they may hold anything, NaN included;
//   - online softmax; a row whose keys are all masked ends as 0 * (1/0) = NaN;
//   - the result is F32 [D, Nh, n_q, N] (heads of a token adjacent).
// Arithmetic is fp32 throughout (dot products via v_dot2 / v_dot4, exp,
// accumulation of the output), closer to the exact value than ggml-cpu's
// fp16 output accumulation for F16 V.
//
// Decomposition (flash-decoding): a wave owns (KV range split, sequence b,
// KV head g, block of RB query rows), where the query rows of a KV head are
// its n_q x (Nh/Nkv) (query position, head) pairs, so a K/V tile is loaded
// once for every query head that shares it (GQA). The wave walks its range
// in tiles of 32 keys: the mask values first (tiles masked for all rows are
// skipped), then all of the tile's K and V bytes with
// coalesced loads into LDS, then q.k with lane = (key, half of D) and one
// cross-half exchange, the softmax update, and p.V with lane = output
// columns. With several splits, each writes (max, sum, unnormalized output)
// to the caller's workspace and k_fa_combine merges them.
#include "launch.h"

namespace mi {

#ifndef MI_FA_WAVES_PER_CU
#define MI_FA_WAVES_PER_CU 8  // splits are chosen so the grid holds about this many waves per CU
#endif
#ifndef MI_FA_DEC_Q8_WAVES_PER_CU
#define MI_FA_DEC_Q8_WAVES_PER_CU 12  // the same for the Q8_0 decode kernel (shorter key splits pay there)
#endif

constexpr int FA_TILE = 32;  // keys per tile
constexpr int FA_MAXT = 16;  // tiles per split at most (the split's mask is staged in LDS)
constexpr int FA_MAX_SPLITS = 1024;  // splits of one key range at most (the merge keeps their weights in LDS)
// floats per row of a matrix-core split half: m, l, 2 unused, o[128] (16-byte aligned rows)
constexpr int FA_PART = 132;
constexpr int FA_SUM_T = 4;  // 64-key tiles per wave of the mask summary

template <int KT> struct FaT;
template <> struct FaT<MI_TYPE_F32> {
    static constexpr int row(int D) { return 4 * D; }
    static constexpr int cb(int) { return 16; }  // load chunk bytes
};
template <> struct FaT<MI_TYPE_F16> {
    static constexpr int row(int D) { return 2 * D; }
    static constexpr int cb(int) { return 16; }
};
template <> struct FaT<MI_TYPE_BF16> {
    static constexpr int row(int D) { return 2 * D; }
    static constexpr int cb(int) { return 16; }
};
template <> struct FaT<MI_TYPE_Q8_0> {
    static constexpr int row(int D) { return D / 32 * 34; }
    // 34-byte blocks: a row of 4k blocks is a multiple of 8 bytes (136 = 8 * 17), else of 4
    static constexpr int cb(int D) { return D % 128 == 0 ? 8 : 4; }
};

typedef _Float16 fa_f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16   fa_bf16x2 __attribute__((ext_vector_type(2)));

// x86 from_float for one 32-element block: quants into q (8 words), scale (fp16 value)
__device__ __forceinline__ float fa_q8_block(const float * x, uint32_t * qw) {
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) {
        amax = fmaxf(amax, fabsf(x[j]));
    }
    constexpr float C  = 1.0f / 127.0f;
    const float     q0 = amax * C;
    const float     d  = __builtin_fmaf(__builtin_fmaf(-q0, 127.0f, amax), C, q0);  // IEEE amax / 127
    const float     id = amax != 0.0f ? 127.0f / amax : 0.0f;
    for (int w = 0; w < 8; ++w) {
        uint32_t acc = 0;
        for (int e = 0; e < 4; ++e) {
            const float q = __builtin_amdgcn_fmed3f(__builtin_rintf(x[4 * w + e] * id), -128.0f, 127.0f);
            acc |= ((uint32_t) (int32_t) q & 0xffu) << (8 * e);
        }
        qw[w] = acc;
    }
    return (float) __builtin_bit_cast(_Float16, f32_to_f16_bits(d));
}

#ifndef MI_FA_WPE
#define MI_FA_WPE 0  // > 0: ask the compiler for at least this many waves per SIMD
#endif
#if MI_FA_WPE > 0
#define MI_FA_OCC __attribute__((amdgpu_waves_per_eu(MI_FA_WPE, 8)))
#else
#define MI_FA_OCC
#endif

// Start-up loads of the split-key kernels. Every load is issued before any
// value is used (a load under a per-element condition is waited on where it
// stands). The split's mask values in a shared mask row, one per key (lane %
// 32) of each of FA_MAXT tiles, keys clamped into the split (values of tiles
// past the split's last are never read).
__device__ __forceinline__ void fa_dec_mask(const char * mrow, int kbeg, int kend, int key, float (&ms)[FA_MAXT]) {
    if (mrow == nullptr) {
#pragma unroll
        for (int t = 0; t < FA_MAXT; ++t) {
            ms[t] = 0.0f;
        }
        return;
    }
    uint16_t hv[FA_MAXT];
#pragma unroll
    for (int t = 0; t < FA_MAXT; ++t) {
        const int k = kbeg + t * FA_TILE + key;
        hv[t]       = *(const uint16_t *) (mrow + (size_t) (k < kend ? k : kend - 1) * 2);
    }
#pragma unroll
    for (int t = 0; t < FA_MAXT; ++t) {
        ms[t] = (float) __builtin_bit_cast(_Float16, hv[t]);
    }
}

// The query row's elements 32 ks + 8 q4 + e (ks < NKS, e < 8) as floats, 0 in
// lanes past the rows (rv false; qp then points at a valid row).
template <int NKS>
__device__ __forceinline__ void fa_dec_q(const char * qp, int tq, int q4, bool rv, float (&f)[NKS][8]) {
    if (tq == MI_TYPE_F32) {
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                f[ks][e] = ((const float *) (qp + (size_t) (32 * ks + 8 * q4) * 4))[e];
            }
        }
    } else {
        uint16_t hv[NKS][8];
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                hv[ks][e] = ((const uint16_t *) (qp + (size_t) (32 * ks + 8 * q4) * 2))[e];
            }
        }
        const bool bf = tq == MI_TYPE_BF16;
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                f[ks][e] = bf ? __uint_as_float((uint32_t) hv[ks][e] << 16) : (float) __builtin_bit_cast(_Float16, hv[ks][e]);
            }
        }
    }
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            f[ks][e] = rv ? f[ks][e] : 0.0f;
        }
    }
}

template <int KT, int D, int RB>
__global__ void __launch_bounds__(64) MI_FA_OCC k_fa_split(const FaArgs a) {
    constexpr int RBYTES = FaT<KT>::row(D);
    constexpr int CB     = FaT<KT>::cb(D);
    constexpr int CPR    = RBYTES / CB;                                    // load chunks per row
    constexpr int NCH    = (FA_TILE * CPR + 63) / 64;                      // chunks per lane per tile
    constexpr int RSTR   = KT == MI_TYPE_Q8_0 ? RBYTES : RBYTES + 16;      // LDS row stride (bank spread)
    constexpr int DPL    = D / 64;                                         // output columns per lane
    constexpr int QW     = KT == MI_TYPE_Q8_0 ? D / 4 : (KT == MI_TYPE_F32 ? D : D / 2);  // q words per row
    using chunk_t        = typename std::conditional<CB == 16, uint4,
                                              typename std::conditional<CB == 8, uint2, uint32_t>::type>::type;

    __shared__ __align__(16) char     kt[FA_TILE * RSTR];
    __shared__ __align__(16) char     vt[FA_TILE * RSTR];
    __shared__ __align__(16) float    qf[RB][D];        // q rows as floats
    __shared__ __align__(16) uint32_t qs[RB][QW];       // q converted to K's dot type
    __shared__ float                  qd[RB][D / 32];    // Q8_0: per-block q scales
    __shared__ __align__(16) float    pt[FA_TILE][RB];   // the tile's probabilities
    __shared__ float                  mt[FA_MAXT * FA_TILE][RB];  // the split's mask values
    __shared__ uint64_t               lt[FA_MAXT];       // per tile: keys some row reads

    const int      lane  = threadIdx.x;
    const uint32_t split = blockIdx.x;
    const uint32_t bg    = blockIdx.y;  // b * nkv + g
    const uint32_t b     = bg / (uint32_t) a.nkv;
    const uint32_t g     = bg - b * (uint32_t) a.nkv;
    const int      r0    = blockIdx.z * RB;

    // rows of this block: (query position iq, head h); invalid rows are masked out entirely
    int  iq_of[RB], h_of[RB];
    bool rv[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        const int gr = r0 + r;
        rv[r]        = gr < a.rows;
        const int gc = rv[r] ? gr : 0;
        iq_of[r]     = gc / a.rk;
        h_of[r]      = (int) g * a.rk + (gc - iq_of[r] * a.rk);
    }

    // mask rows (per row: its query position and head)
    const char * mrow[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        mrow[r] = a.mask ? a.mask + (int64_t) (b % (uint32_t) a.mne3) * a.m3 + (int64_t) (h_of[r] % a.mne2) * a.m2 +
                               (int64_t) iq_of[r] * a.m1
                         : nullptr;
    }
    const uint32_t kb = b / (uint32_t) a.rk3;  // K/V batch index (broadcast over ne3)
    const char *   kg = a.k + (int64_t) kb * a.k3 + (int64_t) g * a.k2;
    const char *   vg = a.v + (int64_t) kb * a.v3 + (int64_t) g * a.v2;

    const int key  = lane & 31;
    const int half = lane >> 5;
    const int kbeg = (int) split * a.chunk;
    const int kend = kbeg + a.chunk < a.n_kv ? kbeg + a.chunk : a.n_kv;
    const int nt   = (kend - kbeg + FA_TILE - 1) / FA_TILE;  // tiles of this split (<= FA_MAXT)

    // the shared mask row's values for every tile of the split, issued first
    float ms[FA_MAXT];
    fa_dec_mask(a.mask != nullptr && a.mshared ? mrow[0] : nullptr, kbeg, kend, key, ms);

    // 1. q rows into LDS as floats: 16-byte loads when q's rows are 16-byte
    //    aligned (elementwise otherwise), all issued before any is used; then
    //    converted to K's dot type from LDS
    {
        constexpr int NQC = (RB * D * 4 / 16 + 63) / 64;  // 16-byte chunks per lane at most (F32 q)
        const int     es  = a.tq == MI_TYPE_F32 ? 4 : 2;
        const int     epc = 16 / es;    // elements per chunk
        const int     cpr = D / epc;    // chunks per row
        uint4         qv[NQC];
        const char *  qp[NQC];
#pragma unroll
        for (int i = 0; i < NQC; ++i) {
            const int c  = lane + 64 * i;
            const int cc = c < RB * cpr ? c : RB * cpr - 1;
            const int r  = cc / cpr;
            qp[i]        = a.q + (int64_t) b * a.q3 + (int64_t) h_of[r] * a.q2 + (int64_t) iq_of[r] * a.q1 +
                    (int64_t) (cc - r * cpr) * 16;
        }
        // the access width is tested once, outside the loads
        if (a.qvec) {
#pragma unroll
            for (int i = 0; i < NQC; ++i) {
                qv[i] = ld16(qp[i]);
            }
        } else if (es == 4) {
#pragma unroll
            for (int i = 0; i < NQC; ++i) {
                const uint32_t * w = (const uint32_t *) qp[i];
                qv[i]              = make_uint4(w[0], w[1], w[2], w[3]);
            }
        } else {
#pragma unroll
            for (int i = 0; i < NQC; ++i) {
                const uint16_t * h = (const uint16_t *) qp[i];
                qv[i]              = make_uint4((uint32_t) h[0] | ((uint32_t) h[1] << 16),
                                                (uint32_t) h[2] | ((uint32_t) h[3] << 16),
                                                (uint32_t) h[4] | ((uint32_t) h[5] << 16),
                                                (uint32_t) h[6] | ((uint32_t) h[7] << 16));
            }
        }
#pragma unroll
        for (int i = 0; i < NQC; ++i) {
            const int c = lane + 64 * i;
            if (c < RB * cpr) {
                const int r  = c / cpr;
                const int e0 = (c - r * cpr) * epc;
                float     f[8];
                if (a.tq == MI_TYPE_F32) {
                    unpack16<MI_TYPE_F32>(qv[i], f);
                } else if (a.tq == MI_TYPE_BF16) {
                    unpack16<MI_TYPE_BF16>(qv[i], f);
                } else {
                    unpack16<MI_TYPE_F16>(qv[i], f);
                }
                for (int e = 0; e < epc; ++e) {
                    qf[r][e0 + e] = rv[r] ? f[e] : 0.0f;
                }
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
    if constexpr (KT == MI_TYPE_Q8_0) {
        // one lane per (row, 32-block): the x86 from_float
        for (int t = lane; t < RB * (D / 32); t += 64) {
            const int r  = t / (D / 32);
            const int bk = t - r * (D / 32);
            qd[r][bk]    = fa_q8_block(&qf[r][bk * 32], &qs[r][bk * 8]);
        }
    } else {
        for (int t = lane; t < RB * QW; t += 64) {
            const int r = t / QW;
            const int w = t - r * QW;
            if constexpr (KT == MI_TYPE_F32) {
                qs[r][w] = __float_as_uint(qf[r][w]);
            } else {
                const float x0 = qf[r][2 * w], x1 = qf[r][2 * w + 1];
                qs[r][w]       = KT == MI_TYPE_F16 ? pack_f16x2(x0, x1) : pack_bf16x2(x0, x1);
            }
        }
    }

    float m[RB], l[RB], o[RB][DPL];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        m[r] = -INFINITY;
        l[r] = 0.0f;
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
            o[r][j] = 0.0f;
        }
    }

    // 2. the split's mask values into LDS, and per tile the set of keys some
    //    row reads (a tile no row reads is skipped). When every row of the wave
    //    uses one mask row (decode: one query position, the heads of one KV
    //    head), one value per key is loaded, for all tiles at once, before the
    //    q conversion above so that the two round trips overlap.
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
    // Per-row mask rows: the values of FA_MG tiles x RB rows are loaded together
    // (keys clamped into the split: every load is in bounds), then used.
    constexpr int FA_MG = 4;
    static_assert(FA_MAXT % FA_MG == 0, "mask tiles are loaded in groups of FA_MG");
#pragma unroll
    for (int t4 = 0; t4 < FA_MAXT; t4 += FA_MG) {
        if (t4 < nt) {
            float xs[FA_MG][RB];
            if (a.mask != nullptr && !a.mshared) {
                uint16_t hv[FA_MG][RB];
#pragma unroll
                for (int u = 0; u < FA_MG; ++u) {
                    const int k  = kbeg + (t4 + u) * FA_TILE + key;
                    const int kc = k < kend ? k : kend - 1;
#pragma unroll
                    for (int r = 0; r < RB; ++r) {
                        hv[u][r] = *(const uint16_t *) (mrow[r] + (size_t) kc * 2);
                    }
                }
#pragma unroll
                for (int u = 0; u < FA_MG; ++u) {
#pragma unroll
                    for (int r = 0; r < RB; ++r) {
                        xs[u][r] = (float) __builtin_bit_cast(_Float16, hv[u][r]);
                    }
                }
            } else {
#pragma unroll
                for (int u = 0; u < FA_MG; ++u) {
#pragma unroll
                    for (int r = 0; r < RB; ++r) {
                        xs[u][r] = a.mask != nullptr ? ms[t4 + u] : 0.0f;
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < FA_MG; ++u) {
                const int t = t4 + u;
                if (t < nt) {
                    const int  t0  = kbeg + t * FA_TILE;
                    const bool ok  = t0 + key < kend;
                    bool       any = false;
#pragma unroll
                    for (int r = 0; r < RB; ++r) {
                        const float x = ok && rv[r] ? xs[u][r] : -INFINITY;
                        if (half == 0) {
                            mt[t * FA_TILE + key][r] = x;
                        }
                        any = any || x != -INFINITY;
                    }
                    const uint64_t lv = __builtin_amdgcn_ballot_w64(any && half == 0);  // bit k: key k is read
                    if (lane == 0) {
                        lt[t] = lv;
                    }
                }
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();

    // 3. K/V tiles, software pipelined: the registers of tile t are staged in
    //    LDS, then receive tile t+1's loads while tile t is computed
    chunk_t kc[NCH], vc[NCH];
    // Every lane loads all of its chunks from a row clamped into the tile (no
    // branches); in a tile with unread keys (masked for every row, or past the
    // end) their chunks are then replaced by zeros, so their bytes never reach
    // the sums. Offsets within a tile fit 32 bits; the tile base is uniform.
    auto load_kv = [&](int t0, uint64_t live) {
        const int    nk  = kend - t0 < FA_TILE ? kend - t0 : FA_TILE;
        const char * kgt = kg + (int64_t) t0 * a.k1;
        const char * vgt = vg + (int64_t) t0 * a.v1;
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const int      c  = lane + 64 * i < FA_TILE * CPR ? lane + 64 * i : FA_TILE * CPR - 1;
            const int      kk = c / CPR < nk ? c / CPR : nk - 1;
            const uint32_t pp = (uint32_t) (c % CPR) * CB;
            const uint32_t ko = (uint32_t) kk * (uint32_t) a.k1 + pp;
            const uint32_t vo = (uint32_t) kk * (uint32_t) a.v1 + pp;
            if constexpr (CB == 16) {
                kc[i] = ld16(kgt + ko);
                vc[i] = ld16(vgt + vo);
            } else {
                kc[i] = *(const chunk_t *) (kgt + ko);
                vc[i] = *(const chunk_t *) (vgt + vo);
            }
        }
        if (live != 0xffffffffull) {
#pragma unroll
            for (int i = 0; i < NCH; ++i) {
                const int  c    = lane + 64 * i;
                const bool keep = c < FA_TILE * CPR && ((live >> (c / CPR)) & 1);
                if (!keep) {
                    kc[i] = chunk_t{};
                    vc[i] = chunk_t{};
                }
            }
        }
    };
    uint64_t live = nt > 0 ? lt[0] : 0;
    if (live) {
        load_kv(kbeg, live);
    }
    for (int t = 0; t < nt; ++t) {
        const int t0 = kbeg + t * FA_TILE;
        const uint64_t next = t + 1 < nt ? lt[t + 1] : 0;
        if (live) {
#pragma unroll
            for (int i = 0; i < NCH; ++i) {
                const int c = lane + 64 * i;
                if (c < FA_TILE * CPR) {
                    const int kk = c / CPR;
                    const int pp = c - kk * CPR;
                    *(chunk_t *) (kt + kk * RSTR + pp * CB) = kc[i];
                    *(chunk_t *) (vt + kk * RSTR + pp * CB) = vc[i];
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            __builtin_amdgcn_wave_barrier();
        }
        if (next) {
            load_kv(t0 + FA_TILE, next);  // in flight during this tile's math
        }
        if (live) {
            // 4. s = q.k for (row, key): lane = (key, half of D)
            float s[RB];
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                s[r] = 0.0f;
            }
            const char * kr = kt + key * RSTR;
            if constexpr (KT == MI_TYPE_Q8_0) {
                constexpr int NBH = D / 64;  // blocks per half
#pragma unroll
                for (int bb = 0; bb < NBH; ++bb) {
                    const int        bk = half * NBH + bb;
                    const uint16_t * bp = (const uint16_t *) (kr + 34 * bk);
                    const float      dk = (float) __builtin_bit_cast(_Float16, bp[0]);
                    uint32_t         kw[8];
#pragma unroll
                    for (int w = 0; w < 8; ++w) {
                        kw[w] = (uint32_t) bp[1 + 2 * w] | ((uint32_t) bp[2 + 2 * w] << 16);
                    }
#pragma unroll
                    for (int r = 0; r < RB; ++r) {
                        int sumi = 0;
#pragma unroll
                        for (int w = 0; w < 8; ++w) {
                            sumi = __builtin_amdgcn_sdot4((int) kw[w], (int) qs[r][bk * 8 + w], sumi, false);
                        }
                        s[r] = __builtin_fmaf(dk * qd[r][bk], (float) sumi, s[r]);
                    }
                }
            } else {
                constexpr int WH = QW / 2;  // words per half
                const uint4 * k4 = (const uint4 *) (kr + half * (RBYTES / 2));
#pragma unroll
                for (int c4 = 0; c4 < WH / 4; ++c4) {
                    const uint4    kv    = k4[c4];
                    const uint32_t kw[4] = { kv.x, kv.y, kv.z, kv.w };
#pragma unroll
                    for (int r = 0; r < RB; ++r) {
                        const uint4    qv    = *(const uint4 *) &qs[r][half * WH + 4 * c4];
                        const uint32_t qw[4] = { qv.x, qv.y, qv.z, qv.w };
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            if constexpr (KT == MI_TYPE_F16) {
                                s[r] = __builtin_amdgcn_fdot2(__builtin_bit_cast(fa_f16x2, kw[e]),
                                                              __builtin_bit_cast(fa_f16x2, qw[e]), s[r], false);
                            } else if constexpr (KT == MI_TYPE_BF16) {
                                s[r] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(fa_bf16x2, kw[e]),
                                                                       __builtin_bit_cast(fa_bf16x2, qw[e]), s[r],
                                                                       false);
                            } else {
                                s[r] = __builtin_fmaf(__uint_as_float(kw[e]), __uint_as_float(qw[e]), s[r]);
                            }
                        }
                    }
                    // bound the scheduler's look-ahead: hoisting every row's q words
                    // for the whole dot product would cost 4 x D/4 registers
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            // 5. full dot (both halves), scale, mask; online softmax update per row
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                const float full  = s[r] + __shfl_xor(s[r], 32, 64);
                const float mvr   = mt[t * FA_TILE + key][r];
                const float x     = mvr == -INFINITY ? -INFINITY : full * a.scale + mvr;
                const float tmax  = group_max<32>(x);
                const float mn    = fmaxf(m[r], tmax);
                float       alpha = 1.0f, p = 0.0f;
                if (mn != -INFINITY) {
                    alpha = __expf(m[r] - mn);  // exp(-inf) = 0 on the first live tile
                    p     = x == -INFINITY ? 0.0f : __expf(x - mn);
                }
                m[r] = mn;
                l[r] = l[r] * alpha + (half == 0 ? p : 0.0f);
#pragma unroll
                for (int j = 0; j < DPL; ++j) {
                    o[r][j] *= alpha;
                }
                if (half == 0) {
                    pt[key][r] = p;
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            __builtin_amdgcn_wave_barrier();

            // 6. o += p.V, lane = output columns [lane*DPL, +DPL). Keys no row reads
            //    (and keys past the end) have p = 0 and zero V bytes in LDS, so the
            //    loop runs over the whole tile without a branch.
#pragma unroll 8
            for (int kk = 0; kk < FA_TILE; ++kk) {
                float pr[RB];
#pragma unroll
                for (int r4 = 0; r4 < RB; r4 += 4) {
                    const float4 p4 = *(const float4 *) &pt[kk][r4];
                    pr[r4]          = p4.x;
                    pr[r4 + 1]      = p4.y;
                    pr[r4 + 2]      = p4.z;
                    pr[r4 + 3]      = p4.w;
                }
                float        vv[DPL];
                const char * vr = vt + kk * RSTR;
                if constexpr (KT == MI_TYPE_Q8_0) {
                    const int      c0 = lane * DPL;
                    const char *   bp = vr + 34 * (c0 / 32);
                    const float    dv = (float) __builtin_bit_cast(_Float16, *(const uint16_t *) bp);
                    const int8_t * qp = (const int8_t *) (bp + 2 + (c0 % 32));
#pragma unroll
                    for (int j = 0; j < DPL; ++j) {
                        vv[j] = (float) qp[j] * dv;
                    }
                } else if constexpr (KT == MI_TYPE_F32) {
#pragma unroll
                    for (int j = 0; j < DPL; ++j) {
                        vv[j] = ((const float *) vr)[lane * DPL + j];
                    }
                } else {
                    const uint16_t * hp = (const uint16_t *) vr + lane * DPL;
#pragma unroll
                    for (int j = 0; j < DPL; ++j) {
                        vv[j] = KT == MI_TYPE_F16 ? (float) __builtin_bit_cast(_Float16, hp[j])
                                                  : __uint_as_float((uint32_t) hp[j] << 16);
                    }
                }
#pragma unroll
                for (int r = 0; r < RB; ++r) {
#pragma unroll
                    for (int j = 0; j < DPL; ++j) {
                        o[r][j] = __builtin_fmaf(pr[r], vv[j], o[r][j]);
                    }
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            __builtin_amdgcn_wave_barrier();  // the next tile overwrites kt, vt, pt
        }
        live = next;
    }

    // 7. row sums across lanes; the final output or this split's partial
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        l[r] = group_sum<64>(l[r]);
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        if (!rv[r]) {
            continue;
        }
        if (a.splits == 1) {
            const float inv = 1.0f / l[r];  // all keys masked: 0 * inf = NaN, as ggml
            float *     yp  = (float *) (a.y + (int64_t) b * a.y3 + (int64_t) iq_of[r] * a.y2 + (int64_t) h_of[r] * a.y1);
#pragma unroll
            for (int j = 0; j < DPL; ++j) {
                yp[lane * DPL + j] = o[r][j] * inv;
            }
        } else {
            float * wp = a.ws + (((int64_t) split * a.nb * a.nkv + bg) * a.rows + r0 + r) * (D + 2);
            if (lane == 0) {
                wp[0] = m[r];
                wp[1] = l[r];
            }
#pragma unroll
            for (int j = 0; j < DPL; ++j) {
                wp[2 + lane * DPL + j] = o[r][j];
            }
        }
    }
}

// Merge the splits of one (sequence, KV head, row): y = sum_s w_s o_s / sum_s w_s l_s,
// w_s = exp(m_s - max_s m_s) (0 for a split whose keys were all masked). A
// workgroup of 256 threads per row: every split's (m, l) loaded at once, the
// weights in LDS; thread t accumulates one 16-byte column chunk over the
// splits s = t / (D/4) (mod 256 / (D/4)), and the partial sums are added
// through LDS. With at most FA_CMB_PRE splits per thread (the usual case) the
// column chunks are loaded together with the (m, l) pairs, before the weights
// are known, so the merge waits for one round of loads; indexes past the last
// split are clamped to it and their weight is 0.
constexpr int FA_CMB_PRE = 8;
template <int D>
__global__ void __launch_bounds__(256) k_fa_combine(const FaArgs a) {
    constexpr int  C4  = D / 4;    // float4 chunks per output row
    constexpr int  SG  = 256 / C4; // split groups
    __shared__ float wsh[FA_MAX_SPLITS];
    __shared__ float red[8];
    __shared__ __align__(16) float4 part[SG][C4];

    const int      tid  = threadIdx.x;
    const uint32_t rec  = blockIdx.x;  // bg * rows + row
    const uint32_t bg   = rec / (uint32_t) a.rows;
    const int      row  = (int) (rec - bg * (uint32_t) a.rows);
    const uint32_t b    = bg / (uint32_t) a.nkv;
    const uint32_t g    = bg - b * (uint32_t) a.nkv;
    const int      iq   = row / a.rk;
    const int      h    = (int) g * a.rk + (row - iq * a.rk);
    const int64_t  sstr = (int64_t) a.nb * a.nkv * a.rows * (D + 2);  // one split's records
    const float *  w0   = a.ws + (int64_t) rec * (D + 2);
    const int      c    = tid % C4;
    const int      sg   = tid / C4;
    const int      last = a.splits - 1;

    const bool pre = a.splits <= SG * FA_CMB_PRE;
    float4     pv[FA_CMB_PRE];
    if (pre) {
#pragma unroll
        for (int j = 0; j < FA_CMB_PRE; ++j) {
            const int s = sg + SG * j;
            pv[j]       = *(const float4 *) (w0 + (int64_t) (s < last ? s : last) * sstr + 2 + 4 * c);
        }
    }
    // pass 1: max over the splits, weights, weighted sum of the row sums
    float ml[FA_MAX_SPLITS / 256], ll[FA_MAX_SPLITS / 256];
    float mloc = -INFINITY;
#pragma unroll
    for (int i = 0; i < FA_MAX_SPLITS / 256; ++i) {
        const int     s  = tid + 256 * i;
        const float * mp = w0 + (int64_t) (s < last ? s : last) * sstr;
        ml[i]            = mp[0];
        ll[i]            = mp[1];
        ml[i]            = s <= last ? ml[i] : -INFINITY;
        mloc             = fmaxf(mloc, ml[i]);
    }
    mloc = group_max<64>(mloc);
    if ((tid & 63) == 0) {
        red[tid >> 6] = mloc;
    }
    __syncthreads();
    const float mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float       lw = 0.0f;
#pragma unroll
    for (int i = 0; i < FA_MAX_SPLITS / 256; ++i) {
        const int   s = tid + 256 * i;
        const float w = ml[i] == -INFINITY ? 0.0f : __expf(ml[i] - mx);
        if (s <= last) {
            wsh[s] = w;
        }
        lw = __builtin_fmaf(w, ll[i], lw);
    }
    lw = group_sum<64>(lw);
    if ((tid & 63) == 0) {
        red[4 + (tid >> 6)] = lw;
    }
    __syncthreads();
    const float L = (red[4] + red[5]) + (red[6] + red[7]);

    // pass 2: weighted outputs
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (pre) {
#pragma unroll
        for (int j = 0; j < FA_CMB_PRE; ++j) {
            const int s = sg + SG * j;
            if (s <= last) {
                const float  w = wsh[s];
                const float4 v = pv[j];
                acc.x          = __builtin_fmaf(w, v.x, acc.x);
                acc.y          = __builtin_fmaf(w, v.y, acc.y);
                acc.z          = __builtin_fmaf(w, v.z, acc.z);
                acc.w          = __builtin_fmaf(w, v.w, acc.w);
            }
        }
    } else {
#pragma unroll 8
        for (int s = sg; s < a.splits; s += SG) {
            const float  w = wsh[s];
            const float4 v = *(const float4 *) (w0 + s * sstr + 2 + 4 * c);
            acc.x          = __builtin_fmaf(w, v.x, acc.x);
            acc.y          = __builtin_fmaf(w, v.y, acc.y);
            acc.z          = __builtin_fmaf(w, v.z, acc.z);
            acc.w          = __builtin_fmaf(w, v.w, acc.w);
        }
    }
    part[sg][c] = acc;
    __syncthreads();
    if (tid < C4) {
        float4 t = part[0][tid];
#pragma unroll
        for (int q = 1; q < SG; ++q) {
            const float4 u = part[q][tid];
            t.x += u.x;
            t.y += u.y;
            t.z += u.z;
            t.w += u.w;
        }
        const float inv = 1.0f / L;  // all keys masked: 0 * inf = NaN, as ggml
        float *     yp  = (float *) (a.y + (int64_t) b * a.y3 + (int64_t) iq * a.y2 + (int64_t) h * a.y1);
        yp[4 * tid]     = t.x * inv;
        yp[4 * tid + 1] = t.y * inv;
        yp[4 * tid + 2] = t.z * inv;
        yp[4 * tid + 3] = t.w * inv;
    }
}

// ---------------------------------------------------------------------------
// Matrix-core path (prefill: many query rows; F16/BF16 K and V; D = 128).
// A workgroup of 4 waves owns 128 query rows of one (sequence, KV head) -- the
// rows are (query position, head) pairs, so the query heads sharing the KV
// head share the workgroup -- and walks all keys in tiles of 64, K and V
// double-buffered in LDS (both row-major; V read transposed). Per wave and tile:
//   S^T = K Q^T   (v_mfma_f32_32x32x16: keys x 32 rows, q converted to K's
//                  type as ggml converts it; products exact, fp32 sums)
//   softmax       (lane-local: a lane holds 32 keys of one row, the other
//                  half-wave the other 32; one exchange per tile)
//   O^T += V^T P^T with P split into a high and a low 16-bit part (two
//                  MFMAs), so P keeps ~16 (BF16) / ~22 (F16) significant bits
// S^T and O^T put a query row in one lane column, so every row statistic
// (max, sum, rescale) stays in the lane. Lane layout of the 32x32x16 MFMA
// (checked on the device): A lane l = row l%32, k = 8*(l/32)+i; B lane l =
// column l%32, same k; D lane l = column l%32, row 8j + 4*(l/32) + i at 4j+i.
// Keys whose mask is -inf get p = 0 (their K/V bytes are multiplied, so they
// must be finite, as every activation the reference feeds here is).
// Q8_0 K and V (the same walk, tiles of 64 keys):
//   S^T           per 32-element block: v_mfma_i32_32x32x32_i8 of the K quants
//                 (LDS) and q converted to Q8_0 with the x86 quantizer (exact
//                 int32 block dots), and the block's d_k d_q as an fp16 outer
//                 product on the matrix core (exact); s = the four scaled dots
//                 summed by a chain of fmas in block order
//   V             dequantized once per tile into LDS: V' = q d_v exactly, as a
//                 bf16 high part RN(V') and an f16 low part V' - RN(V') (exact:
//                 at most 10 significant bits on the fp16 grid), so V' is held
//                 exactly for every finite d_v
//   O^T += V^T P^T as three MFMAs: bf16 high x (P high + P low), f16 low x P
//                 rounded to f16; P keeps ~16 bits against V's high part
// ---------------------------------------------------------------------------
#ifndef MI_FA_DEC
#define MI_FA_DEC 1  // decode (one query position, <= 16 heads per KV head) on the 16x16 matrix cores
#endif
#ifndef MI_FA_MFMA_Q8
#define MI_FA_MFMA_Q8 1  // prefill over Q8_0 K/V on the matrix cores (else the split path)
#endif
#ifndef MI_FA_MFMA_MIN_ROWS
#define MI_FA_MFMA_MIN_ROWS 64  // (query position, head) rows per KV head from which the MFMA path is used
#endif

// transposed LDS reads of 16-bit elements (gfx950 ds_read_b64_tr_b16)
typedef short fa_v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) fa_v4s fa_lds_v4s;

template <int KT> struct FaM;
template <> struct FaM<MI_TYPE_BF16> {
    typedef __bf16 e;
    typedef __bf16 x8 __attribute__((ext_vector_type(8)));
    static __device__ __forceinline__ uint16_t bits(float v) { return f32_to_bf16_bits(v); }
    static __device__ __forceinline__ float    val(uint16_t h) { return __uint_as_float((uint32_t) h << 16); }
};
template <> struct FaM<MI_TYPE_F16> {
    typedef _Float16 e;
    typedef _Float16 x8 __attribute__((ext_vector_type(8)));
    static __device__ __forceinline__ uint16_t bits(float v) { return f32_to_f16_bits(v); }
    static __device__ __forceinline__ float    val(uint16_t h) { return (float) __builtin_bit_cast(_Float16, h); }
};
typedef float fa_f32x16 __attribute__((ext_vector_type(16)));

template <int KT>
__device__ __forceinline__ fa_f32x16 fa_mma(const typename FaM<KT>::x8 & a, const typename FaM<KT>::x8 & b,
                                            const fa_f32x16 & c) {
    if constexpr (KT == MI_TYPE_BF16) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
}

// Decode on the matrix cores (F16/BF16 K and V, D = 128, one query position,
// at most 16 query heads per KV head, a mask row shared by every head). A wave
// owns (key split, sequence, KV head) as k_fa_split does and walks 32-key tiles,
// the mask's dead tiles skipped before any K/V byte is read, the next tile's
// loads in flight under the current one's math. With v_mfma_f32_16x16x32
// (lane l: A[l%16][8(l/16)+e], B[8(l/16)+e][l%16], C[4(l/16)+r][l%16]):
//   S^T = K Q^T: A = K rows from LDS, B = the query heads (padded to 16) in K's
//   type; lane l then holds the scores of head l%16 for keys 16 mt + 4 (l/16) + r.
//   O^T += V^T P^T: B = those 8 probabilities as they sit (a high and a low
//   16-bit part, two MFMAs); A = V^T in that key order, read from the row-major V
//   tile in LDS with two transposed reads (keys 4 q + r, then 16 + 4 q + r).
// Keys no head reads (masked, past the end) have p = 0 and zero K/V bytes in
// LDS, whatever the cache holds there. Partials and the merge are k_fa_split's.
#ifndef MI_FA_DEC_WPE
#define MI_FA_DEC_WPE 0  // > 0: ask the compiler for at least this many waves per SIMD
#endif
#if MI_FA_DEC_WPE > 0
#define MI_FA_DEC_OCC __attribute__((amdgpu_waves_per_eu(MI_FA_DEC_WPE, 8)))
#else
#define MI_FA_DEC_OCC
#endif
template <int KT>
__global__ void __launch_bounds__(64) MI_FA_DEC_OCC k_fa_dec(const FaArgs a) {
    using M          = FaM<KT>;
    using x8         = typename M::x8;
    constexpr int D   = 128;
    constexpr int T   = FA_TILE;       // keys per tile
    constexpr int VR  = D * 2 + 32;    // V row stride (bytes): 8 rows on distinct banks for transposed reads
    constexpr int NKS = D / 32;        // k-steps of S (32 dims each)
    constexpr int NDT = D / 16;        // 16-dim tiles of O^T
    constexpr int KC  = T * D * 2 / 16 / 64;  // 16-byte K chunks per lane per tile (8)
    constexpr int VC  = KC / 2;               // V key-pair chunks per lane per tile (4)
    typedef float f4 __attribute__((ext_vector_type(4)));

    __shared__ __align__(16) char vt[T * VR];       // the tile's V rows (row-major)
    __shared__ float              mt[FA_MAXT * T];  // the split's mask values
    __shared__ uint32_t           lt[FA_MAXT];      // per tile: keys some head reads

    const int      lane  = threadIdx.x;
    const int      c16   = lane & 15, q4 = lane >> 4;
    const uint32_t split = blockIdx.x;
    const uint32_t bg    = blockIdx.y;
    const uint32_t b     = bg / (uint32_t) a.nkv;
    const uint32_t g     = bg - b * (uint32_t) a.nkv;
    const bool     rv    = c16 < a.rows;
    const int      h     = (int) g * a.rk + (rv ? c16 : 0);
    const uint32_t kb    = b / (uint32_t) a.rk3;
    const char *   kg    = a.k + (int64_t) kb * a.k3 + (int64_t) g * a.k2;
    const char *   vg    = a.v + (int64_t) kb * a.v3 + (int64_t) g * a.v2;
    const char *   mrow  = a.mask ? a.mask + (int64_t) (b % (uint32_t) a.mne3) * a.m3 : nullptr;
    const int      kbeg  = (int) split * a.chunk;
    const int      kend  = kbeg + a.chunk < a.n_kv ? kbeg + a.chunk : a.n_kv;
    const int      nt    = (kend - kbeg + T - 1) / T;
    const int      key   = lane & 31;

    // the split's mask values (one per key) and the query row, issued first
    float ms[FA_MAXT];
    fa_dec_mask(mrow, kbeg, kend, key, ms);
    float qf[NKS][8];
    fa_dec_q<NKS>(a.q + (int64_t) b * a.q3 + (int64_t) h * a.q2, a.tq, q4, rv, qf);
    // Q^T operands: k-step ks holds q[head c16][32 ks + 8 q4 + e] in K's type (RNE)
    x8 qb[NKS];
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            qb[ks][e] = __builtin_bit_cast(typename M::e, M::bits(qf[ks][e]));
        }
    }
    // mask values into LDS and per tile the keys some head reads (the mask row is
    // every head's, so a masked key is masked for all of them)
#pragma unroll
    for (int t = 0; t < FA_MAXT; ++t) {
        if (t < nt) {
            const int   k0 = kbeg + t * T + key;
            const float x  = k0 < kend ? ms[t] : -INFINITY;
            if (lane < 32) {
                mt[t * T + key] = x;
            }
            const uint64_t lv = __builtin_amdgcn_ballot_w64(lane < 32 && x != -INFINITY);
            if (lane == 0) {
                lt[t] = (uint32_t) lv;
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();

    // K goes straight into the S MFMAs' A operands: lane (c16, q4) of k-step ks
    // holds K[key 16 mt + c16][32 ks + 8 q4 .. + 7] (a masked key's score is
    // replaced by -inf, whatever its bytes). V chunk i: keys 2 m and 2 m + 1,
    // m = 4 i + lane / 16, the same 16-byte part of both; unread keys' V bytes
    // are replaced by zeros. Keys are clamped into the split.
    x8    ka[2][NKS];
    uint4 vc[2 * VC];
    auto  load_k = [&](int t0) {
        const int nk = kend - t0 < T ? kend - t0 : T;
#pragma unroll
        for (int mt2 = 0; mt2 < 2; ++mt2) {
            const int kk = 16 * mt2 + c16;
            const int kr = kk < nk ? kk : nk - 1;
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
                ka[mt2][ks] = __builtin_bit_cast(x8, ld16(kg + (int64_t) (t0 + kr) * a.k1 + (32 * ks + 8 * q4) * 2));
            }
        }
    };
    auto load_v = [&](int t0, uint32_t live) {
        const int nk = kend - t0 < T ? kend - t0 : T;
#pragma unroll
        for (int i = 0; i < VC; ++i) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int kk = 2 * (4 * i + q4) + j;
                const int kr = kk < nk ? kk : nk - 1;
                vc[2 * i + j] = ld16(vg + (int64_t) (t0 + kr) * a.v1 + c16 * 16);
                if (!((live >> kk) & 1u)) {
                    vc[2 * i + j] = make_uint4(0, 0, 0, 0);
                }
            }
        }
    };

    f4 o[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
        o[dt] = f4{ 0.0f, 0.0f, 0.0f, 0.0f };
    }
    float    mrun = -INFINITY, lrun = 0.0f;
    uint32_t live = nt > 0 ? lt[0] : 0u;
    if (live) {
        load_k(kbeg);
        load_v(kbeg, live);
    }
    for (int t = 0; t < nt; ++t) {
        const int      t0   = kbeg + t * T;
        const uint32_t next = t + 1 < nt ? lt[t + 1] : 0u;
        if (live) {
#pragma unroll
            for (int i = 0; i < VC; ++i) {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    *(uint4 *) (vt + (2 * (4 * i + q4) + j) * VR + c16 * 16) = vc[2 * i + j];
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            __builtin_amdgcn_wave_barrier();
        }
        if (next) {
            load_v(t0 + T, next);  // in flight during this tile's math
        }
        f4 s[2] = { f4{ 0.0f, 0.0f, 0.0f, 0.0f }, f4{ 0.0f, 0.0f, 0.0f, 0.0f } };
        if (live) {
            // S^T for keys 16 mt + [0, 16) x the 16 (padded) heads
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
#pragma unroll
                for (int mt2 = 0; mt2 < 2; ++mt2) {
                    if constexpr (KT == MI_TYPE_BF16) {
                        s[mt2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[mt2][ks], qb[ks], s[mt2], 0, 0, 0);
                    } else {
                        s[mt2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[mt2][ks], qb[ks], s[mt2], 0, 0, 0);
                    }
                }
            }
        }
        if (next) {
            load_k(t0 + T);  // the A operands are free once this tile's S is issued
        }
        if (live) {
            // softmax: this lane's 8 keys of head c16, then the other 24 in lanes ^ 16, ^ 32
            float x[8];
            float tmax = -INFINITY;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int   kk = 16 * (e >> 2) + 4 * q4 + (e & 3);
                const float mv = mt[t * T + kk];
                x[e]           = mv == -INFINITY ? -INFINITY : s[e >> 2][e & 3] * a.scale + mv;
                tmax           = fmaxf(tmax, x[e]);
            }
            tmax           = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
            tmax           = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
            const float mn = fmaxf(mrun, tmax);
            float       alpha = 1.0f;
            x8          phi, plo;
            float       psum = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float    p  = mn == -INFINITY || x[e] == -INFINITY ? 0.0f : __expf(x[e] - mn);
                const uint16_t hb = M::bits(p);
                psum += p;
                phi[e] = __builtin_bit_cast(typename M::e, hb);
                plo[e] = __builtin_bit_cast(typename M::e, M::bits(p - M::val(hb)));
            }
            if (mn != -INFINITY) {
                alpha = __expf(mrun - mn);  // exp(-inf) = 0 on the first live tile
            }
            mrun = mn;
            lrun = lrun * alpha + psum;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
                o[dt] *= alpha;
            }
            // O^T += V^T P^T: A = V^T row 16 dt + c16 at keys 4 q4 + r and 16 + 4 q4 + r
            // (P's order), by two transposed reads of the row-major tile: lane m of a
            // 16-lane group addresses V[K0 + m / 4][D0 + 4 (m % 4)], and lane j receives
            // V[K0 .. K0 + 3][D0 + j]
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
                const char *  vp = vt + (4 * q4 + c16 / 4) * VR + (16 * dt + 4 * (c16 & 3)) * 2;
                const fa_v4s  v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((fa_lds_v4s *) vp);             // keys 4 q4 + r
                const fa_v4s  v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((fa_lds_v4s *) (vp + 16 * VR));  // keys 16 + 4 q4 + r
                const x8      va = __builtin_bit_cast(x8, __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7));
                if constexpr (KT == MI_TYPE_BF16) {
                    o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, phi, o[dt], 0, 0, 0);
                    o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, plo, o[dt], 0, 0, 0);
                } else {
                    o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, phi, o[dt], 0, 0, 0);
                    o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, plo, o[dt], 0, 0, 0);
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            __builtin_amdgcn_wave_barrier();  // the next tile overwrites vt
        }
        live = next;
    }

    // the head's sum over its 4 lanes; lane (c16, q4) holds O^T[16 dt + 4 q4 + r][c16]
    lrun += __shfl_xor(lrun, 16, 64);
    lrun += __shfl_xor(lrun, 32, 64);
    if (!rv) {
        return;
    }
    if (a.splits == 1) {
        const float inv = 1.0f / lrun;  // all keys masked: 0 * inf = NaN, as ggml
        float *     yp  = (float *) (a.y + (int64_t) b * a.y3 + (int64_t) h * a.y1);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                yp[16 * dt + 4 * q4 + r] = o[dt][r] * inv;
            }
        }
    } else {
        float * wp = a.ws + (((int64_t) split * a.nb * a.nkv + bg) * a.rows + c16) * (D + 2);
        if (q4 == 0) {
            wp[0] = mrun;
            wp[1] = lrun;
        }
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                wp[2 + 16 * dt + 4 * q4 + r] = o[dt][r];
            }
        }
    }
}

// Decode on the matrix cores over a Q8_0 cache (D = 128, one query position,
// at most 16 query heads per KV head, a mask row shared by every head): the
// decomposition of k_fa_dec (a wave per key split, sequence and KV head; dead
// tiles skipped before any K/V byte is read; the next tile's loads in flight)
// with the Q8_0 arithmetic of k_fa_split:
//   S^T = K Q^T block by block with v_mfma_i32_16x16x32_i8 (lane l: A[l%16]
//   [8(l/16)+e], B[8(l/16)+e][l%16], C[4(l/16)+r][l%16]; checked on the
//   device): A = 8 quants of key 16 mt + c16 read from the tile's raw rows in
//   LDS (2-byte aligned 8-byte reads), B = q converted to Q8_0 with the x86
//   quantizer as it sits in the lane (head c16, elements 32 kb + 8 q4 + e). The
//   exact int32 block dots are scaled as k_fa_split scales them (fma(d_k *
//   d_q, dot, s), blocks 0-1 and 2-3 summed apart, then added), so the scores
//   equal its scores.
//   O^T += V^T P^T per 32-column block b of V: B = p * d_v[key][b] (rounded
//   once) as a high and a low bf16 part; A = the V tile's quants as bf16
//   (exact), row-major in LDS and read transposed as in k_fa_dec. l sums p.
// Keys no head reads get p = 0 and d_v = 0, so their bytes (integers, or a
// NaN scale) never reach the output.
#ifndef MI_FA_DEC_Q8
#define MI_FA_DEC_Q8 1  // Q8_0 caches take k_fa_dec_q8 (else the split path)
#endif
__global__ void __launch_bounds__(64) MI_FA_DEC_OCC k_fa_dec_q8(const FaArgs a) {
    typedef __bf16 x8 __attribute__((ext_vector_type(8)));
    typedef float  f4 __attribute__((ext_vector_type(4)));
    typedef int    i4 __attribute__((ext_vector_type(4)));
    constexpr int D   = 128;
    constexpr int T   = FA_TILE;                // keys per tile
    constexpr int NB  = D / 32;                 // Q8_0 blocks per row
    constexpr int RB  = NB * 34;                // bytes per cache row (136)
    constexpr int VR  = D * 2 + 32;             // bf16 V row stride (bytes), as k_fa_dec
    constexpr int NDT = D / 16;                 // 16-dim tiles of O^T

    __shared__ __align__(16) char  kraw[T * RB];  // the tile's K rows as stored (136-byte rows)
    __shared__ __align__(16) char  vt[T * VR];    // V quants as bf16, row-major
    __shared__ __align__(16) float dks[NB][T];    // K block scales [block][key]
    __shared__ __align__(16) float dvs[NB][T];    // V block scales, 0 for keys no head reads
    __shared__ float               mt[FA_MAXT * T];
    __shared__ uint32_t            lt[FA_MAXT];

    const int      lane  = threadIdx.x;
    const int      c16   = lane & 15, q4 = lane >> 4;
    const uint32_t split = blockIdx.x;
    const uint32_t bg    = blockIdx.y;
    const uint32_t b     = bg / (uint32_t) a.nkv;
    const uint32_t g     = bg - b * (uint32_t) a.nkv;
    const bool     rv    = c16 < a.rows;
    const int      h     = (int) g * a.rk + (rv ? c16 : 0);
    const uint32_t kb3   = b / (uint32_t) a.rk3;
    const char *   kg    = a.k + (int64_t) kb3 * a.k3 + (int64_t) g * a.k2;
    const char *   vg    = a.v + (int64_t) kb3 * a.v3 + (int64_t) g * a.v2;
    const char *   mrow  = a.mask ? a.mask + (int64_t) (b % (uint32_t) a.mne3) * a.m3 : nullptr;
    const int      kbeg  = (int) split * a.chunk;
    const int      kend  = kbeg + a.chunk < a.n_kv ? kbeg + a.chunk : a.n_kv;
    const int      nt    = (kend - kbeg + T - 1) / T;
    const int      key   = lane & 31;

    // the split's mask values (one per key) and the query row, issued first
    float ms[FA_MAXT];
    fa_dec_mask(mrow, kbeg, kend, key, ms);
    float qf[NB][8];
    fa_dec_q<NB>(a.q + (int64_t) b * a.q3 + (int64_t) h * a.q2, a.tq, q4, rv, qf);
    // q converted to Q8_0 (x86 from_float, as fa_q8_block): lane (c16, q4) holds
    // elements 32 kb + 8 q4 + e of head c16, so each block's amax is a max over
    // lanes c16 + 16 q4; B operand of block kb = its 8 quants, d_q its scale
    long  qb8[NB];
    float dq[NB];
    {
#pragma unroll
        for (int kb = 0; kb < NB; ++kb) {
            const float * f    = qf[kb];
            float         amax = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                amax = fmaxf(amax, fabsf(f[e]));
            }
            amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
            amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
            constexpr float C  = 1.0f / 127.0f;
            const float     q0 = amax * C;
            const float     d  = __builtin_fmaf(__builtin_fmaf(-q0, 127.0f, amax), C, q0);  // IEEE amax / 127
            const float     id = amax != 0.0f ? 127.0f / amax : 0.0f;
            uint64_t        w  = 0;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float q = __builtin_amdgcn_fmed3f(__builtin_rintf(f[e] * id), -128.0f, 127.0f);
                w |= (uint64_t) ((uint32_t) (int32_t) q & 0xffu) << (8 * e);
            }
            qb8[kb] = (long) w;
            dq[kb]  = (float) __builtin_bit_cast(_Float16, f32_to_f16_bits(d));
        }
    }
    // mask values into LDS and per tile the keys some head reads
#pragma unroll
    for (int t = 0; t < FA_MAXT; ++t) {
        if (t < nt) {
            const int   k0 = kbeg + t * T + key;
            const float x  = k0 < kend ? ms[t] : -INFINITY;
            if (lane < 32) {
                mt[t * T + key] = x;
            }
            const uint64_t lv = __builtin_amdgcn_ballot_w64(lane < 32 && x != -INFINITY);
            if (lane == 0) {
                lt[t] = (uint32_t) lv;
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();

    // Tile loads: lane (key kk = lane / 2, half hf = lane % 2) loads bytes
    // [68 hf, 68 hf + 68) of its key's K and V rows -- blocks 2 hf and 2 hf + 1
    // -- as 17 words w[0..16]: eight 8-byte loads (row bytes 0..63, or
    // 72..135) and one 4-byte load (64..67, or 68..71), rows 8-byte aligned
    // (the planner checks the strides and bases). Keys past the split are
    // clamped into it. Offsets inside a tile fit 32 bits (the planner keeps
    // 32 rows below 4 GB).
    const int      kk  = lane >> 1, hf = lane & 1;
    const uint32_t o8  = hf ? 72u : 0u;     // the 8-byte loads' first byte
    const uint32_t o4  = hf ? 68u : 64u;    // the 4-byte load's byte
    uint2          kq8[8], vq8[8];
    uint32_t       kq4, vq4;
    auto           load_tile = [&](int t0) {
        const int      nk  = kend - t0 < T ? kend - t0 : T;
        const uint32_t kr  = (uint32_t) (kk < nk ? kk : nk - 1);
        const char *   kt0 = kg + (int64_t) t0 * a.k1;
        const char *   vt0 = vg + (int64_t) t0 * a.v1;
        const uint32_t ko  = kr * (uint32_t) a.k1, vo = kr * (uint32_t) a.v1;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            kq8[j] = *(const uint2 *) (kt0 + ko + o8 + 8 * j);
            vq8[j] = *(const uint2 *) (vt0 + vo + o8 + 8 * j);
        }
        kq4 = *(const uint32_t *) (kt0 + ko + o4);
        vq4 = *(const uint32_t *) (vt0 + vo + o4);
    };
    // the 17 words in row order: w[i] = bytes 68 hf + 4 i .. + 3
    auto words = [&](const uint2 * q8, uint32_t q4, uint32_t * w) {
#pragma unroll
        for (int i = 0; i < 17; ++i) {
            const int      j0 = i / 2, j1 = (i - 1) / 2;               // the 8-byte load holding word i (hf 0 / 1)
            const uint32_t w0 = i < 16 ? (i % 2 ? q8[j0].y : q8[j0].x) : q4;
            const uint32_t w1 = i > 0 ? ((i - 1) % 2 ? q8[j1].y : q8[j1].x) : q4;
            w[i]              = hf ? w1 : w0;
        }
    };

    f4 o[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
        o[dt] = f4{ 0.0f, 0.0f, 0.0f, 0.0f };
    }
    float    mrun = -INFINITY, lrun = 0.0f;
    uint32_t live = nt > 0 ? lt[0] : 0u;
    if (live) {
        load_tile(kbeg);
    }
    for (int t = 0; t < nt; ++t) {
        const int      t0   = kbeg + t * T;
        const uint32_t next = t + 1 < nt ? lt[t + 1] : 0u;
        if (live) {
            // K: the half-row into the raw tile, its block scales into dks. V:
            // its block scales into dvs (0 for a key no head reads) and its
            // quants as bf16 (exact) into the row-major tile.
            const bool rd = (live >> kk) & 1u;
            uint32_t   w[17];
            words(kq8, kq4, w);
            {
                char * kp = kraw + kk * RB + 68 * hf;  // 4-byte aligned
#pragma unroll
                for (int i = 0; i < 17; ++i) {
                    *(uint32_t *) (kp + 4 * i) = w[i];
                }
                dks[2 * hf][kk]     = (float) __builtin_bit_cast(_Float16, (uint16_t) (w[0] & 0xffffu));
                dks[2 * hf + 1][kk] = (float) __builtin_bit_cast(_Float16, (uint16_t) (w[8] >> 16));
            }
            words(vq8, vq4, w);
            {
                dvs[2 * hf][kk]     = rd ? (float) __builtin_bit_cast(_Float16, (uint16_t) (w[0] & 0xffffu)) : 0.0f;
                dvs[2 * hf + 1][kk] = rd ? (float) __builtin_bit_cast(_Float16, (uint16_t) (w[8] >> 16)) : 0.0f;
                // quants: first block at half-row bytes 2..33, second at 36..67
                uint32_t qa[8], qb[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    qa[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2);
                    qb[i] = w[9 + i];
                }
#pragma unroll
                for (int bb = 0; bb < 2; ++bb) {
                    const uint32_t * qw = bb ? qb : qa;
                    uint32_t         bw[16];
#pragma unroll
                    for (int w4 = 0; w4 < 8; ++w4) {
                        const int32_t x = (int32_t) qw[w4];
                        bw[2 * w4]      = pack_bf16x2((float) (int8_t) (x & 0xff), (float) (int8_t) ((x >> 8) & 0xff));
                        bw[2 * w4 + 1]  = pack_bf16x2((float) (int8_t) ((x >> 16) & 0xff), (float) (int8_t) (x >> 24));
                    }
                    uint4 * dst = (uint4 *) (vt + kk * VR + 64 * (2 * hf + bb));
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        dst[c] = make_uint4(bw[4 * c], bw[4 * c + 1], bw[4 * c + 2], bw[4 * c + 3]);
                    }
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            __builtin_amdgcn_wave_barrier();
        }
        if (next) {
            load_tile(t0 + T);  // in flight during this tile's math
        }
        if (live) {
            // S^T for keys 16 mt + [0, 16) x the 16 (padded) heads, block by block
            f4 s[2];
#pragma unroll
            for (int mt2 = 0; mt2 < 2; ++mt2) {
                i4 acc[NB];
#pragma unroll
                for (int kb = 0; kb < NB; ++kb) {
                    const long ka = *(const long *) (kraw + (16 * mt2 + c16) * RB + 34 * kb + 2 + 8 * q4);
                    acc[kb]       = __builtin_amdgcn_mfma_i32_16x16x32_i8(ka, qb8[kb], i4{ 0, 0, 0, 0 }, 0, 0, 0);
                }
                // the scales of keys 16 mt + 4 q4 + r, r < 4, per block
                f4 dk[NB];
#pragma unroll
                for (int kb = 0; kb < NB; ++kb) {
                    dk[kb] = *(const f4 *) &dks[kb][16 * mt2 + 4 * q4];
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float sa = 0.0f, sb = 0.0f;
                    sa        = __builtin_fmaf(dk[0][r] * dq[0], (float) acc[0][r], sa);
                    sa        = __builtin_fmaf(dk[1][r] * dq[1], (float) acc[1][r], sa);
                    sb        = __builtin_fmaf(dk[2][r] * dq[2], (float) acc[2][r], sb);
                    sb        = __builtin_fmaf(dk[3][r] * dq[3], (float) acc[3][r], sb);
                    s[mt2][r] = sa + sb;
                }
            }
            // softmax as k_fa_dec: this lane's 8 keys of head c16, then the other 24 in lanes ^ 16, ^ 32
            float x[8];
            float tmax = -INFINITY;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int   kk = 16 * (e >> 2) + 4 * q4 + (e & 3);
                const float mv = mt[t * T + kk];
                x[e]           = mv == -INFINITY ? -INFINITY : s[e >> 2][e & 3] * a.scale + mv;
                tmax           = fmaxf(tmax, x[e]);
            }
            tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
            // Lazy rescale (as k_fa_mfma): the reference max moves only when some
            // head's max passes it by more than ln 256, so p <= 256 and O, l are
            // rescaled only then
            if (__builtin_amdgcn_ballot_w64(tmax > mrun + 5.5451774f) != 0) {
                __asm__ volatile("");  // a real branch: the 32 multiplies are not speculated
                const float mn    = fmaxf(mrun, tmax);
                const float alpha = mn == -INFINITY ? 1.0f : __expf(mrun - mn);  // exp(-inf) = 0 on the first live tile
                mrun              = mn;
                lrun *= alpha;
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) {
                    o[dt] *= alpha;
                }
            }
            float p[8], psum = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                p[e] = mrun == -INFINITY || x[e] == -INFINITY ? 0.0f : __expf(x[e] - mrun);
                psum += p[e];
            }
            lrun += psum;
            // O^T += V^T P'^T per V block: B = p * d_v[key][block] (high and low
            // bf16 parts) for keys 4 q4 + r and 16 + 4 q4 + r; A = V^T row 16 dt + c16
            // at those keys by two transposed reads of the bf16 tile (as k_fa_dec)
#pragma unroll
            for (int bk = 0; bk < NB; ++bk) {
                const f4 d0 = *(const f4 *) &dvs[bk][4 * q4];
                const f4 d1 = *(const f4 *) &dvs[bk][16 + 4 * q4];
                // pairs through the packed conversion (RNE): the high parts, their
                // values back as floats, the remainders, the low parts
                uint32_t hw[4], lw[4];
#pragma unroll
                for (int e2 = 0; e2 < 4; ++e2) {
                    const float pa = p[2 * e2] * (e2 < 2 ? d0[2 * e2] : d1[2 * e2 - 4]);
                    const float pb = p[2 * e2 + 1] * (e2 < 2 ? d0[2 * e2 + 1] : d1[2 * e2 - 3]);
                    hw[e2]         = pack_bf16x2(pa, pb);
                    lw[e2]         = pack_bf16x2(pa - __uint_as_float(hw[e2] << 16), pb - __uint_as_float(hw[e2] & 0xffff0000u));
                }
                const x8 phi = __builtin_bit_cast(x8, make_uint4(hw[0], hw[1], hw[2], hw[3]));
                const x8 plo = __builtin_bit_cast(x8, make_uint4(lw[0], lw[1], lw[2], lw[3]));
#pragma unroll
                for (int dh = 0; dh < 2; ++dh) {
                    const int     dt = 2 * bk + dh;
                    const char *  vp = vt + (4 * q4 + c16 / 4) * VR + (16 * dt + 4 * (c16 & 3)) * 2;
                    const fa_v4s  v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((fa_lds_v4s *) vp);             // keys 4 q4 + r
                    const fa_v4s  v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((fa_lds_v4s *) (vp + 16 * VR));  // keys 16 + 4 q4 + r
                    const x8      va = __builtin_bit_cast(x8, __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7));
                    o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, phi, o[dt], 0, 0, 0);
                    o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, plo, o[dt], 0, 0, 0);
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            __builtin_amdgcn_wave_barrier();  // the next tile overwrites the LDS tiles
        }
        live = next;
    }

    // the head's sum over its 4 lanes; lane (c16, q4) holds O^T[16 dt + 4 q4 + r][c16]
    lrun += __shfl_xor(lrun, 16, 64);
    lrun += __shfl_xor(lrun, 32, 64);
    if (!rv) {
        return;
    }
    if (a.splits == 1) {
        const float inv = 1.0f / lrun;  // all keys masked: 0 * inf = NaN, as ggml
        float *     yp  = (float *) (a.y + (int64_t) b * a.y3 + (int64_t) h * a.y1);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                yp[16 * dt + 4 * q4 + r] = o[dt][r] * inv;
            }
        }
    } else {
        float * wp = a.ws + (((int64_t) split * a.nb * a.nkv + bg) * a.rows + c16) * (D + 2);
        if (q4 == 0) {
            wp[0] = mrun;
            wp[1] = lrun;
        }
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                wp[2 + 16 * dt + 4 * q4 + r] = o[dt][r];
            }
        }
    }
}

// Mask summary for the matrix-core path, one wave per (mask batch and head,
// group of 16 query positions, FA_SUM_T consecutive 64-key tiles): lane = 4
// keys (4 * (lane % 16)) of rows lane / 16 + 4 i of each tile, as 8-byte loads
// when the mask rows allow it.
// The attention kernel then loads no mask values for a tile whose values are
// all 0 and skips the math of a tile whose keys are all -inf for its rows.
__global__ void __launch_bounds__(64) k_fa_mask_summary(const FaArgs a) {
    // FA_SUM_T consecutive tiles per wave: all of their loads are issued before
    // any flag is formed
    const int      lane = threadIdx.x;
    const uint32_t grp = blockIdx.y, mh = blockIdx.z;
    const uint32_t m3 = mh / (uint32_t) a.mne2, m2 = mh - m3 * (uint32_t) a.mne2;
    const char *   mp  = a.mask + (int64_t) m3 * a.m3 + (int64_t) m2 * a.m2;
    const int      ntl = (a.n_kv + 63) / 64;
    const int      kl  = 4 * (lane & 15);  // this lane's 4 keys within a tile
    // Loads are unconditional, rows and keys clamped into the mask (values
    // outside it are never used below), so that all of them are in flight
    // before the first is used; only a lane whose 4 keys straddle the end of
    // a row loads them one by one afterwards.
    uint16_t       hv[FA_SUM_T][4][4];
    if (a.mvec && a.n_kv >= 4) {
        uint2 w[FA_SUM_T][4];
#pragma unroll
        for (int tt = 0; tt < FA_SUM_T; ++tt) {
            const int k4 = ((int) blockIdx.x * FA_SUM_T + tt) * 64 + kl;
            const int ks = k4 + 3 < a.n_kv ? k4 : 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int iq = (int) grp * 16 + (lane >> 4) + 4 * i;
                w[tt][i]     = *(const uint2 *) (mp + (int64_t) (iq < a.n_q ? iq : a.n_q - 1) * a.m1 + (int64_t) ks * 2);
            }
        }
#pragma unroll
        for (int tt = 0; tt < FA_SUM_T; ++tt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                hv[tt][i][0] = (uint16_t) w[tt][i].x;
                hv[tt][i][1] = (uint16_t) (w[tt][i].x >> 16);
                hv[tt][i][2] = (uint16_t) w[tt][i].y;
                hv[tt][i][3] = (uint16_t) (w[tt][i].y >> 16);
            }
        }
#pragma unroll
        for (int tt = 0; tt < FA_SUM_T; ++tt) {
            const int k4 = ((int) blockIdx.x * FA_SUM_T + tt) * 64 + kl;
            if (k4 < a.n_kv && k4 + 3 >= a.n_kv) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int    iq = (int) grp * 16 + (lane >> 4) + 4 * i;
                    const char * rp = mp + (int64_t) (iq < a.n_q ? iq : a.n_q - 1) * a.m1;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        hv[tt][i][e] = *(const uint16_t *) (rp + (int64_t) (k4 + e < a.n_kv ? k4 + e : a.n_kv - 1) * 2);
                    }
                }
            }
        }
    } else {
#pragma unroll
        for (int tt = 0; tt < FA_SUM_T; ++tt) {
            const int k4 = ((int) blockIdx.x * FA_SUM_T + tt) * 64 + kl;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int    iq = (int) grp * 16 + (lane >> 4) + 4 * i;
                const char * rp = mp + (int64_t) (iq < a.n_q ? iq : a.n_q - 1) * a.m1;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    hv[tt][i][e] = *(const uint16_t *) (rp + (int64_t) (k4 + e < a.n_kv ? k4 + e : a.n_kv - 1) * 2);
                }
            }
        }
    }
#pragma unroll
    for (int tt = 0; tt < FA_SUM_T; ++tt) {
        const int tile = (int) blockIdx.x * FA_SUM_T + tt;
        const int k4   = tile * 64 + kl;
        bool      live = false, nz = false;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int  iq    = (int) grp * 16 + (lane >> 4) + 4 * i;
            const bool rowok = tile < ntl && iq < a.n_q;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const bool     ok = rowok && k4 + e < a.n_kv;
                const uint16_t h  = hv[tt][i][e];
                live              = live || (ok && h != 0xFC00u);          // not -inf
                nz                = nz || (ok && (h & 0x7FFFu) != 0);      // not +-0
            }
        }
        const uint64_t lv = __builtin_amdgcn_ballot_w64(live), nv = __builtin_amdgcn_ballot_w64(nz);
        if (lane == 0 && tile < ntl) {
            a.msum[((int64_t) mh * a.ngq + grp) * ntl + tile] = (uint8_t) ((lv ? 1 : 0) | (nv ? 2 : 0));
        }
    }
}

// Lanes l and l ^ 32 combined: v_permlane32_swap of a value with itself leaves
// each lane its own value and its partner's, in one order or the other, so the
// max and the (commutative) sum do not depend on which.
__device__ __forceinline__ float fa_xhalf_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float fa_xhalf_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// raw buffer loads (32-bit offsets, range-checked: reads past the end return 0)
typedef __amdgpu_buffer_rsrc_t fa_rsrc;
__device__ __forceinline__ fa_rsrc fa_make_rsrc(const char * base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void *) base, (short) 0, (int) bytes, 0x00020000);
}
__device__ __forceinline__ uint4 fa_bld16(fa_rsrc r, uint32_t voff, uint32_t soff) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int) voff, (int) soff, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
}

#ifndef MI_FA_ITEM_ORDER
#define MI_FA_ITEM_ORDER 1  // 1: row blocks in descending order across the (sequence, KV head) pairs
#endif
// Work item -> (row block, sequence and KV head). Order 1: row blocks in
// descending order, each over every (sequence, KV head) before the next. Under
// a causal mask a later row block holds more live key tiles, so the longest
// items start first and the shortest fill the last round (longest first); with
// items of equal length the order changes nothing but which run together.
// Order 0: every row block of one (sequence, KV head) in turn.
__device__ __forceinline__ void fa_item(const FaArgs & a, uint32_t item, uint32_t & rbk, uint32_t & bg) {
    if (MI_FA_ITEM_ORDER == 1) {
        const uint32_t nbg = (uint32_t) (a.nb * a.nkv);
        const uint32_t i   = item / nbg;
        rbk                = (uint32_t) a.rblk - 1 - i;
        bg                 = item - i * nbg;
    } else {
        rbk = item % (uint32_t) a.rblk;
        bg  = item / (uint32_t) a.rblk;
    }
}

#ifndef MI_FA_PRIO_PV
#define MI_FA_PRIO_PV 1  // > 0: the wave's issue priority in its P.V section (MFMAs between the P conversions)
#endif
#ifndef MI_FA_MFMA_WPE
#define MI_FA_MFMA_WPE 2  // waves per SIMD: 2 caps registers at 256 (two workgroups per CU, 144 KB of LDS)
#endif
// MSK: a mask (and its summary) is given; without one the kernel is compiled
// with no per-tile summary reads at all.
template <int KT, int D, bool MSK>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(MI_FA_MFMA_WPE, MI_FA_MFMA_WPE)))
k_fa_mfma(const FaArgs a) {
    constexpr bool Q8 = KT == MI_TYPE_Q8_0;
    using M           = FaM<Q8 ? MI_TYPE_BF16 : KT>;  // type of the P.V operands (Q8_0: V's bf16 high part)
    using x8          = typename M::x8;
    typedef int      i32x4 __attribute__((ext_vector_type(4)));
    typedef int      i32x16 __attribute__((ext_vector_type(16)));
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    constexpr int BQ = 128, BK = 64;
    constexpr int KS = Q8 ? D + 16 : D * 2 + 16;  // K row stride in LDS (bytes; Q8_0: the quants): 16-byte bank spread
    constexpr int VR = D * 2 + 64;   // V row stride (bytes): rows 16 banks apart, conflict-free transposed reads
    constexpr int KC = D * 2 / 16;   // 16-byte chunks per K/V row
    constexpr int NC = BK * KC / 256;  // chunks per thread per tile (K and V each; even)
    constexpr int NKS = D / 16;      // k-steps of the S MFMA (Q8_0: 8 elements of a lane's 16 per block)
    constexpr int NDB = D / 32;      // 32-row blocks of O^T (Q8_0: also the blocks of a row)
    constexpr int RBY = Q8 ? NDB * 34 : D * 2;  // bytes of a K/V row
    static_assert(NC * 256 == BK * KC, "tile chunks");
    static_assert(D * 2 % 256 == 0, "the V row stride's bank spread assumes whole 256-byte rows");
    static_assert(!Q8 || BK * NDB == 256, "Q8_0 tiles: one thread per (key, block)");

    // K tiles double-buffered; V tiles double-buffered, or for Q8_0 one tile
    // as its bf16 high part (vt[0]) and f16 low part (vt[1])
    __shared__ __align__(16) char     kt[2][BK * KS];
    __shared__ __align__(16) char     vt[2][BK * VR];
    __shared__ __align__(16) uint16_t kds[2][Q8 ? BK * NDB : 1];  // Q8_0: K block scales [key][block]

    const int      tid  = threadIdx.x;
    const int      wave = tid >> 6;
    const int      lane = tid & 63;
    const int      n    = lane & 31;  // this lane's query row within the wave
    const int      hh   = lane >> 5;
    // work item = (row block, sequence and KV head); the items after the first
    // tfull run as two workgroups, one per half of the key tiles (the last,
    // partial round of workgroups then ends in half the time), and leave partials
    uint32_t item = blockIdx.x, part = 0;
    if (item >= a.tfull) {
        const uint32_t j = item - a.tfull;
        item             = a.tfull + j / 2;
        part             = 1 + (j & 1);
    }
    uint32_t       rbk, bg;
    fa_item(a, item, rbk, bg);
    const uint32_t b    = bg / (uint32_t) a.nkv;
    const uint32_t g    = bg - b * (uint32_t) a.nkv;
    const int      r    = (int) rbk * BQ + wave * 32 + n;
    const bool     rvld = r < a.rows;
    const int      rc   = rvld ? r : a.rows - 1;
    const int      iq   = rc / a.rk;
    const int      h    = (int) g * a.rk + (rc - iq * a.rk);
    const uint32_t kb   = b / (uint32_t) a.rk3;
    const char *   kg   = a.k + (int64_t) kb * a.k3 + (int64_t) g * a.k2;
    const char *   vg   = a.v + (int64_t) kb * a.v3 + (int64_t) g * a.v2;
    const char *   mrow = a.mask ? a.mask + (int64_t) (b % (uint32_t) a.mne3) * a.m3 + (int64_t) (h % a.mne2) * a.m2 +
                                      (int64_t) iq * a.m1
                                 : nullptr;

    // Q^T operands: k-step ks needs q[row][16 ks + 8 hh + i], converted to K's type (RNE).
    // Q8_0: block j needs q[row][32 j + 16 hh + i], i < 16 (ks = 2 j + i / 8), as
    // its x86 Q8_0 quants; d_q of each block kept as fp16 bits.
    // (q's type and access width are tested once, outside the loads, so that
    // every load is in flight before the first is used)
    auto qe = [&](int ks) { return Q8 ? 32 * (ks >> 1) + 16 * hh + 8 * (ks & 1) : 16 * ks + 8 * hh; };
    x8       qb[NKS];
    i32x4    qa[NDB];
    uint16_t dq16[NDB];
    {
        const char * qp = a.q + (int64_t) b * a.q3 + (int64_t) h * a.q2 + (int64_t) iq * a.q1;
        float        f[NKS][8];
        if (a.tq == MI_TYPE_F32) {
            if (a.qvec) {
                uint4 u[NKS][2];
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) {
                    const char * p = qp + (size_t) qe(ks) * 4;
                    u[ks][0]       = ld16(p);
                    u[ks][1]       = ld16(p + 16);
                }
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) {
                    unpack16<MI_TYPE_F32>(u[ks][0], f[ks]);
                    unpack16<MI_TYPE_F32>(u[ks][1], f[ks] + 4);
                }
            } else {
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        f[ks][e] = ((const float *) (qp + (size_t) qe(ks) * 4))[e];
                    }
                }
            }
        } else {
            uint4 v[NKS];
            if (a.qvec) {
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) {
                    v[ks] = ld16(qp + (size_t) qe(ks) * 2);
                }
            } else {
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) {
                    const uint16_t * q16 = (const uint16_t *) (qp + (size_t) qe(ks) * 2);
                    v[ks] = make_uint4((uint32_t) q16[0] | ((uint32_t) q16[1] << 16), (uint32_t) q16[2] | ((uint32_t) q16[3] << 16),
                                       (uint32_t) q16[4] | ((uint32_t) q16[5] << 16), (uint32_t) q16[6] | ((uint32_t) q16[7] << 16));
                }
            }
            if (a.tq == MI_TYPE_BF16) {
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) {
                    unpack16<MI_TYPE_BF16>(v[ks], f[ks]);
                }
            } else {
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) {
                    unpack16<MI_TYPE_F16>(v[ks], f[ks]);
                }
            }
        }
        if constexpr (Q8) {
            // x86 from_float per block (as fa_q8_block): the block's 32 elements sit
            // in lanes l and l ^ 32, so its amax is one exchange away
#pragma unroll
            for (int j = 0; j < NDB; ++j) {
                float x[16];
                float amax = 0.0f;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    x[i] = rvld ? f[2 * j + i / 8][i % 8] : 0.0f;
                    amax = fmaxf(amax, fabsf(x[i]));
                }
                amax              = fa_xhalf_max(amax);
                constexpr float C  = 1.0f / 127.0f;
                const float     q0 = amax * C;
                const float     d  = __builtin_fmaf(__builtin_fmaf(-q0, 127.0f, amax), C, q0);  // IEEE amax / 127
                const float     id = amax != 0.0f ? 127.0f / amax : 0.0f;
                uint32_t        w[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    uint32_t acc = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float q = __builtin_amdgcn_fmed3f(__builtin_rintf(x[4 * k + e] * id), -128.0f, 127.0f);
                        acc |= ((uint32_t) (int32_t) q & 0xffu) << (8 * e);
                    }
                    w[k] = acc;
                }
                qa[j]   = i32x4{ (int) w[0], (int) w[1], (int) w[2], (int) w[3] };
                dq16[j] = f32_to_f16_bits(d);
            }
        } else {
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    qb[ks][e] = __builtin_bit_cast(typename M::e, M::bits(rvld ? f[ks][e] : 0.0f));
                }
            }
        }
    }

    // K and V tile loads: chunk c = tid + 256 i -> key c / KC, 16-byte part c % KC
    // (a row is read by KC consecutive threads) and stored row-major in LDS; the
    // P.V operands are read from V with transposed LDS reads. Buffer loads with
    // the whole 32-bit offset in the per-lane operand, which the range check
    // covers (the planner keeps the key range below 4 GB).
    constexpr int KR = 256 / KC;  // K rows per load round
    static_assert(KC <= 32 && 256 % KC == 0, "tile chunks");
    uint4          kr[NC], vr[NC];
    const uint32_t ko0 = (uint32_t) (tid / KC) * (uint32_t) a.k1 + (uint32_t) (tid % KC) * 16;
    const uint32_t vo0 = (uint32_t) (tid / KC) * (uint32_t) a.v1 + (uint32_t) (tid % KC) * 16;
    // Q8_0: thread (key qk, block qc) loads the 9 words of its key's 136-byte row
    // that hold block qc: bytes [34 qc, 34 qc + 36), 2 bytes earlier for odd qc
    // (4-byte aligned: the planner checks strides and bases), so the block's
    // scale sits at byte 0 (even qc) or 2 (odd) of the words, its quants after it
    const uint32_t qk = (uint32_t) tid >> 2, qc = (uint32_t) tid & 3u;
    const bool     qodd = (qc & 1u) != 0;
    const uint32_t qko  = qk * (uint32_t) a.k1 + 34u * qc - (qodd ? 2u : 0u);
    const uint32_t qvo  = qk * (uint32_t) a.v1 + 34u * qc - (qodd ? 2u : 0u);
    uint32_t       kw[9], vw[9];
    // buffers end at the last key's row: keys past the end read as zeros
    const fa_rsrc  krs = fa_make_rsrc(kg, (uint32_t) ((int64_t) (a.n_kv - 1) * a.k1 + RBY));
    const fa_rsrc  vrs = fa_make_rsrc(vg, (uint32_t) ((int64_t) (a.n_kv - 1) * a.v1 + RBY));
    auto load_tile = [&](int t0) {
        const uint32_t ks0 = (uint32_t) t0 * (uint32_t) a.k1;
        const uint32_t vs0 = (uint32_t) t0 * (uint32_t) a.v1;
        if constexpr (Q8) {
            const uint32_t kb0 = qko + ks0, vb0 = qvo + vs0;
#pragma unroll
            for (int j = 0; j < 9; ++j) {
                kw[j] = __builtin_amdgcn_raw_buffer_load_b32(krs, (int) (kb0 + 4 * j), 0, 0);
            }
#pragma unroll
            for (int j = 0; j < 9; ++j) {
                vw[j] = __builtin_amdgcn_raw_buffer_load_b32(vrs, (int) (vb0 + 4 * j), 0, 0);
            }
        } else {
#pragma unroll
            for (int i = 0; i < NC; ++i) {
                kr[i] = fa_bld16(krs, ko0 + ks0 + (uint32_t) (KR * i) * (uint32_t) a.k1, 0);
            }
#pragma unroll
            for (int i = 0; i < NC; ++i) {
                vr[i] = fa_bld16(vrs, vo0 + vs0 + (uint32_t) (KR * i) * (uint32_t) a.v1, 0);
            }
        }
    };
    // Q8_0: the block's 32 quants from the 9 words (shifted by 2 bytes for even qc)
    auto q8_quants = [&](const uint32_t (&w)[9], uint32_t (&qw)[8]) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            qw[i] = qodd ? w[i + 1] : __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2);
        }
    };
    // K (Q8_0: the quants and the block scale; V goes through store_v)
    auto store_tile = [&](int buf) {
        if constexpr (Q8) {
            uint32_t qw[8];
            q8_quants(kw, qw);
            char * kp = kt[buf] + qk * KS + 32 * qc;
            *(uint4 *) kp        = make_uint4(qw[0], qw[1], qw[2], qw[3]);
            *(uint4 *) (kp + 16) = make_uint4(qw[4], qw[5], qw[6], qw[7]);
            kds[buf][qk * NDB + qc] = (uint16_t) (kw[0] >> (qodd ? 16 : 0));
        } else {
#pragma unroll
            for (int i = 0; i < NC; ++i) {
                const int c = tid + 256 * i;
                *(uint4 *) (kt[buf] + (c / KC) * KS + (c % KC) * 16) = kr[i];
            }
#pragma unroll
            for (int i = 0; i < NC; ++i) {
                const int c = tid + 256 * i;
                *(uint4 *) (vt[buf] + (c / KC) * VR + (c % KC) * 16) = vr[i];
            }
        }
    };
    // Q8_0 V: V' = q d_v of the thread's block, exactly (fma(q + 128, d, -128 d)
    // rounds the exact product, which fp32 holds), stored as its bf16 high part
    // RN(V') into vt[0] and its low part V' - RN(V') into vt[1] as f16 (exact).
    // The buffer is single: the caller separates this store from the previous
    // tile's reads by a barrier.
    auto store_v = [&]() {
        if constexpr (Q8) {
            uint32_t qw[8];
            q8_quants(vw, qw);
            // a non-finite scale reads as 0: a key whose mask is -inf for a row enters
            // the P.V products with p = 0, so the V' of a slot that holds garbage
            // (never written, past a sequence's length) must be finite
            const float d0 = (float) __builtin_bit_cast(_Float16, (uint16_t) (vw[0] >> (qodd ? 16 : 0)));
            const float dv = __builtin_isfinite(d0) ? d0 : 0.0f;
            const float nd = -128.0f * dv;
            uint32_t    hw[16], lw[16];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t x = qw[i] ^ 0x80808080u;  // q + 128 per byte
                float          v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[e] = __builtin_fmaf((float) ((x >> (8 * e)) & 0xffu), dv, nd);
                }
#pragma unroll
                for (int h2 = 0; h2 < 2; ++h2) {
                    const uint32_t hp = pack_bf16x2(v[2 * h2], v[2 * h2 + 1]);
                    hw[2 * i + h2]    = hp;
                    lw[2 * i + h2]    = pack_f16x2(v[2 * h2] - bf16_lo(hp), v[2 * h2 + 1] - bf16_hi(hp));
                }
            }
            uint4 * hp = (uint4 *) (vt[0] + qk * VR + 64 * qc);
            uint4 * lp = (uint4 *) (vt[1] + qk * VR + 64 * qc);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                hp[c] = make_uint4(hw[4 * c], hw[4 * c + 1], hw[4 * c + 2], hw[4 * c + 3]);
                lp[c] = make_uint4(lw[4 * c], lw[4 * c + 1], lw[4 * c + 2], lw[4 * c + 3]);
            }
        }
    };
    // mask values of this lane's 32 keys of a tile (key 32 bk + 8 j + 4 hh + i:
    // groups of 4), as 4 fp16 per 8-byte load when the mask rows allow it and
    // the tile lies inside the row; the choice is uniform, and within it every
    // load is unconditional (keys clamped), so all 8 groups are in flight at once
    auto load_mask = [&](int t0, uint2 (&mr)[2][4]) {
        if (a.mvec && t0 + BK <= a.n_kv) {
#pragma unroll
            for (int bk = 0; bk < 2; ++bk) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    mr[bk][j] = *(const uint2 *) (mrow + (size_t) (t0 + 32 * bk + 8 * j + 4 * hh) * 2);
                }
            }
        } else {
            uint16_t hv[2][4][4];
#pragma unroll
            for (int bk = 0; bk < 2; ++bk) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int k4 = t0 + 32 * bk + 8 * j + 4 * hh;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int kc = k4 + i < a.n_kv ? k4 + i : a.n_kv - 1;
                        hv[bk][j][i] = *(const uint16_t *) (mrow + (size_t) kc * 2);
                    }
                }
            }
#pragma unroll
            for (int bk = 0; bk < 2; ++bk) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    mr[bk][j] = make_uint2((uint32_t) hv[bk][j][0] | ((uint32_t) hv[bk][j][1] << 16),
                                           (uint32_t) hv[bk][j][2] | ((uint32_t) hv[bk][j][3] << 16));
                }
            }
        }
    };

    fa_f32x16 o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
        o[db] = fa_f32x16{};
    }
    float       mrun = -INFINITY, lrun = 0.0f;
    const float sl2  = a.scale * 1.4426950408889634f;  // scale * log2(e)
    const int   ntl  = (a.n_kv + BK - 1) / BK;
    const bool  allr = (int) (rbk * BQ + BQ) <= a.rows;  // every row of the workgroup valid
    int         tb   = part == 2 ? a.tmid : 0;             // this workgroup's key tiles [tb, te)
    int         te   = part == 1 ? a.tmid : ntl;
    // per tile, from the mask summary of this lane's row (one tile ahead): does
    // the wave read the tile's mask values, does it have a live key at all
    const uint8_t * sp =
        MSK ? a.msum + (((int64_t) (b % (uint32_t) a.mne3) * a.mne2 + h % a.mne2) * a.ngq + iq / 16) * ntl
            : nullptr;
    // The tile loop, compiled twice in the masked kernel: with the per-tile
    // summary reads (MK), and without them for a workgroup whose mask rows are
    // all zero over its key range (every summary byte 1: live, no nonzero
    // value) -- the padding mask of unpadded DiT sequences.
    auto tiles = [&](auto mtag) {
    constexpr bool MK = decltype(mtag)::value;
    auto flag = [&](int t) -> int {
        if constexpr (MK) {
            return t < te ? (int) sp[t] : 0;
        } else {
            return t < te ? 1 : 0;
        }
    };
    if (tb >= te) {
        return;  // no tile with a live key for any row of the workgroup
    }
    int  fcur = flag(tb);
    load_tile(tb * BK);
    store_tile(0);
    store_v();
    __syncthreads();
    for (int t = tb; t < te; ++t) {
        const int cur   = (t - tb) & 1;
        const int t0    = t * BK;
        const int fnext = flag(t + 1);
        if (t + 1 < te) {
            load_tile(t0 + BK);  // in flight during this tile's math
        }
        if (__builtin_amdgcn_ballot_w64(rvld && (fcur & 1)) != 0) {  // some row of the wave has a live key
        const bool mload = __builtin_amdgcn_ballot_w64(rvld && (fcur & 2)) != 0;
        // general form: mask values, -inf keys, keys past the end, invalid rows
        // or a negative scale; else the tile is clean
        const bool gen = mload || t0 + BK > a.n_kv || !allr || !(sl2 >= 0.0f);
        uint2      mr[2][4];
        if (mload) {
            load_mask(t0, mr);  // in flight during the S MFMAs
        }
        // S^T for keys [32 bk, 32 bk + 32) x this wave's 32 rows (two independent chains)
        fa_f32x16 sacc[2] = { fa_f32x16{}, fa_f32x16{} };
        if constexpr (Q8) {
            // per block j: the int32 dots (A = 16 quants of key 32 bk + n, B = q's),
            // d_k d_q in the same layout from an fp16 MFMA whose k-slot 0 carries the
            // two scales (slot 8, the other half-wave's, and the rest zero), then
            // s = fma(d_k d_q, dot, s) in block order
#pragma unroll
            for (int bk = 0; bk < 2; ++bk) {
                const uint2 kd4 = *(const uint2 *) &kds[cur][(32 * bk + n) * NDB];  // the key's 4 scales
#pragma unroll
                for (int j = 0; j < NDB; ++j) {
                    const i32x4  ka = *(const i32x4 *) (kt[cur] + (32 * bk + n) * KS + 32 * j + 16 * hh);
                    const i32x16 dd = __builtin_amdgcn_mfma_i32_32x32x32_i8(ka, qa[j], i32x16{}, 0, 0, 0);
                    const uint32_t kdw = j < 2 ? kd4.x : kd4.y;
                    h8 sk = {}, sq = {};
                    sk[0] = __builtin_bit_cast(_Float16, (uint16_t) (hh == 0 ? (kdw >> (16 * (j & 1))) & 0xffffu : 0u));
                    sq[0] = __builtin_bit_cast(_Float16, (uint16_t) (hh == 0 ? dq16[j] : 0u));
                    const fa_f32x16 sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(sk, sq, fa_f32x16{}, 0, 0, 0);
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        sacc[bk][e] = j == 0 ? sc[e] * (float) dd[e] : __builtin_fmaf(sc[e], (float) dd[e], sacc[bk][e]);
                    }
                }
            }
        } else {
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
#pragma unroll
                for (int bk = 0; bk < 2; ++bk) {
                    const x8 kv = *(const x8 *) (kt[cur] + (32 * bk + n) * KS + (16 * ks + 8 * hh) * 2);
                    sacc[bk]    = fa_mma<KT>(kv, qb[ks], sacc[bk]);
                }
            }
        }
        // softmax in base 2, x = (dot * scale + mask) * log2 e. General form: x is
        // written over the scores and p = exp2(x - m). Clean form (every value
        // finite, scale >= 0): the row max of the raw dots times scale * log2 e is
        // the max of x, and p = exp2(dot * scale * log2 e - m) in one fma.
        float tmax = -INFINITY, c1 = sl2;
        if (gen) {
            c1 = 1.0f;
#pragma unroll
            for (int bk = 0; bk < 2; ++bk) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int      key = t0 + 32 * bk + 8 * j + 4 * hh + i;
                        const uint32_t w   = mload ? (i < 2 ? mr[bk][j].x : mr[bk][j].y) : 0u;
                        const float    m = (float) __builtin_bit_cast(_Float16, (uint16_t) (w >> (16 * (i & 1))));
                        const bool     off = m == -INFINITY || key >= a.n_kv || !rvld;
                        const float    v = off ? -INFINITY : sacc[bk][4 * j + i] * sl2 + m * 1.4426950408889634f;
                        sacc[bk][4 * j + i] = v;
                        tmax                = fmaxf(tmax, v);
                    }
                }
            }
        } else {
#pragma unroll
            for (int bk = 0; bk < 2; ++bk) {
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    tmax = fmaxf(tmax, sacc[bk][q]);
                }
            }
            tmax *= sl2;
        }
        tmax = fa_xhalf_max(tmax);  // the row's other 32 keys sit in lane ^ 32
        // Lazy rescale: p = exp2(x - mrun) against a reference max that moves only
        // when some row's max grows past it by more than 8 (p <= 2^8 stays exact
        // enough in fp32 and in the 16-bit parts); O and l are rescaled then only.
        if (__builtin_amdgcn_ballot_w64(tmax > mrun + 8.0f) != 0) {
            __asm__ volatile("");  // a real branch: the 64 multiplies are not speculated
            const float mn  = fmaxf(mrun, tmax);
            const float alp = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(mrun - mn);
            mrun            = mn;
            lrun *= alp;
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    o[db][q] *= alp;
                }
            }
        }
        // a row with no live key yet has mrun = -inf and only -inf values: p = 0
        const float nmn  = mrun == -INFINITY ? 0.0f : -mrun;
        float       psum = 0.0f;
        if constexpr (MI_FA_PRIO_PV > 0) {
            __builtin_amdgcn_s_setprio(MI_FA_PRIO_PV);
        }
        // O^T += V^T P^T. MFMA (bk, jj) covers keys 32 bk + 16 jj + [0, 16): k-slot
        // 8 hh + 4 jh + i is key 32 bk + 16 jj + 8 jh + 4 hh + i (S^T accumulator
        // 8 jj + 4 jh + i); A lane = V^T row 32 db + n at those keys
#pragma unroll
        for (int bk = 0; bk < 2; ++bk) {
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                // A = V^T rows 32 db + l % 32 at those keys, by transposed reads of the
                // row-major V tile: lane m of a 16-lane group addresses V[K0 + m / 4][D0 +
                // 4 (m % 4)], and lane j of the group receives V[K0 .. K0 + 3][D0 + j]
                auto vread = [&](const char * tile, int db) {
                    const char * vp = tile + (32 * bk + 16 * jj + 4 * hh + (lane & 15) / 4) * VR +
                                      (32 * db + 16 * ((lane >> 4) & 1) + 4 * (lane & 3)) * 2;
                    const fa_v4s v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((fa_lds_v4s *) vp);           // keys +0..3
                    const fa_v4s v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((fa_lds_v4s *) (vp + 8 * VR));  // keys +8..11
                    return __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
                };
                if constexpr (Q8) {
                    // P as bf16 high + low parts against V's bf16 high part, and P as
                    // f16 against its f16 low part (|low| <= 2^-8 |V'|)
                    uint32_t ph[4], pl[4], pf[4];
#pragma unroll
                    for (int pr = 0; pr < 4; ++pr) {
                        const float p0 = __builtin_amdgcn_exp2f(fmaf(sacc[bk][8 * jj + 2 * pr], c1, nmn));
                        const float p1 = __builtin_amdgcn_exp2f(fmaf(sacc[bk][8 * jj + 2 * pr + 1], c1, nmn));
                        psum += p0;
                        psum += p1;
                        ph[pr] = pack_bf16x2(p0, p1);
                        pl[pr] = pack_bf16x2(p0 - bf16_lo(ph[pr]), p1 - bf16_hi(ph[pr]));
                        pf[pr] = pack_f16x2(p0, p1);
                    }
                    const x8 phi = __builtin_bit_cast(x8, ph), plo = __builtin_bit_cast(x8, pl);
                    const h8 pfh = __builtin_bit_cast(h8, pf);
                    x8       va[NDB];
                    h8       vl[NDB];
#pragma unroll
                    for (int db = 0; db < NDB; ++db) {
                        va[db] = __builtin_bit_cast(x8, vread(vt[0], db));
                        vl[db] = __builtin_bit_cast(h8, vread(vt[1], db));
                    }
#pragma unroll
                    for (int db = 0; db < NDB; ++db) {
                        o[db] = fa_mma<MI_TYPE_BF16>(va[db], phi, o[db]);
                    }
#pragma unroll
                    for (int db = 0; db < NDB; ++db) {
                        o[db] = fa_mma<MI_TYPE_BF16>(va[db], plo, o[db]);
                    }
#pragma unroll
                    for (int db = 0; db < NDB; ++db) {
                        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vl[db], pfh, o[db], 0, 0, 0);
                    }
                } else {
                    x8 phi, plo;
#pragma unroll
                    for (int slot = 0; slot < 8; ++slot) {
                        const float    p  = __builtin_amdgcn_exp2f(fmaf(sacc[bk][8 * jj + slot], c1, nmn));
                        const uint16_t hb = M::bits(p);
                        psum += p;
                        phi[slot] = __builtin_bit_cast(typename M::e, hb);
                        plo[slot] = __builtin_bit_cast(typename M::e, M::bits(p - M::val(hb)));
                    }
                    x8 va[NDB];
#pragma unroll
                    for (int db = 0; db < NDB; ++db) {
                        va[db] = __builtin_bit_cast(x8, vread(vt[cur], db));
                    }
#pragma unroll
                    for (int db = 0; db < NDB; ++db) {
                        o[db] = fa_mma<KT>(va[db], phi, o[db]);
                    }
#pragma unroll
                    for (int db = 0; db < NDB; ++db) {
                        o[db] = fa_mma<KT>(va[db], plo, o[db]);
                    }
                }
            }
        }
        lrun += psum;
        if constexpr (MI_FA_PRIO_PV > 0) {
            __builtin_amdgcn_s_setprio(0);
        }
        }  // live
        if (t + 1 < te) {
            store_tile(cur ^ 1);
        }
        fcur = fnext;
        __syncthreads();
        if constexpr (Q8) {
            if (t + 1 < te) {  // uniform: the next tile's V once every wave has read this one's
                store_v();
                __syncthreads();
            }
        }
    }
    };
    bool clean = !MSK;
    if constexpr (MSK) {
        // One pass over this lane's summary bytes: are they all "live, zero"
        // (then the workgroup may skip the per-tile reads), and which tiles hold
        // a live key for the row. The workgroup then walks only the tiles from
        // the first to the last live one of any of its rows (a sliding-window
        // mask leaves a few of them), with the same tiles and order for every
        // wave. Independent loads (no short-circuit): a chain of dependent byte
        // loads would cost a memory latency per tile.
        // The bytes are read 16 at a time, all 16 loads issued before any is
        // used: one memory latency per 16 tiles, where a loop of single loads
        // waits once per tile.
        uint32_t c  = 1;
        int      lo = te, hi = tb - 1;
        if (rvld) {
            for (int t16 = tb; t16 < te; t16 += 16) {
                uint32_t f[16];
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    f[j] = sp[t16 + j < te ? t16 + j : te - 1];  // past the range: a repeat of the last byte
                }
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int t = t16 + j;
                    if (t < te) {
                        c &= (uint32_t) (f[j] == 1);
                        lo = (f[j] & 1) && t < lo ? t : lo;
                        hi = (f[j] & 1) ? t : hi;
                    }
                }
            }
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            lo = min(lo, __shfl_xor(lo, off, 64));
            hi = max(hi, __shfl_xor(hi, off, 64));
        }
        __shared__ int wrange[4][2];
        if (lane == 0) {
            wrange[wave][0] = lo;
            wrange[wave][1] = hi;
        }
        clean = __syncthreads_and((int) c) != 0;  // workgroup-uniform: the waves share the K/V tiles
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            lo = min(lo, wrange[w][0]);
            hi = max(hi, wrange[w][1]);
        }
        tb = lo;
        te = hi + 1;
    }
    if (clean) {
        tiles(std::false_type{});
    } else {
        tiles(std::true_type{});
    }
    // rows: sum over both half-waves' keys; y[b][iq][h][d], d = 32 db + 8 j + 4 hh + i
    lrun = fa_xhalf_sum(lrun);
    if (part != 0) {  // half of the keys: (m, l, o) relative to exp2(m), merged by k_fa_mfma_combine
        if (rvld) {
            float * pp = a.fpart + ((size_t) (blockIdx.x - a.tfull) * BQ + wave * 32 + n) * FA_PART;
            if (hh == 0) {
                pp[0] = mrun;
                pp[1] = lrun;
            }
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    *(float4 *) (pp + 4 + 32 * db + 8 * j + 4 * hh) =
                        make_float4(o[db][4 * j], o[db][4 * j + 1], o[db][4 * j + 2], o[db][4 * j + 3]);
                }
            }
        }
        return;
    }
    if (rvld) {
        const float inv = 1.0f / lrun;  // all keys masked: 0 * inf = NaN, as ggml
        float *     yp  = (float *) (a.y + (int64_t) b * a.y3 + (int64_t) iq * a.y2 + (int64_t) h * a.y1);
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 v = make_float4(o[db][4 * j] * inv, o[db][4 * j + 1] * inv, o[db][4 * j + 2] * inv,
                                             o[db][4 * j + 3] * inv);
                float *      d = yp + 32 * db + 8 * j + 4 * hh;
                if (a.yvec) {
                    *(float4 *) d = v;
                } else {
                    d[0] = v.x;
                    d[1] = v.y;
                    d[2] = v.z;
                    d[3] = v.w;
                }
            }
        }
    }
}

// Merge the two key halves of a split work item (its 128 rows): with w_i =
// exp2(m_i - max m) (0 for a half with no live key), y = (w_0 o_0 + w_1 o_1) /
// (w_0 l_0 + w_1 l_1); a row with no live key in either half is NaN, as ggml.
// 8 rows per workgroup, 32 lanes per row, 4 columns per lane.
__global__ void __launch_bounds__(256) k_fa_mfma_combine(const FaArgs a) {
    const uint32_t row  = blockIdx.x * 8 + threadIdx.x / 32;  // split item * 128 + row of the block
    const uint32_t j    = row / 128, rr = row % 128;
    uint32_t       rbk, bg;
    fa_item(a, a.tfull + j, rbk, bg);
    const int      r    = (int) (rbk * 128 + rr);
    if (r >= a.rows) {
        return;
    }
    const uint32_t b  = bg / (uint32_t) a.nkv;
    const uint32_t g  = bg - b * (uint32_t) a.nkv;
    const int      iq = r / a.rk;
    const int      h  = (int) g * a.rk + (r - iq * a.rk);
    const float *  p0 = a.fpart + ((size_t) (2 * j) * 128 + rr) * FA_PART;
    const float *  p1 = a.fpart + ((size_t) (2 * j + 1) * 128 + rr) * FA_PART;
    const float2   s0 = *(const float2 *) p0, s1 = *(const float2 *) p1;  // (m, l)
    const float    mx = fmaxf(s0.x, s1.x);
    const float    w0 = s0.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s0.x - mx);
    const float    w1 = s1.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s1.x - mx);
    const float    il = 1.0f / (w0 * s0.y + w1 * s1.y);
    const int      d  = 4 * (threadIdx.x % 32);
    const float4   o0 = *(const float4 *) (p0 + 4 + d), o1 = *(const float4 *) (p1 + 4 + d);
    float *        yp = (float *) (a.y + (int64_t) b * a.y3 + (int64_t) iq * a.y2 + (int64_t) h * a.y1);
    yp[d]             = (w0 * o0.x + w1 * o1.x) * il;
    yp[d + 1]         = (w0 * o0.y + w1 * o1.y) * il;
    yp[d + 2]         = (w0 * o0.z + w1 * o1.z) * il;
    yp[d + 3]         = (w0 * o0.w + w1 * o1.w) * il;
}

// query rows per wave: 4, or 8 for 16-bit and Q8_0 K/V at D = 64 (more would
// spill registers: each row keeps its output columns and scores in registers)
static int fa_rb(int rows, int D, int kt) {
    return D == 64 && kt != MI_TYPE_F32 && rows > 4 ? 8 : 4;
}

// rows per wave and KV splits for a problem; the workspace holds one
// (max, sum, D outputs) record per split and row when there is more than one split
void flash_attn_plan(FaArgs & a, int D) {
    a.rows          = a.n_q * a.rk;
    const int rb    = fa_rb(a.rows, D, a.kt);
    a.rblocks       = (a.rows + rb - 1) / rb;
    // rows r0..r0+rb-1 of a wave share one query position when n_q == 1 or rb
    // divides Nh/Nkv, and one mask head when the mask does not vary by head
    a.mshared = a.mask != nullptr && a.mne2 == 1 && (a.n_q == 1 || a.rk % rb == 0);
    // Q8_0 K/V are loaded as 4-byte words: row starts 4-byte aligned (strides and bases)
    const bool q8 = MI_FA_MFMA_Q8 && a.kt == MI_TYPE_Q8_0 && a.k1 % 4 == 0 && a.k2 % 4 == 0 && a.k3 % 4 == 0 &&
                    a.v1 % 4 == 0 && a.v2 % 4 == 0 && a.v3 % 4 == 0 && aligned(a.k, 4) && aligned(a.v, 4);
    a.mfma = (a.kt == MI_TYPE_F16 || a.kt == MI_TYPE_BF16 || q8) && D == 128 && a.rows >= MI_FA_MFMA_MIN_ROWS &&
             a.n_kv > 0 && (uint64_t) (a.n_kv + 64) * (uint64_t) (a.k1 > a.v1 ? a.k1 : a.v1) < (1ull << 32);
    if (a.mfma) {
        a.chunk  = a.n_kv;
        a.splits = 1;
        a.ngq    = (a.n_q + 15) / 16;
        // whole items fill full rounds of the resident workgroups (two per CU);
        // a last round at most half full runs as key halves instead
        a.rblk             = (a.rows + 127) / 128;
        const int64_t items = (int64_t) a.rblk * a.nb * a.nkv;
        const int64_t slots = (int64_t) num_cus() * 2;
        const int64_t rest  = items % slots;
        const int     ntl   = (a.n_kv + 63) / 64;
        a.tmid              = (ntl + 1) / 2;
        a.tfull             = (int) items;
        if (items > slots && rest > 0 && 2 * rest <= slots && ntl >= 2) {
            a.tfull = (int) (items - rest);
        }
        a.tsplit = (int) (items - a.tfull);
        return;
    }
    if (a.n_kv == 0 || a.rows == 0 || a.nb == 0) {  // no keys: one pass that writes NaN rows (0 * (1/0), as ggml)
        a.chunk  = FA_TILE;
        a.splits = 1;
        return;
    }
    // decode on the matrix cores: one wave holds every query head of a KV head
    a.dec = MI_FA_DEC && (a.kt == MI_TYPE_F16 || a.kt == MI_TYPE_BF16) && D == 128 && a.n_q == 1 &&
            a.rows <= 16 && (a.mask == nullptr || a.mne2 == 1);
    // Q8_0 caches: rows are loaded as 8-byte words, so every row start must be
    // 8-byte aligned (136-byte rows: strides and bases multiples of 8), and a
    // tile's 32 rows must span less than 4 GB (32-bit offsets)
    a.dec = a.dec || (MI_FA_DEC_Q8 && a.kt == MI_TYPE_Q8_0 && D == 128 && a.n_q == 1 && a.rows <= 16 &&
                      (a.mask == nullptr || a.mne2 == 1) && a.k1 % 8 == 0 && a.k2 % 8 == 0 && a.k3 % 8 == 0 &&
                      a.v1 % 8 == 0 && a.v2 % 8 == 0 && a.v3 % 8 == 0 && aligned(a.k, 8) && aligned(a.v, 8) &&
                      a.k1 < ((int64_t) 1 << 26) && a.v1 < ((int64_t) 1 << 26));
    if (a.dec) {
        a.rblocks = 1;
    }
    const int64_t pairs  = (int64_t) a.nb * a.nkv * a.rblocks;
    const int64_t want   = (int64_t) num_cus() * (a.dec && a.kt == MI_TYPE_Q8_0 ? MI_FA_DEC_Q8_WAVES_PER_CU : MI_FA_WAVES_PER_CU);
    const int64_t tiles  = (a.n_kv + FA_TILE - 1) / FA_TILE;
    int64_t       splits = (want + pairs - 1) / pairs;
    splits               = splits < 1 ? 1 : (splits > tiles ? tiles : splits);
    int64_t       per    = (tiles + splits - 1) / splits;  // tiles per split
    per                  = per > FA_MAXT ? FA_MAXT : per;
    if ((tiles + per - 1) / per > FA_MAX_SPLITS) {
        return;  // more than FA_MAX_SPLITS * FA_MAXT * FA_TILE keys: rejected by the caller (splits = 0)
    }
    a.chunk              = (int) (per * FA_TILE);
    a.splits             = (int) ((a.n_kv + a.chunk - 1) / a.chunk);
}

size_t flash_attn_part_offset(const FaArgs & a) {
    const size_t msum = (size_t) a.nb * a.nh * a.ngq * ((a.n_kv + 63) / 64);
    return (msum + 255) / 256 * 256;
}

size_t flash_attn_workspace(const FaArgs & a, int D) {
    if (a.mfma) {  // the mask summary, sized for the largest mask a call may pass (one per batch and head),
                   // then the partials of split items
        return flash_attn_part_offset(a) + (size_t) a.tsplit * 2 * 128 * FA_PART * sizeof(float);
    }
    return a.splits > 1 ? (size_t) a.splits * a.nb * a.nkv * a.rows * (D + 2) * sizeof(float) : 0;
}

template <int KT, int D>
static void launch_kd(const FaArgs & a, hipStream_t s) {
    const dim3 grid((uint32_t) a.splits, (uint32_t) (a.nb * a.nkv), (uint32_t) a.rblocks);
    if constexpr (D == 128 && (KT == MI_TYPE_F16 || KT == MI_TYPE_BF16)) {
        if (a.dec) {
            MI_LAUNCH((k_fa_dec<KT>), grid, dim3(64), 0, s, a);
            if (a.splits > 1) {
                MI_LAUNCH((k_fa_combine<D>), dim3((uint32_t) (a.nb * a.nkv * a.rows)), dim3(256), 0, s, a);
            }
            return;
        }
    }
    if constexpr (D == 128 && KT == MI_TYPE_Q8_0) {
        if (a.dec) {
            MI_LAUNCH(k_fa_dec_q8, grid, dim3(64), 0, s, a);
            if (a.splits > 1) {
                MI_LAUNCH((k_fa_combine<D>), dim3((uint32_t) (a.nb * a.nkv * a.rows)), dim3(256), 0, s, a);
            }
            return;
        }
    }
    if constexpr (D == 64 && KT != MI_TYPE_F32) {
        if (fa_rb(a.rows, D, KT) == 8) {
            MI_LAUNCH((k_fa_split<KT, D, 8>), grid, dim3(64), 0, s, a);
        } else {
            MI_LAUNCH((k_fa_split<KT, D, 4>), grid, dim3(64), 0, s, a);
        }
    } else {
        MI_LAUNCH((k_fa_split<KT, D, 4>), grid, dim3(64), 0, s, a);
    }
    if (a.splits > 1) {
        MI_LAUNCH((k_fa_combine<D>), dim3((uint32_t) (a.nb * a.nkv * a.rows)), dim3(256), 0, s, a);
    }
}

template <int KT>
static int launch_k(const FaArgs & a, int D, hipStream_t s) {
    switch (D) {
        case 64:
            launch_kd<KT, 64>(a, s);
            return MI_OK;
        case 128:
            launch_kd<KT, 128>(a, s);
            return MI_OK;
        case 256:
            if constexpr (KT != MI_TYPE_F32) {
                launch_kd<KT, 256>(a, s);
                return MI_OK;
            }
            return MI_ERR_UNSUPPORTED;
        default:
            return MI_ERR_UNSUPPORTED;
    }
}

int launch_flash_attn(const FaArgs & a, int kt, int D, hipStream_t s) {
    if (a.rows == 0 || a.nb == 0 || a.nkv == 0) {
        return MI_OK;
    }
    if (a.mfma) {
        if (a.msum != nullptr) {
            MI_LAUNCH(k_fa_mask_summary, dim3((uint32_t) (((a.n_kv + 63) / 64 + FA_SUM_T - 1) / FA_SUM_T),
                                                       (uint32_t) a.ngq,
                                                       (uint32_t) (a.mne3 * a.mne2)),
                               dim3(64), 0, s, a);
        }
        const dim3 grid((uint32_t) (a.tfull + 2 * a.tsplit));
        if (kt == MI_TYPE_Q8_0) {
            if (a.msum) {
                MI_LAUNCH((k_fa_mfma<MI_TYPE_Q8_0, 128, true>), grid, dim3(256), 0, s, a);
            } else {
                MI_LAUNCH((k_fa_mfma<MI_TYPE_Q8_0, 128, false>), grid, dim3(256), 0, s, a);
            }
        } else if (kt == MI_TYPE_BF16) {
            if (a.msum) {
                MI_LAUNCH((k_fa_mfma<MI_TYPE_BF16, 128, true>), grid, dim3(256), 0, s, a);
            } else {
                MI_LAUNCH((k_fa_mfma<MI_TYPE_BF16, 128, false>), grid, dim3(256), 0, s, a);
            }
        } else {
            if (a.msum) {
                MI_LAUNCH((k_fa_mfma<MI_TYPE_F16, 128, true>), grid, dim3(256), 0, s, a);
            } else {
                MI_LAUNCH((k_fa_mfma<MI_TYPE_F16, 128, false>), grid, dim3(256), 0, s, a);
            }
        }
        if (a.tsplit > 0) {
            MI_LAUNCH(k_fa_mfma_combine, dim3((uint32_t) a.tsplit * 16), dim3(256), 0, s, a);
        }
        return MI_OK;
    }
    switch (kt) {
        case MI_TYPE_F16:
            return launch_k<MI_TYPE_F16>(a, D, s);
        case MI_TYPE_BF16:
            return launch_k<MI_TYPE_BF16>(a, D, s);
        case MI_TYPE_Q8_0:
            return launch_k<MI_TYPE_Q8_0>(a, D, s);
        case MI_TYPE_F32:
            return launch_k<MI_TYPE_F32>(a, D, s);
        default:
            return MI_ERR_TYPE;
    }
}

}  // namespace mi
