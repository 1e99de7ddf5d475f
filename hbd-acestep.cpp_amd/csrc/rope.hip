// rope.hip -- per-head RMSNorm (QK-norm) fused with NEOX rotary embedding.
//
// ggml node chain reproduced for each head row of D elements (reference:
// qwen3-lm.h:372-379, 660-667; qwen3-enc.h:165-174; dit-graph.h:183-196):
//   n = rms_norm(x, eps) * w                      (optional)
//   ggml_rope_ext mode 2 (NEOX): for pair i < n_dims/2
//     theta_0 = (float)pos, theta_{i+1} = theta_i * theta_scale   (fp32 chain)
//     c = cosf(freq_scale*theta_i)*attn_factor, s = sinf(...)*attn_factor
//     (cos/sin from sincos_rot, trig.h: |error| < 1e-7 against exact sin/cos)
//     y_i = n_i*c - n_{i+h}*s ;  y_{i+h} = n_i*s + n_{i+h}*c     (h = n_dims/2)
// theta_scale = powf(freq_base, -2/n_dims) is computed on the host, with the
// host libm, as ggml-cpu does.
//
// Fast path (n_dims == ne0 == D in {64, 128, 256}): a wave handles one token
// at a time and walks its tokens with the next one's loads in flight. A
// lane holds 16 bytes of the first half of a head row and the matching 16
// bytes of the second half, so both members of every rotated pair are in the
// same lane (no cross-lane exchange for the rotation). A head row is spread
// over L = D/2/VEC lanes and reduced with DPP. The token's cos/sin table is
// built once per token in LDS and reused for all its Q and K head rows.
// Inputs may be strided views of the fused QKV projection output, so no
// separate contiguous copy is needed.
#include "launch.h"
#include "trig.h"

namespace mi {

#ifndef MI_ROPE_PF
#define MI_ROPE_PF 3  // row batches (64/L head rows each) loaded ahead per wave
#endif
#ifndef MI_ROPE_ONE_ROUND
#define MI_ROPE_ONE_ROUND 1  // split tokens with more than PF batches over several work items
#endif

// One wave per (token, group of head batches) work item: a whole token per
// item when there are enough tokens to fill the chip, a few batches per item
// otherwise (decode). The grid is persistent (the workgroups that fit on the
// chip at once) and each wave walks its items with a stride, software
// pipelined: the loads of the next item's first PF batches are issued before
// the current item is computed, so every wave keeps a token's rows in flight
// while it computes and stores the previous one. The two register sets
// alternate between even and odd steps (no copies, which would wait for the
// loads). The first item's loads are issued before anything else, the Q/K
// norm weights are then staged once per workgroup in LDS.
//
// Per item, lane 0 runs the token's fp32 theta chain into LDS, lane l turns
// theta_l into cos/sin (sincos_rot) and stores them back, and every lane then
// reads the VEC pairs it rotates. The wave streams the token's head rows in
// batches of R = 64/L rows, Q rows first, then K rows; a batch never mixes Q
// and K, so the segment (pointers, strides, weights) is wave-uniform and its
// addressing stays scalar. Lanes whose row lies past the segment end load
// nothing and store nothing (whole L-lane groups, so the DPP row sums stay per
// group).
#ifndef MI_ROPE_WG_PER_CU
#define MI_ROPE_WG_PER_CU 0  // grid cap in workgroups per CU; 0: as many as fit at once
#endif
#ifndef MI_ROPE_WPE
#define MI_ROPE_WPE 0  // > 0: ask the compiler for at least this many waves per SIMD
#endif
#if MI_ROPE_WPE > 0
#define MI_ROPE_OCC __attribute__((amdgpu_waves_per_eu(MI_ROPE_WPE, 8)))
#else
#define MI_ROPE_OCC
#endif

struct HeadItem {
    uint32_t bbeg, bend;  // batch range
    uint32_t i2, i3;      // token coordinates
    int32_t  pos;         // the token's position (rope only)
};

template <int TI, int TO, int D, bool NORM, bool ROPE>
__global__ void __launch_bounds__(256) MI_ROPE_OCC k_heads(const HeadArgs a, uint32_t nb0, uint32_t nb, uint32_t bpw,
                                                           FastDiv dgroups) {
    constexpr int VI   = TT<TI>::VEC;
    constexpr int EI   = TT<TI>::ES;
    constexpr int EO   = TT<TO>::ES;
    constexpr int HALF = D / 2;
    constexpr int L    = HALF / VI;  // lanes per head row
    constexpr int R    = 64 / L;     // head rows per batch
    constexpr int PF   = MI_ROPE_PF;
    constexpr int PL   = (HALF + 63) / 64;  // cos/sin pairs per lane
    static_assert(PF <= L, "a round's batch scales are computed by the first PF lanes of each row group");

    __shared__ float tab[4][2][HALF];  // per wave: cos | sin (theta staged in the cos half)
    __shared__ float wt[2][D];         // Q and K norm weights

    const int      lane = threadIdx.x & 63;
    const uint32_t wv   = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int      j    = lane % L;
    const int      g    = lane / L;

    // per-lane byte offsets inside a batch, per segment
    int64_t lx[2], ly[2];
#pragma unroll
    for (int sg = 0; sg < 2; ++sg) {
        lx[sg] = (int64_t) g * a.seg[sg].xs1 + (int64_t) (j * VI) * EI;
        ly[sg] = (int64_t) g * a.seg[sg].ys1 + (int64_t) (j * VI) * EO;
    }

    const uint32_t ngroups = dgroups.d;
    const uint32_t nitems  = a.ntok * ngroups;
    const uint32_t stride  = gridDim.x * 4;

    auto decode = [&](uint32_t item) {
        HeadItem       it;
        const uint32_t t = dgroups.div(item);
        it.bbeg          = (item - t * ngroups) * bpw;
        it.bend          = it.bbeg + bpw < nb ? it.bbeg + bpw : nb;
        it.i3            = a.dne2.div(t);
        it.i2            = t - it.i3 * a.ne2;
        return it;
    };
    // batch b: segment and first head row (both wave-uniform)
    auto seg_of = [&](uint32_t b, int & sg, uint32_t & h0) {
        sg = b >= nb0 ? 1 : 0;
        h0 = (b - (sg ? nb0 : 0u)) * R;
    };
    auto load_batch = [&](const HeadItem & it, uint32_t b0, uint4 * v0, uint4 * v1) {
#pragma unroll
        for (int k = 0; k < PF; ++k) {
            if (b0 + k < it.bend) {
                int      sg;
                uint32_t h0;
                seg_of(b0 + k, sg, h0);
                const HeadSeg & S  = a.seg[sg];
                const char *    xp = S.x + (int64_t) it.i3 * S.xs3 + (int64_t) it.i2 * S.xs2 + (int64_t) h0 * S.xs1 + lx[sg];
                v0[k]              = make_uint4(0, 0, 0, 0);
                v1[k]              = make_uint4(0, 0, 0, 0);
                if (h0 + g < S.heads) {
                    v0[k] = ld16(xp);
                    v1[k] = ld16(xp + (size_t) HALF * EI);
                }
            }
        }
    };

    // one item: rows of `it` arrive in c0/c1 (first PF batches already
    // issued); the next item's first batches are issued into n0/n1
    auto step = [&](uint32_t item, HeadItem & it, uint4 * c0, uint4 * c1, uint4 * n0, uint4 * n1) {
        const uint32_t nxt    = item + stride;
        const bool     one    = it.bend - it.bbeg <= (uint32_t) PF;  // a single load round
        HeadItem       nx     = it;
        // the next item's position is a scalar load, so that waiting for it
        // never waits for the rows in flight
        auto           ahead  = [&]() {
            if (nxt < nitems) {
                nx = decode(nxt);
                if constexpr (ROPE) {
                    nx.pos = ld_scalar_i32(a.pos, nx.i2);
                }
                load_batch(nx, nx.bbeg, n0, n1);
            }
        };
        if (one) {
            ahead();
        }

        float cv[VI], sv[VI];
        if constexpr (ROPE) {
            float *     ct = tab[wv][0];
            float *     st = tab[wv][1];
            const float p  = (float) it.pos;  // loaded with the item's rows (scalar)
            if (lane == 0) {
                float th = p;
                ct[0]    = th;
                for (int i = 1; i < HALF; ++i) {
                    th    = th * a.theta_scale;
                    ct[i] = th;
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            __builtin_amdgcn_wave_barrier();
            float th[PL];
#pragma unroll
            for (int q = 0; q < PL; ++q) {
                th[q] = lane + 64 * q < HALF ? ct[lane + 64 * q] : 0.0f;
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int q = 0; q < PL; ++q) {
                if (lane + 64 * q < HALF) {
                    float sn, cs;
                    sincos_rot(a.freq_scale * th[q], &sn, &cs);
                    ct[lane + 64 * q] = cs * a.mscale;
                    st[lane + 64 * q] = sn * a.mscale;
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int e = 0; e < VI; ++e) {
                cv[e] = ct[j * VI + e];
                sv[e] = st[j * VI + e];
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            __builtin_amdgcn_wave_barrier();
        }

        for (uint32_t b0 = it.bbeg; b0 < it.bend; b0 += PF) {
            if (b0 > it.bbeg) {
                load_batch(it, b0, c0, c1);
                if (b0 + PF >= it.bend) {
                    ahead();
                }
            }
            // the round's row scales in one pass: after the row sums, lane j < PF
            // of each L-lane group takes batch j's sum and computes its scale;
            // batch k's rows then read lane k of their group
            float scl = 1.0f;
            if constexpr (NORM) {
                sq_t<TI> mine = 0;
#pragma unroll
                for (int k = 0; k < PF; ++k) {
                    float x0[VI], x1[VI];
                    unpack16<TI>(c0[k], x0);
                    unpack16<TI>(c1[k], x1);
                    sq_t<TI> ss = 0;
#pragma unroll
                    for (int e = 0; e < VI; ++e) {
                        ss = sq_acc<TI>(ss, x0[e]);
                    }
#pragma unroll
                    for (int e = 0; e < VI; ++e) {
                        ss = sq_acc<TI>(ss, x1[e]);
                    }
                    ss   = group_sum<L>(ss);
                    mine = j == k ? ss : mine;
                }
                scl = rms_scale(mine, D, a.eps);
                // unpack again below rather than keeping the round's floats live
                // (that costs a wave slot per SIMD)
#pragma unroll
                for (int k = 0; k < PF; ++k) {
                    opaque(c0[k]);
                    opaque(c1[k]);
                }
            }
#pragma unroll
            for (int k = 0; k < PF; ++k) {
                if (b0 + k >= it.bend) {
                    continue;
                }
                int      sg;
                uint32_t h0;
                seg_of(b0 + k, sg, h0);
                float x0[VI], x1[VI];
                unpack16<TI>(c0[k], x0);
                unpack16<TI>(c1[k], x1);
                if constexpr (NORM) {
                    const float   scale = __shfl(scl, g * L + k, 64);
                    const float * w     = wt[sg];
#pragma unroll
                    for (int e = 0; e < VI; ++e) {
                        x0[e] = x0[e] * scale * w[j * VI + e];
                        x1[e] = x1[e] * scale * w[HALF + j * VI + e];
                    }
                }
                if constexpr (ROPE) {
#pragma unroll
                    for (int e = 0; e < VI; ++e) {
                        const float a0  = x0[e] * cv[e];
                        const float b0_ = x1[e] * sv[e];
                        const float a1  = x0[e] * sv[e];
                        const float b1  = x1[e] * cv[e];
                        x0[e]           = a0 - b0_;
                        x1[e]           = a1 + b1;
                    }
                }
                const HeadSeg & S = a.seg[sg];
                if (h0 + g < S.heads) {
                    char * yp = S.y + (int64_t) it.i3 * S.ys3 + (int64_t) it.i2 * S.ys2 + (int64_t) h0 * S.ys1 + ly[sg];
                    store_vec<TO, VI>(yp, x0);
                    store_vec<TO, VI>(yp + (size_t) HALF * EO, x1);
                }
            }
        }
        it = nx;
    };

    uint4    va0[PF], va1[PF], vb0[PF], vb1[PF];
    uint32_t item = blockIdx.x * 4 + wv;
    HeadItem it{};
    if (item < nitems) {
        it = decode(item);
        if constexpr (ROPE) {
            it.pos = ld_scalar_i32(a.pos, it.i2);
        }
        load_batch(it, it.bbeg, va0, va1);
    }
    if constexpr (NORM) {
        for (int i = threadIdx.x; i < 2 * D; i += 256) {
            const float * w = i < D ? a.seg[0].w : (a.nseg > 1 ? a.seg[1].w : nullptr);
            wt[i / D][i % D] = w ? w[i % D] : 1.0f;
        }
        __syncthreads();
    }
    while (item < nitems) {
        step(item, it, va0, va1, vb0, vb1);
        item += stride;
        if (item >= nitems) {
            break;
        }
        step(item, it, vb0, vb1, va0, va1);
        item += stride;
    }
}

template <int TI, int TO>
__global__ void __launch_bounds__(256) k_heads_generic(const HeadArgs a) {
    constexpr int EI   = TT<TI>::ES;
    constexpr int EO   = TT<TO>::ES;
    const int     lane = threadIdx.x & 63;
    const int     wpb  = blockDim.x >> 6;
    const int     half = a.n_dims / 2;
    for (int sgi = 0; sgi < a.nseg; ++sgi) {
        const HeadSeg & S     = a.seg[sgi];
        const uint64_t  nrows = (uint64_t) a.ntok * S.heads;
        for (uint64_t r = (uint64_t) blockIdx.x * wpb + (threadIdx.x >> 6); r < nrows; r += (uint64_t) gridDim.x * wpb) {
            const uint32_t t  = (uint32_t) (r / S.heads);
            const uint32_t h  = (uint32_t) (r - (uint64_t) t * S.heads);
            const uint32_t i3 = a.dne2.div(t);
            const uint32_t i2 = t - i3 * a.ne2;
            const char *   xp = S.x + (int64_t) i3 * S.xs3 + (int64_t) i2 * S.xs2 + (int64_t) h * S.xs1;
            char *         yp = S.y + (int64_t) i3 * S.ys3 + (int64_t) i2 * S.ys2 + (int64_t) h * S.ys1;
            float          scale = 1.0f;
            if (a.norm) {
                sq_t<TI> s = 0;  // the fast kernels' accumulator: double for F32 rows, fp32 fma for BF16/F16
                for (int i = lane; i < a.ne0; i += 64) {
                    const float f = load_elem<TI>(xp + (size_t) i * EI);
                    s             = sq_acc<TI>(s, f);
                }
                s     = group_sum<64>(s);
                scale = rms_scale(s, a.ne0, a.eps);
            }
            auto nval = [&](int i) {
                float v = load_elem<TI>(xp + (size_t) i * EI);
                if (a.norm) {
                    v = v * scale;
                    if (S.w) {
                        v = v * S.w[i];
                    }
                }
                return v;
            };
            if (a.pos) {
                const float p = (float) a.pos[i2];
                for (int ic = lane; ic < half; ic += 64) {
                    float theta = p;
                    for (int k = 0; k < ic; ++k) {
                        theta = theta * a.theta_scale;
                    }
                    const float th = a.freq_scale * theta;
                    float       sv, cv;
                    sincos_rot(th, &sv, &cv);
                    const float c  = cv * a.mscale;
                    const float sn = sv * a.mscale;
                    const float x0 = nval(ic);
                    const float x1 = nval(ic + half);
                    const float a0 = x0 * c;
                    const float b0 = x1 * sn;
                    const float a1 = x0 * sn;
                    const float b1 = x1 * c;
                    store_elem<TO>(yp + (size_t) ic * EO, a0 - b0);
                    store_elem<TO>(yp + (size_t) (ic + half) * EO, a1 + b1);
                }
                for (int i = a.n_dims + lane; i < a.ne0; i += 64) {
                    store_elem<TO>(yp + (size_t) i * EO, nval(i));
                }
            } else {
                for (int i = lane; i < a.ne0; i += 64) {
                    store_elem<TO>(yp + (size_t) i * EO, nval(i));
                }
            }
        }
    }
}

// Grid of the workgroups (4 waves, one item each at a time) that fit on the
// chip at once, or fewer when there are fewer items; each kernel's
// occupancy is queried once.
template <auto kernel, typename... Args>
static void launch_persistent(uint64_t items, hipStream_t s, Args... args) {
    static const int per_cu = [&]() {
        int n = 0;
        if (MI_ROPE_WG_PER_CU > 0 ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void *>(kernel), 256, 0) !=
                hipSuccess ||
            n < 1) {
            n = MI_ROPE_WG_PER_CU > 0 ? MI_ROPE_WG_PER_CU : 4;
        }
        return n;
    }();
    uint64_t       grid = (items + 3) / 4;
    const uint64_t cap  = (uint64_t) num_cus() * (uint64_t) per_cu;
    grid                = grid > cap ? cap : grid;
    MI_LAUNCH(kernel, dim3((uint32_t) grid), dim3(256), 0, s, args...);
}

template <int TI, int TC, int D, int ROUND, bool TOCACHE>
__global__ void k_heads_kv(const HeadArgs a, const HeadKV kv, uint32_t nbq, uint32_t nbk, FastDiv dnbt);

template <int TI, int TO, int D>
static void launch_fast(const HeadArgs & a, hipStream_t s) {
    {
        // Tokens with more head batches than one load round (F32 rows: Qwen3's
        // 16 + 8 or 32 + 8 heads of 128 are 6 or 10 batches of 4 rows) take the
        // one-shot kernel, a wave per (token, batch) with its own cos/sin: the
        // persistent kernel would walk those batches in several dependent rounds.
        constexpr int  L   = D / 2 / TT<TI>::VEC;
        constexpr int  R   = 64 / L;
        const uint32_t nbq = (a.seg[0].heads + R - 1) / R;
        const uint32_t nbk = a.nseg > 1 ? (a.seg[1].heads + R - 1) / R : 0u;
        if (nbq + nbk > (uint32_t) MI_ROPE_PF) {
            const uint64_t waves = (uint64_t) a.ntok * (nbq + nbk);
            HeadKV         kv{};
            MI_LAUNCH((k_heads_kv<TI, TI, D, 0, false>), dim3((uint32_t) ((waves + 3) / 4)), dim3(256), 0,
                               s, a, kv, nbq, nbk, FastDiv(nbq + nbk));
            return;
        }
    }
    constexpr int  L   = D / 2 / TT<TI>::VEC;
    constexpr int  R   = 64 / L;
    const uint32_t h0  = a.seg[0].heads;
    const uint32_t h1  = a.nseg > 1 ? a.seg[1].heads : 0u;
    const uint32_t nb0 = (h0 + R - 1) / R;
    const uint32_t nb  = nb0 + (h1 + R - 1) / R;
    // one wave per token when there are enough tokens to fill the chip (cos/sin
    // computed once per token); otherwise split each token's batches over up to
    // nb waves so that every wave makes a single memory round trip
    const uint64_t want = (uint64_t) num_cus() * 8;
    uint32_t       grp  = (uint32_t) ((want + a.ntok - 1) / a.ntok);
#if MI_ROPE_ONE_ROUND
    // at most PF batches per item: one load round, which the item before it
    // already issued (the cos/sin table is then built once per item)
    const uint32_t rounds = (nb + MI_ROPE_PF - 1) / MI_ROPE_PF;
    grp                   = grp < rounds ? rounds : grp;
#endif
    grp                 = grp < 1 ? 1 : (grp > nb ? nb : grp);
    const uint32_t bpw  = (nb + grp - 1) / grp;
    grp                 = (nb + bpw - 1) / bpw;
    const uint64_t items = (uint64_t) a.ntok * grp;
    const FastDiv  dg(grp);
    const bool     rope = a.pos != nullptr;
    if (a.norm && rope) {
        launch_persistent<k_heads<TI, TO, D, true, true>>(items, s, a, nb0, nb, bpw, dg);
    } else if (a.norm) {
        launch_persistent<k_heads<TI, TO, D, true, false>>(items, s, a, nb0, nb, bpw, dg);
    } else {
        launch_persistent<k_heads<TI, TO, D, false, true>>(items, s, a, nb0, nb, bpw, dg);
    }
}

template <int TI, int TO>
static int launch_t(HeadArgs & a, bool fast, hipStream_t s) {
    if (fast) {
        switch (a.ne0) {
            case 64:
                launch_fast<TI, TO, 64>(a, s);
                return MI_OK;
            case 128:
                launch_fast<TI, TO, 128>(a, s);
                return MI_OK;
            case 256:
                launch_fast<TI, TO, 256>(a, s);
                return MI_OK;
            default:
                break;
        }
    }
    uint64_t rows = 0;
    for (int i = 0; i < a.nseg; ++i) {
        rows = rows > (uint64_t) a.ntok * a.seg[i].heads ? rows : (uint64_t) a.ntok * a.seg[i].heads;
    }
    uint64_t grid = (rows + 3) / 4;
    const uint64_t cap = (uint64_t) num_cus() * 16;
    grid = grid > cap ? cap : (grid ? grid : 1);
    MI_LAUNCH((k_heads_generic<TI, TO>), dim3((uint32_t) grid), dim3(256), 0, s, a);
    return MI_OK;
}

int launch_heads(HeadArgs & a, int tin, int tout, hipStream_t s) {
    if (a.ntok == 0) {
        return MI_OK;
    }
    a.dne2 = FastDiv(a.ne2);
    // fast path preconditions: full-width rotation (or none), D in {64,128,256},
    // 16-byte aligned rows, same in/out type
    const uint64_t hall = (uint64_t) a.seg[0].heads + (a.nseg > 1 ? a.seg[1].heads : 0u);
    bool fast = (a.pos == nullptr || a.n_dims == a.ne0) && (a.ne0 == 64 || a.ne0 == 128 || a.ne0 == 256) &&
                tin == tout && (a.norm || a.pos) && (uint64_t) a.ntok * hall < (1ull << 31);
    for (int i = 0; i < a.nseg && fast; ++i) {
        const HeadSeg & S = a.seg[i];
        fast = aligned(S.x, 16) && aligned(S.y, 16) && S.xs1 % 16 == 0 && S.xs2 % 16 == 0 && S.xs3 % 16 == 0 &&
               S.ys1 % 16 == 0 && S.ys2 % 16 == 0 && S.ys3 % 16 == 0 && (!S.w || aligned(S.w, 16));
    }
    switch (tin) {
        case MI_TYPE_F32:
            switch (tout) {
                case MI_TYPE_F32:
                    return launch_t<MI_TYPE_F32, MI_TYPE_F32>(a, fast, s);
                case MI_TYPE_BF16:
                    return launch_t<MI_TYPE_F32, MI_TYPE_BF16>(a, false, s);
                default:
                    return launch_t<MI_TYPE_F32, MI_TYPE_F16>(a, false, s);
            }
        case MI_TYPE_BF16:
            switch (tout) {
                case MI_TYPE_F32:
                    return launch_t<MI_TYPE_BF16, MI_TYPE_F32>(a, false, s);
                case MI_TYPE_BF16:
                    return launch_t<MI_TYPE_BF16, MI_TYPE_BF16>(a, fast, s);
                default:
                    return launch_t<MI_TYPE_BF16, MI_TYPE_F16>(a, false, s);
            }
        default:
            switch (tout) {
                case MI_TYPE_F32:
                    return launch_t<MI_TYPE_F16, MI_TYPE_F32>(a, false, s);
                case MI_TYPE_BF16:
                    return launch_t<MI_TYPE_F16, MI_TYPE_BF16>(a, false, s);
                default:
                    return launch_t<MI_TYPE_F16, MI_TYPE_F16>(a, fast, s);
            }
    }
}

}  // namespace mi

// ---------------------------------------------------------------------------
// QK-norm -> rope fused with the KV-cache store (decode: qwen3-lm.h:660-703);
// with TOCACHE false, the one-shot form of the plain QK-norm -> rope (K to its
// output like Q, no V batches).
// One wave per (token, batch of R head rows) over the Q, K and V batches of
// every token, with k_heads' lane layout and arithmetic (the same VI-element
// chunks per lane, the same row sums and group reduction, the same theta chain
// and sincos_rot), so Q equals mi_qk_norm_rope's output bit for bit and the
// cache holds what mi_kv_store writes from it. K is rounded to the activation
// type before the cache cast, as the separate ops store and reload it; V is
// clamped first when asked (qwen3-lm.h:674-677). Q8_0 caches: a 32-element
// block spans 32 / VI lanes of a row; they share the block's amax (DPP max),
// each writes its VI quants (2-byte aligned) and the first the fp16 scale.
namespace mi {

template <int TI, int TC, int D, int ROUND, bool TOCACHE = true>
__global__ void __launch_bounds__(256) k_heads_kv(const HeadArgs a, const HeadKV kv, uint32_t nbq, uint32_t nbk,
                                                  FastDiv dnbt) {
    constexpr int VI   = TT<TI>::VEC;
    constexpr int EI   = TT<TI>::ES;
    constexpr int HALF = D / 2;
    constexpr int L    = HALF / VI;  // lanes per head row
    constexpr int R    = 64 / L;     // head rows per batch
    constexpr int PL   = (HALF + 63) / 64;
    constexpr int LPB  = 32 / VI;    // lanes per Q8_0 block

    __shared__ float tab[4][2][HALF];

    const int      lane = threadIdx.x & 63;
    const uint32_t wv   = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int      j    = lane % L;
    const int      g    = lane / L;
    const uint32_t item = blockIdx.x * 4 + wv;
    if (item >= a.ntok * dnbt.d) {
        return;  // whole wave
    }
    const uint32_t tok = dnbt.div(item);
    const uint32_t bt  = item - tok * dnbt.d;
    const int      sg  = bt < nbq ? 0 : (bt < nbq + nbk ? 1 : 2);  // Q, K, V: wave-uniform
    const uint32_t h   = (bt - (sg == 0 ? 0u : sg == 1 ? nbq : nbq + nbk)) * R + g;
    const uint32_t i3  = a.dne2.div(tok);
    const uint32_t i2  = tok - i3 * a.ne2;
    const HeadSeg & S  = a.seg[sg == 0 ? 0 : 1];
    const bool     ok  = h < S.heads;  // V has K's heads

    // the position is a scalar load, so that the angle chain below waits for
    // it alone, not for the rows
    int32_t pos = 0;
    if (sg < 2 && a.pos) {
        pos = ld_scalar_i32(a.pos, i2);
    }
    const char * xp = sg == 2 ? kv.v + (int64_t) i3 * kv.vs3 + (int64_t) i2 * kv.vs2 + (int64_t) h * kv.vs1
                              : S.x + (int64_t) i3 * S.xs3 + (int64_t) i2 * S.xs2 + (int64_t) h * S.xs1;
    uint4 c0 = make_uint4(0, 0, 0, 0), c1 = make_uint4(0, 0, 0, 0);
    if (ok) {
        c0 = ld16(xp + (size_t) (j * VI) * EI);
        c1 = ld16(xp + (size_t) (HALF + j * VI) * EI);
    }
    float x0[VI], x1[VI];
    unpack16<TI>(c0, x0);
    unpack16<TI>(c1, x1);

    if (sg < 2) {
        float cv[VI], sv[VI];
        if (a.pos) {
            float *     ct = tab[wv][0];
            float *     st = tab[wv][1];
            const float p  = (float) pos;
            if (lane == 0) {
                float th = p;
                ct[0]    = th;
                for (int i = 1; i < HALF; ++i) {
                    th    = th * a.theta_scale;
                    ct[i] = th;
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            __builtin_amdgcn_wave_barrier();
            float th[PL];
#pragma unroll
            for (int q = 0; q < PL; ++q) {
                th[q] = lane + 64 * q < HALF ? ct[lane + 64 * q] : 0.0f;
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int q = 0; q < PL; ++q) {
                if (lane + 64 * q < HALF) {
                    float sn, cs;
                    sincos_rot(a.freq_scale * th[q], &sn, &cs);
                    ct[lane + 64 * q] = cs * a.mscale;
                    st[lane + 64 * q] = sn * a.mscale;
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int e = 0; e < VI; ++e) {
                cv[e] = ct[j * VI + e];
                sv[e] = st[j * VI + e];
            }
        }
        if (a.norm) {
            sq_t<TI> ss = 0;
#pragma unroll
            for (int e = 0; e < VI; ++e) {
                ss = sq_acc<TI>(ss, x0[e]);
            }
#pragma unroll
            for (int e = 0; e < VI; ++e) {
                ss = sq_acc<TI>(ss, x1[e]);
            }
            ss                = group_sum<L>(ss);
            const float scale = rms_scale(ss, D, a.eps);
            if (S.w) {
#pragma unroll
                for (int e = 0; e < VI; ++e) {
                    x0[e] = x0[e] * scale * S.w[j * VI + e];
                    x1[e] = x1[e] * scale * S.w[HALF + j * VI + e];
                }
            } else {
#pragma unroll
                for (int e = 0; e < VI; ++e) {
                    x0[e] = x0[e] * scale;
                    x1[e] = x1[e] * scale;
                }
            }
        }
        if (a.pos) {
#pragma unroll
            for (int e = 0; e < VI; ++e) {
                const float a0  = x0[e] * cv[e];
                const float b0_ = x1[e] * sv[e];
                const float a1  = x0[e] * sv[e];
                const float b1  = x1[e] * cv[e];
                x0[e]           = a0 - b0_;
                x1[e]           = a1 + b1;
            }
        }
        if (sg == 0 || !TOCACHE) {
            if (ok) {
                char * yp = S.y + (int64_t) i3 * S.ys3 + (int64_t) i2 * S.ys2 + (int64_t) h * S.ys1;
                store_vec<TI, VI>(yp + (size_t) (j * VI) * EI, x0);
                store_vec<TI, VI>(yp + (size_t) (HALF + j * VI) * EI, x1);
            }
            return;
        }
    } else if (kv.clamp_v) {
#pragma unroll
        for (int e = 0; e < VI; ++e) {
            const float c0_ = x0[e] < 65504.0f ? x0[e] : 65504.0f;
            const float c1_ = x1[e] < 65504.0f ? x1[e] : 65504.0f;
            x0[e]           = c0_ > -65504.0f ? c0_ : -65504.0f;
            x1[e]           = c1_ > -65504.0f ? c1_ : -65504.0f;
        }
    }
    // K or V to the cache, from the value the activation type holds
#pragma unroll
    for (int e = 0; e < VI; ++e) {
        x0[e] = round_to<TI>(x0[e]);
        x1[e] = round_to<TI>(x1[e]);
    }
    const uint32_t b    = kv.dT.div(tok);
    const int64_t  slot = (int64_t) kv.pos0[b] + (tok - b * kv.T);
    const int64_t  set  = kv.sets ? (int64_t) kv.sets[b] : (int64_t) b;
    if (slot < 0 || slot >= kv.max_seq || set < 0 || set >= kv.n_sets) {
        if (ok && j == 0 && kv.d_err) {
            atomicAdd(kv.d_err, 1);
        }
        return;
    }
    char * crow = (sg == 1 ? kv.kc : kv.vc) + slot * kv.cnb1 + (int64_t) h * kv.cnb2 + set * kv.cnb3;
    if constexpr (TC == MI_TYPE_Q8_0) {
#pragma unroll
        for (int part = 0; part < 2; ++part) {
            const float * f    = part ? x1 : x0;
            const int     el   = (part ? HALF : 0) + j * VI;  // first element of this lane's chunk
            float         amax = 0.0f;
#pragma unroll
            for (int e = 0; e < VI; ++e) {
                amax = fmaxf(amax, fabsf(f[e]));
            }
            amax          = group_max<LPB>(amax);
            const float d = div127(amax);
            float       id;
            if constexpr (ROUND == MI_Q8_0_REF) {
                id = d != 0.0f ? 1.0f / d : 0.0f;
            } else {
                id = amax != 0.0f ? 127.0f / amax : 0.0f;
            }
            uint32_t wq[VI / 4];
#pragma unroll
            for (int q = 0; q < VI / 4; ++q) {
                uint32_t acc = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float v = f[4 * q + e] * id;
                    float       r;
                    if constexpr (ROUND == MI_Q8_0_REF) {
                        r = round_half_away(v);
                    } else {
                        r = __builtin_amdgcn_fmed3f(__builtin_rintf(v), -128.0f, 127.0f);
                    }
                    acc |= ((uint32_t) (int32_t) r & 0xffu) << (8 * e);
                }
                wq[q] = acc;
            }
            if (ok) {
                char *     bp = crow + (size_t) (el / 32) * 34;
                uint16_t * qp = (uint16_t *) (bp + 2 + el % 32);
#pragma unroll
                for (int q = 0; q < VI / 4; ++q) {
                    qp[2 * q]     = (uint16_t) (wq[q] & 0xffffu);
                    qp[2 * q + 1] = (uint16_t) (wq[q] >> 16);
                }
                if (el % 32 == 0) {
                    *(uint16_t *) bp = f32_to_f16_bits(d);
                }
            }
        }
    } else {
        constexpr int EC = TT<TC>::ES;
        if (ok) {
            store_vec<TC, VI>(crow + (size_t) (j * VI) * EC, x0);
            store_vec<TC, VI>(crow + (size_t) (HALF + j * VI) * EC, x1);
        }
    }
}

template <int TI, int TC, int D>
static void launch_kv_d(const HeadArgs & a, const HeadKV & kv, int rounding, uint32_t nbq, uint32_t nbk,
                        uint32_t nbt, hipStream_t s) {
    const uint64_t waves = (uint64_t) a.ntok * nbt;
    const dim3     grid((uint32_t) ((waves + 3) / 4));
    if constexpr (TC == MI_TYPE_Q8_0) {
        if (rounding == MI_Q8_0_REF) {
            MI_LAUNCH((k_heads_kv<TI, TC, D, MI_Q8_0_REF>), grid, dim3(256), 0, s, a, kv, nbq, nbk,
                               FastDiv(nbt));
            return;
        }
    }
    MI_LAUNCH((k_heads_kv<TI, TC, D, MI_Q8_0_CPU_X86>), grid, dim3(256), 0, s, a, kv, nbq, nbk, FastDiv(nbt));
}

template <int TI, int TC>
static int launch_kv_t(const HeadArgs & a, const HeadKV & kv, int rounding, hipStream_t s) {
    const int      VI  = TT<TI>::VEC;
    const int      L   = a.ne0 / 2 / VI;
    const uint32_t R   = (uint32_t) (64 / L);
    const uint32_t nbq = (a.seg[0].heads + R - 1) / R;
    const uint32_t nbk = (a.seg[1].heads + R - 1) / R;
    const uint32_t nbt = nbq + 2 * nbk;
    switch (a.ne0) {
        case 64:
            launch_kv_d<TI, TC, 64>(a, kv, rounding, nbq, nbk, nbt, s);
            return MI_OK;
        case 128:
            launch_kv_d<TI, TC, 128>(a, kv, rounding, nbq, nbk, nbt, s);
            return MI_OK;
        case 256:
            launch_kv_d<TI, TC, 256>(a, kv, rounding, nbq, nbk, nbt, s);
            return MI_OK;
        default:
            return MI_ERR_UNSUPPORTED;
    }
}

template <int TI>
static int launch_kv_c(const HeadArgs & a, const HeadKV & kv, int tcache, int rounding, hipStream_t s) {
    switch (tcache) {
        case MI_TYPE_Q8_0:
            return launch_kv_t<TI, MI_TYPE_Q8_0>(a, kv, rounding, s);
        case MI_TYPE_F16:
            return launch_kv_t<TI, MI_TYPE_F16>(a, kv, rounding, s);
        case MI_TYPE_BF16:
            return launch_kv_t<TI, MI_TYPE_BF16>(a, kv, rounding, s);
        case MI_TYPE_F32:
            return launch_kv_t<TI, MI_TYPE_F32>(a, kv, rounding, s);
        default:
            return MI_ERR_TYPE;
    }
}

int launch_heads_kv(HeadArgs & a, const HeadKV & kv, int tin, int tcache, int rounding, hipStream_t s) {
    if (a.ntok == 0) {
        return MI_OK;
    }
    a.dne2 = FastDiv(a.ne2);
    // the k_heads fast-path layout: whole rotation (or none), 16-byte rows
    bool fast = (a.pos == nullptr || a.n_dims == a.ne0) && (a.ne0 == 64 || a.ne0 == 128 || a.ne0 == 256) &&
                (uint64_t) a.ntok * (a.seg[0].heads + 2ull * a.seg[1].heads) < (1ull << 31);
    for (int i = 0; i < 2 && fast; ++i) {
        const HeadSeg & S = a.seg[i];
        fast = aligned(S.x, 16) && S.xs1 % 16 == 0 && S.xs2 % 16 == 0 && S.xs3 % 16 == 0 && (!S.w || aligned(S.w, 16));
    }
    const HeadSeg & Q = a.seg[0];
    fast = fast && aligned(Q.y, 16) && Q.ys1 % 16 == 0 && Q.ys2 % 16 == 0 && Q.ys3 % 16 == 0;
    fast = fast && aligned(kv.v, 16) && kv.vs1 % 16 == 0 && kv.vs2 % 16 == 0 && kv.vs3 % 16 == 0;
    // cache rows: 16-byte vectors for F16/BF16/F32 (half a row for F32 of D = 64 is 128 bytes);
    // Q8_0 rows are 2-byte aligned blocks
    const size_t ca = tcache == MI_TYPE_Q8_0 ? 2 : 16;
    fast = fast && aligned(kv.kc, ca) && aligned(kv.vc, ca) && kv.cnb1 % ca == 0 && kv.cnb2 % ca == 0 &&
           kv.cnb3 % ca == 0;
    if (!fast) {
        return MI_ERR_UNSUPPORTED;
    }
    switch (tin) {
        case MI_TYPE_F32:
            return launch_kv_c<MI_TYPE_F32>(a, kv, tcache, rounding, s);
        case MI_TYPE_BF16:
            return launch_kv_c<MI_TYPE_BF16>(a, kv, tcache, rounding, s);
        default:
            return launch_kv_c<MI_TYPE_F16>(a, kv, tcache, rounding, s);
    }
}

}  // namespace mi
