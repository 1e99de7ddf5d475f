// ggml_mul_mat(w, x) with Q8_0 weights and F32 activations, the way ggml-cpu
// computes it: each row of x is quantized to Q8_0 (the x86 from_float:
// id = 127 / amax, round to nearest even, saturate), and each output is
// sum over blocks b of (d_w[b] * d_x[b]) * sum_i q_w[i] q_x[i] -- an exact int32
// dot per block, scaled in fp32 (ggml_vec_dot_q8_0_q8_0).
// Reference call sites: qwen3_linear (qwen3-enc.h:86-88) for the Q/K/V, O,
// gate/up and down projections, dit_ggml_linear (dit-graph.h:36-49), and the
// LM head over the Q8_0 token table (qwen3-lm.h:755).
//
// Weights are repacked once, at load, into the "R64" layout (lossless: the same
// 34 bytes per block): rows in groups of 64 (the last group zero-padded), and per
// (group g, block b) the 32 quants of the 64 rows as two 1 KB halves -- half j,
// lane l holds bytes [16 j, 16 j + 16) of row 64 g + l's block -- followed, after
// all quants, by the scales d[g][b][l] (fp16). A wave with lane = row then reads
// every quant byte with fully coalesced 16-byte loads.
//
// Matrix-vector kernel (up to 8 rows of x, the batched decode shapes): one wave
// per (row group, key split); lanes are weight rows, the quantized x is uniform
// across the wave and read through the scalar cache; sdot4 per 4 quants. Up to
// 8 key splits of a row group share a workgroup and are added in LDS in wave
// order; with more, each workgroup writes its partial sums and a small kernel
// adds them in workgroup order, so the result does not depend on scheduling.
#include "common.h"
#include "launch.h"

namespace mi {

__global__ void __launch_bounds__(256) k_q8_0_repack(const char * src, int64_t nb1, uint32_t n, uint32_t nbk,
                                                     uint32_t ng, char * dst) {
    const uint64_t i     = (uint64_t) blockIdx.x * 256u + threadIdx.x;  // ((g * nbk + b) * 64 + l)
    const uint64_t total = (uint64_t) ng * nbk * 64;
    if (i >= total) {
        return;
    }
    const uint32_t l   = (uint32_t) (i % 64);
    const uint64_t gb  = i / 64;
    const uint32_t b   = (uint32_t) (gb % nbk);
    const uint32_t row = (uint32_t) (gb / nbk) * 64 + l;
    uint32_t       q[8] = { 0, 0, 0, 0, 0, 0, 0, 0 };
    uint16_t       d    = 0;
    if (row < n) {
        const uint16_t * p = (const uint16_t *) (src + (int64_t) row * nb1 + (int64_t) b * 34);
        d                  = p[0];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            q[k] = (uint32_t) p[1 + 2 * k] | ((uint32_t) p[2 + 2 * k] << 16);
        }
    }
    char * qd = dst + gb * 2048 + 16 * l;
    *(uint4 *) qd          = make_uint4(q[0], q[1], q[2], q[3]);
    *(uint4 *) (qd + 1024) = make_uint4(q[4], q[5], q[6], q[7]);
    *(uint16_t *) (dst + (uint64_t) ng * nbk * 2048 + i * 2) = d;
}

// d = amax / 127, the IEEE quotient (q0 = amax * (1/127) corrected by one fma)
__device__ __forceinline__ float mm_div127(float amax) {
    constexpr float C  = 1.0f / 127.0f;
    const float     q0 = amax * C;
    const float     r  = __builtin_fmaf(-q0, 127.0f, amax);
    return __builtin_fmaf(r, C, q0);
}

// x rows -> Q8_0 (x86 rounding), block-major: quants xq[b][m][32] and widened
// scales xd[b][m] at a row stride mp >= m (the matrix-vector kernel reads all
// rows of a block in one 32 * m + 4 * m byte run with a few wide scalar loads;
// the matrix kernel reads 32-row tiles); 8 lanes per 32-element block, and the
// blocks of a wave are one block of 8 consecutive rows: each row's 128 input
// bytes are a whole line, and the wave's quants one contiguous 256-byte run.
#ifndef MI_QX_U
#define MI_QX_U 4  // blocks per 8-lane group, a grid stride apart, all loads issued first
#endif
__global__ void __launch_bounds__(256) k_mmv_quant_x(const MmvArgs a) {
    constexpr int  U     = MI_QX_U;
    const uint32_t gid   = blockIdx.x * 256u + threadIdx.x;
    const uint32_t grp   = gid / 8, sub = gid % 8;
    const uint32_t total = a.m * a.nbk;
    const uint32_t ngrp  = gridDim.x * 32u;  // 8-lane groups in the grid
    auto           ld4   = [&](const char * p, float (&v)[4]) {
        if (a.xvec) {
            const float4 q = *(const float4 *) p;
            v[0]           = q.x;
            v[1]           = q.y;
            v[2]           = q.z;
            v[3]           = q.w;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[e] = ((const float *) p)[e];
            }
        }
    };
    // the U blocks' inputs (g and u for the SwiGLU prologue), all in flight at once
    float f[U][4], h[U][4];
#pragma unroll
    for (int k = 0; k < U; ++k) {
        const uint32_t blk = grp + (uint32_t) k * ngrp;
        if (blk < total) {  // uniform over the 8 lanes of a block
            const uint32_t b = blk / a.m, m = blk - b * a.m;
            if (a.glu) {
                const int64_t off = (int64_t) m * a.gu1 + (int64_t) (b * 32 + sub * 4) * 4;
                ld4(a.g + off, f[k]);
                ld4(a.u + off, h[k]);
            } else {
                ld4(a.x + (int64_t) m * a.x1 + (int64_t) (b * 32 + sub * 4) * 4, f[k]);
            }
        }
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
        const uint32_t blk = grp + (uint32_t) k * ngrp;
        if (blk >= total) {
            break;  // whole groups of 8 lanes; later blocks are further out
        }
        const uint32_t b = blk / a.m, m = blk - b * a.m;
        float          x[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[e] = a.glu ? silu_f(f[k][e]) * h[k][e] : f[k][e];  // x = silu(g) * u, as mi_swiglu computes it
        }
        float amax = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
        amax       = group_max<8>(amax);
        const float d  = mm_div127(amax);
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        uint32_t    w  = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float q = __builtin_amdgcn_fmed3f(__builtin_rintf(x[e] * id), -128.0f, 127.0f);
            w |= ((uint32_t) (int32_t) q & 0xffu) << (8 * e);
        }
        *(uint32_t *) (a.xq + ((int64_t) b * a.mp + m) * 32 + sub * 4) = w;
        if (sub == 0) {
            a.xd[(int64_t) b * a.mp + m] = (float) __builtin_bit_cast(_Float16, f32_to_f16_bits(d));
        }
    }
}

// RMSNorm*w and the quantization of x in one kernel (the norm -> product
// prologue), one workgroup per row: the scale from the double sum of the float
// squares and x' = (x * scale) * w, the arithmetic of mi_rms_norm on F32 rows
// (only the order of the double additions differs, which leaves the float mean
// unchanged short of a double rounding tie); then x' is quantized as
// k_mmv_quant_x does, 8 lanes per 32-element block. With an addend (a.ab), x is
// the residual sum a.x + a.ab, written to a.sum in the first pass (the
// arithmetic of mi_add_rms_norm) and formed again from the two inputs in the
// second. With a gate (a.gate) the addend is scaled first, x + ab * gate (the
// arithmetic of mi_add_rms_norm's gated form); with a modulate (a.msc, a.msh)
// the normalized rows become (x' * (msc + 1)) + msh, each step rounded as
// mi_rms_norm_modulate rounds it.
__global__ void __launch_bounds__(256) k_mmv_quant_x_norm(const MmvArgs a) {
    __shared__ double red[4];
    __shared__ float  scl;
    const uint32_t m   = blockIdx.x;
    const int      tid = threadIdx.x;
    const char *   xr  = a.x + (int64_t) m * a.x1;
    auto           ld4 = [&](const char * p, float (&v)[4]) {
        if (a.xvec) {
            const float4 q = *(const float4 *) p;
            v[0]           = q.x;
            v[1]           = q.y;
            v[2]           = q.z;
            v[3]           = q.w;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[e] = ((const float *) p)[e];
            }
        }
    };
    const char * br = a.ab ? a.ab + (int64_t) m * a.ab1 : nullptr;
    // x (or the residual sum) at element i: 4 floats
    auto xv = [&](uint32_t i, float (&v)[4]) {
        ld4(xr + (size_t) i * 4, v);
        if (br) {
            float b4[4];
            ld4(br + (size_t) i * 4, b4);
            if (a.gate) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    b4[e] = b4[e] * a.gate[i + e];
                }
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[e] = v[e] + b4[e];
            }
        }
    };
    double ss = 0.0;
    for (uint32_t i = 4u * (uint32_t) tid; i < a.k; i += 1024u) {
        float v[4];
        xv(i, v);
        if (a.sum) {
            float * sp = (float *) (a.sum + (int64_t) m * a.sum1) + i;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                sp[e] = v[e];
            }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            ss += (double) (v[e] * v[e]);
        }
    }
    ss = group_sum<64>(ss);
    if ((tid & 63) == 0) {
        red[tid >> 6] = ss;
    }
    __syncthreads();
    if (tid == 0) {
        scl = rms_scale(red[0] + red[1] + red[2] + red[3], (int) a.k, a.eps);
    }
    __syncthreads();
    const float    scale = scl;
    const uint32_t sub   = (uint32_t) tid & 7u;
    for (uint32_t b = (uint32_t) tid >> 3; b < a.nbk; b += 32u) {  // the 8 lanes of a block share b
        const uint32_t i0 = b * 32u + sub * 4u;
        float          f[4];
        xv(i0, f);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float v = f[e] * scale;
            f[e]          = v * a.nw[i0 + e];
        }
        if (a.msc) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                f[e] = f[e] * (a.msc[i0 + e] + 1.0f);
                f[e] = f[e] + a.msh[i0 + e];
            }
        }
        float amax = fmaxf(fmaxf(fabsf(f[0]), fabsf(f[1])), fmaxf(fabsf(f[2]), fabsf(f[3])));
        amax       = group_max<8>(amax);
        const float d  = mm_div127(amax);
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        uint32_t    w  = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float q = __builtin_amdgcn_fmed3f(__builtin_rintf(f[e] * id), -128.0f, 127.0f);
            w |= ((uint32_t) (int32_t) q & 0xffu) << (8 * e);
        }
        *(uint32_t *) (a.xq + ((int64_t) b * a.mp + m) * 32 + sub * 4) = w;
        if (sub == 0) {
            a.xd[(int64_t) b * a.mp + m] = (float) __builtin_bit_cast(_Float16, f32_to_f16_bits(d));
        }
    }
}

// The same prologue for longer x (prefill): a workgroup per 8 consecutive rows.
// Lane (row r0 + l / 8, part l % 8) of wave w holds 4 elements of each of its
// row's blocks w, w + 4, ... in registers, all loaded at once: their float
// squares summed in double, over the row's 8 lanes and over the 4 waves (LDS),
// give the row's scale; the same registers are then scaled, multiplied by w,
// quantized and stored, so that each store instruction writes the 8 rows'
// quants of one block as one 256-byte run of the block-major layout (one
// workgroup per row wrote 32-byte pieces 32 * mp bytes apart). With an addend
// the residual sum is formed once and written in the first pass (ADD: a.ab is
// given, so that the plain prologue holds no registers for it); the gate and
// the modulate as in k_mmv_quant_x_norm. Rows of x are at most 4 * NBW blocks.
template <int NBW, bool ADD>
__global__ void __launch_bounds__(256) k_mmv_quant_x_norm8(const MmvArgs a) {
    __shared__ double red[4][8];
    __shared__ float  scl[8];
    const int      tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const uint32_t row = blockIdx.x * 8u + (uint32_t) (lane >> 3), sub = (uint32_t) lane & 7u;
    const bool     rv  = row < a.m;  // uniform over a row's 8 lanes
    const uint32_t rc  = rv ? row : a.m - 1;
    const char *   xr  = a.x + (int64_t) rc * a.x1;
    const char *   br  = ADD ? a.ab + (int64_t) rc * a.ab1 : nullptr;
    auto           ld4 = [&](const char * p, float (&v)[4]) {
        if (a.xvec) {
            const float4 q = *(const float4 *) p;
            v[0]           = q.x;
            v[1]           = q.y;
            v[2]           = q.z;
            v[3]           = q.w;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[e] = ((const float *) p)[e];
            }
        }
    };
    // every load unconditional (blocks past the row clamped to its last one), so
    // all are in flight before the first is used
    float v[NBW][4], u[ADD ? NBW : 1][4];
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
        const uint32_t b  = (uint32_t) wv + 4u * (uint32_t) j;
        const uint32_t bc = b < a.nbk ? b : a.nbk - 1;
        ld4(xr + (size_t) (bc * 32u + sub * 4u) * 4, v[j]);
        if constexpr (ADD) {
            ld4(br + (size_t) (bc * 32u + sub * 4u) * 4, u[j]);
        }
    }
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
        const uint32_t b = (uint32_t) wv + 4u * (uint32_t) j;
        if (b < a.nbk && rv) {
            if constexpr (ADD) {
                if (a.gate) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        u[j][e] = u[j][e] * a.gate[b * 32u + sub * 4u + e];
                    }
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[j][e] = v[j][e] + u[j][e];
                }
                if (a.sum) {
                    *(float4 *) ((float *) (a.sum + (int64_t) row * a.sum1) + b * 32u + sub * 4u) =
                        make_float4(v[j][0], v[j][1], v[j][2], v[j][3]);
                }
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                ss += (double) (v[j][e] * v[j][e]);
            }
        }
    }
    ss = group_sum<8>(ss);
    if (sub == 0) {
        red[wv][lane >> 3] = ss;
    }
    __syncthreads();
    if (tid < 8) {
        scl[tid] = rms_scale(red[0][tid] + red[1][tid] + red[2][tid] + red[3][tid], (int) a.k, a.eps);
    }
    __syncthreads();
    const float scale = scl[lane >> 3];
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
        const uint32_t b = (uint32_t) wv + 4u * (uint32_t) j;
        if (b >= a.nbk) {
            break;  // uniform over the wave
        }
        const uint32_t i0 = b * 32u + sub * 4u;
        float          f[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            f[e] = (v[j][e] * scale) * a.nw[i0 + e];
        }
        if (a.msc) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                f[e] = f[e] * (a.msc[i0 + e] + 1.0f);
                f[e] = f[e] + a.msh[i0 + e];
            }
        }
        float amax = fmaxf(fmaxf(fabsf(f[0]), fabsf(f[1])), fmaxf(fabsf(f[2]), fabsf(f[3])));
        amax       = group_max<8>(amax);
        const float d  = mm_div127(amax);
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        uint32_t    wq = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float q = __builtin_amdgcn_fmed3f(__builtin_rintf(f[e] * id), -128.0f, 127.0f);
            wq |= ((uint32_t) (int32_t) q & 0xffu) << (8 * e);
        }
        if (rv) {
            *(uint32_t *) (a.xq + ((int64_t) b * a.mp + row) * 32 + sub * 4) = wq;
            if (sub == 0) {
                a.xd[(int64_t) b * a.mp + row] = (float) __builtin_bit_cast(_Float16, f32_to_f16_bits(d));
            }
        }
    }
}

#ifndef MI_MMV_UNROLL
#define MI_MMV_UNROLL 4  // blocks whose weight loads are issued together
#endif

// y element (m, n) as stored: the product, or ggml_add(product, res) then, with
// rclamp, ggml_clamp -- the residual add fused after the product (one rounding,
// as the separate add; the add is commutative, so the operand order is ggml's)
__device__ __forceinline__ float mm_epilogue(const MmvArgs & a, uint32_t m, uint32_t n, float v) {
    if (a.res != nullptr) {
        if (a.rgate) {
            v = v * a.rgate[n];  // ggml_add(res, ggml_mul(product, gate)): the product rounded first
        }
        v = v + *(const float *) (a.res + (int64_t) m * a.res1 + (int64_t) n * 4);
        if (a.rclamp) {
            v = clamp_ggml(v, a.rlo, a.rhi);
        }
    }
    return v;
}

// The epilogue split in two for an output group: the residual values loaded
// first (all of a group's loads in flight together; callers clamp m and n into
// the output), then added (with the clamp) as mm_epilogue adds them.
__device__ __forceinline__ float mm_res(const MmvArgs & a, uint32_t m, uint32_t n) {
    return *(const float *) (a.res + (int64_t) m * a.res1 + (int64_t) n * 4);
}
__device__ __forceinline__ float mm_add_res(const MmvArgs & a, float v, float r, uint32_t n) {
    if (a.rgate) {
        v = v * a.rgate[n];
    }
    v = v + r;
    return a.rclamp ? clamp_ggml(v, a.rlo, a.rhi) : v;
}

template <int M>
__global__ void __launch_bounds__(512) k_mmv_q8_0(const MmvArgs a) {
    extern __shared__ float red[];  // [wave][m][lane], W * M * 64 floats when W > 1
    const uint32_t g = blockIdx.x, s1 = blockIdx.y;
    const int      tid = threadIdx.x, l = tid & 63;
    const int      w   = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: x loads stay scalar
    const int      W   = (int) a.wpg;
    const uint32_t s   = s1 * (uint32_t) W + (uint32_t) w;  // this wave's key split
    const uint32_t b0  = s * a.bps < a.nbk ? s * a.bps : a.nbk;
    const uint32_t b1  = b0 + a.bps < a.nbk ? b0 + a.bps : a.nbk;
    const char *   wq  = a.w + (uint64_t) g * a.nbk * 2048 + 16 * l;
    const char *   wd  = a.w + a.qbytes + (uint64_t) g * a.nbk * 128 + 2 * l;
    const char * __restrict__ xq  = a.xq;
    const float * __restrict__ xd = a.xd;
    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        acc[m] = 0.0f;
    }
    constexpr int U = MI_MMV_UNROLL;
    auto block = [&](const uint4 & w0, const uint4 & w1, uint16_t dh, uint32_t b) {
        const uint32_t wv[8] = { w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w };
        const float    dw    = (float) __builtin_bit_cast(_Float16, dh);
        const uint32_t * xb  = (const uint32_t *) (xq + (size_t) b * (M * 32));
        const float *    xdb = xd + (size_t) b * M;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            int isum = 0;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                isum = __builtin_amdgcn_sdot4((int) wv[k], (int) xb[8 * m + k], isum, false);
            }
            acc[m] = __builtin_fmaf((float) isum, dw * xdb[m], acc[m]);
        }
    };
    // two register sets of U blocks: the loads of one are in flight while the
    // other's dot products run
    uint4    a0[U], a1[U], c0[U], c1[U];
    uint16_t ad[U], cd[U];
    auto load = [&](uint4 (&w0)[U], uint4 (&w1)[U], uint16_t (&dh)[U], uint32_t bb) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            w0[u] = ld16(wq + (size_t) (bb + u) * 2048);
            w1[u] = ld16(wq + (size_t) (bb + u) * 2048 + 1024);
            dh[u] = *(const uint16_t *) (wd + (size_t) (bb + u) * 128);
        }
    };
    auto run = [&](const uint4 (&w0)[U], const uint4 (&w1)[U], const uint16_t (&dh)[U], uint32_t bb) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            block(w0[u], w1[u], dh[u], bb + u);
        }
    };
    uint32_t b = b0;
    if (b + U <= b1) {
        load(a0, a1, ad, b);
    }
    while (b + U <= b1) {
        const bool nc = b + 2 * U <= b1;
        if (nc) {
            load(c0, c1, cd, b + U);
        }
        run(a0, a1, ad, b);
        b += U;
        if (!nc) {
            break;
        }
        const bool na = b + 2 * U <= b1;
        if (na) {
            load(a0, a1, ad, b + U);
        }
        run(c0, c1, cd, b);
        b += U;
        if (!na) {
            break;
        }
    }
    for (; b < b1; ++b) {
        block(ld16(wq + (size_t) b * 2048), ld16(wq + (size_t) b * 2048 + 1024),
              *(const uint16_t *) (wd + (size_t) b * 128), b);
    }
    const uint32_t row = g * 64 + l;
    auto store_y = [&](int m, float v) {
        if (row < a.n) {
            *(float *) (a.y + (int64_t) m * a.y1 + (int64_t) row * 4) = mm_epilogue(a, (uint32_t) m, row, v);
        }
    };
    if (W == 1 && a.splits == 1) {
        if (a.res != nullptr) {
            const uint32_t rc = row < a.n ? row : a.n - 1;
            float          r[M];
#pragma unroll
            for (int m = 0; m < M; ++m) {
                r[m] = mm_res(a, (uint32_t) m, rc);
            }
#pragma unroll
            for (int m = 0; m < M; ++m) {
                if (row < a.n) {
                    *(float *) (a.y + (int64_t) m * a.y1 + (int64_t) row * 4) = mm_add_res(a, acc[m], r[m], row);
                }
            }
            return;
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
            store_y(m, acc[m]);
        }
        return;
    }
    // the workgroup's splits, added in wave order; wave w then owns rows m = w, w + W, ...
#pragma unroll
    for (int m = 0; m < M; ++m) {
        red[(w * M + m) * 64 + l] = acc[m];
    }
    __syncthreads();
    for (int m = w; m < M; m += W) {
        float v = 0.0f;
        for (int w2 = 0; w2 < W; ++w2) {
            v += red[(w2 * M + m) * 64 + l];
        }
        if (a.splits == 1) {
            store_y(m, v);
        } else {
            a.part[((size_t) s1 * M + m) * a.npad + row] = v;
        }
    }
}

// y[m][row] = sum over the workgroups' partials, in workgroup order (splits > 1)
template <int M>
__global__ void __launch_bounds__(256) k_mmv_reduce(const MmvArgs a) {
    const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
    if (gid >= M * a.npad) {
        return;
    }
    const uint32_t m = gid / a.npad, row = gid - m * a.npad;
    if (row >= a.n) {
        return;
    }
    const float * pp = a.part + (size_t) m * a.npad + row;
    const size_t  st = (size_t) M * a.npad;
    float         v  = 0.0f;
    uint32_t      s2 = 0;
    for (; s2 + 8 <= a.splits; s2 += 8) {
        float t[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            t[j] = pp[(s2 + j) * st];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            v += t[j];
        }
    }
    for (; s2 < a.splits; ++s2) {
        v += pp[s2 * st];
    }
    *(float *) (a.y + (int64_t) m * a.y1 + (int64_t) row * 4) = mm_epilogue(a, m, row, v);
}


// Matrix kernel (more than 8 rows of x: prefill, the DiT): a workgroup of 4
// waves owns 128 rows of x x 128 weight rows; each wave a 64 x 64 tile as 2 x 2
// v_mfma_i32_32x32x32_i8 tiles (D rows = rows of x, columns = weight rows, so a
// lane stores consecutive outputs). Per 32-element block: one MFMA per tile
// gives the exact int32 block dots, and acc = fma(float(isum), d_w * d_x, acc)
// scales them in block order -- the arithmetic of the matrix-vector kernel
// (the d_w * d_x products come from an f32 outer-product MFMA, exactly).
// Operands come straight from global memory in MFMA lane order: x from the
// block-major quantized rows (lane l: row l % 32, bytes 16 (l / 32) of the
// block), weights from the R64 layout (a 32-row half of a group is two 512-byte
// runs), so no LDS staging is needed; one block ahead is in flight.
#ifndef MI_MMQ_PRIO
#define MI_MMQ_PRIO 1  // > 0: the wave's issue priority while it issues a block's MFMAs
#endif
#ifndef MI_MMQ_WG_PER_CU
#define MI_MMQ_WG_PER_CU 2  // resident workgroups of the matrix kernel per CU (2 waves per SIMD)
#endif
#ifndef MI_MMQ_MAX_KSPLIT
#define MI_MMQ_MAX_KSPLIT 4  // key splits of the matrix kernel at most
#endif
#ifndef MI_MMQ_MIN_BPS
#define MI_MMQ_MIN_BPS 32  // blocks of 32 keys per split at least
#endif
typedef int mm_i32x4 __attribute__((ext_vector_type(4)));
typedef int mm_i32x16 __attribute__((ext_vector_type(16)));
typedef float mm_f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 mm_f16x8 __attribute__((ext_vector_type(8)));

__global__ void __launch_bounds__(256) k_mmq_q8_0(const MmvArgs a) {
    const int      tid = threadIdx.x, l = tid & 63, wv = tid >> 6;
    const int      hh  = l >> 5, c = l & 31;
    const uint32_t m0  = blockIdx.y * 128 + (wv >> 1) * 64;  // rows of x (padded to 128)
    const uint32_t n0  = blockIdx.x * 128 + (wv & 1) * 64;   // weight rows
    const uint32_t g   = n0 / 64;                             // R64 row group
    if (g >= a.ng) {
        return;  // whole wave
    }
    const char *   wq = a.w + (uint64_t) g * a.nbk * 2048 + (size_t) hh * 1024 + 16 * c;
    const char *   wd = a.w + a.qbytes + (uint64_t) g * a.nbk * 128 + 2 * c;
    const char *   xq = a.xq + (size_t) (m0 + c) * 32 + hh * 16;
    const float *  xd = a.xd + m0;
    const uint64_t xqs = (uint64_t) a.mp * 32;  // per block
    float          acc[2][2][16];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                acc[i][j][e] = 0.0f;
            }
        }
    }
    struct Blk {
        uint4    x[2], w[2];
        uint16_t dw[2];
        float    dx[2];
    };
    auto load = [&](Blk & k, uint32_t b) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {  // x tile i: rows m0 + 32 i + c
            k.x[i]  = *(const uint4 *) (xq + b * xqs + (size_t) i * 32 * 32);
            k.dx[i] = xd[(size_t) b * a.mp + 32 * i + c];
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {  // weight tile j: rows n0 + 32 j + c
            k.w[j]  = *(const uint4 *) (wq + (size_t) b * 2048 + 512 * j);  // cached: every row tile of x reads it
            k.dw[j] = *(const uint16_t *) (wd + (size_t) b * 128 + 64 * j);
        }
    };
    // the block's scales d_x[m] d_w[n] as a 32 x 32 outer product on the matrix
    // core, in the D layout of the int32 dots, so each output costs one
    // conversion and one fma. Both scales are fp16 values (d_x was rounded to
    // fp16 when x was quantized), so an fp16 MFMA with k-slot 0 carrying them and
    // the other 15 slots zero forms every product exactly, at half the matrix-core
    // time of an fp32 outer product.
    auto run = [&](const Blk & k) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const mm_i32x4 av = { (int) k.x[i].x, (int) k.x[i].y, (int) k.x[i].z, (int) k.x[i].w };
            mm_f16x8       sx = {};
            sx[0]             = hh == 0 ? (_Float16) k.dx[i] : (_Float16) 0.0f;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const mm_i32x4  bv = { (int) k.w[j].x, (int) k.w[j].y, (int) k.w[j].z, (int) k.w[j].w };
                if constexpr (MI_MMQ_PRIO > 0) {
                    __builtin_amdgcn_s_setprio(MI_MMQ_PRIO);
                }
                const mm_i32x16 d  = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, mm_i32x16{}, 0, 0, 0);
                mm_f16x8        sw = {};
                sw[0]              = hh == 0 ? __builtin_bit_cast(_Float16, k.dw[j]) : (_Float16) 0.0f;
                const mm_f32x16 sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(sx, sw, mm_f32x16{}, 0, 0, 0);
                if constexpr (MI_MMQ_PRIO > 0) {
                    __builtin_amdgcn_s_setprio(0);
                }
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    acc[i][j][e] = __builtin_fmaf((float) d[e], sc[e], acc[i][j][e]);
                }
            }
        }
    };
    // this workgroup's blocks: split blockIdx.z of the key range
    const uint32_t bb = blockIdx.z * a.bps;
    const uint32_t be = bb + a.bps < a.nbk ? bb + a.bps : a.nbk;
    Blk            k0, k1;
    uint32_t       b = bb;
    if (b < be) {
        load(k0, b);
    }
    while (b < be) {
        const bool n1 = b + 1 < be;
        if (n1) {
            load(k1, b + 1);
        }
        run(k0);
        ++b;
        if (!n1) {
            break;
        }
        const bool n0b = b + 1 < be;
        if (n0b) {
            load(k0, b + 1);
        }
        run(k1);
        ++b;
        if (!n0b) {
            break;
        }
    }
    if (a.splits > 1) {
        // the split's sums to the workspace [split][mp][npad] (every row and
        // column of the tile lies inside the padded extent); k_mmq_reduce adds
        // the splits in order and applies the epilogue
        float * pp = a.part + (size_t) blockIdx.z * a.mp * a.npad;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        pp[(size_t) (m0 + 32 * i + 8 * q + 4 * hh + e) * a.npad + n0 + 32 * j + c] = acc[i][j][4 * q + e];
                    }
                }
            }
        }
        return;
    }
    // D lane l: column n0 + 32 j + c, rows m0 + 32 i + 8 q + 4 hh + e; with a
    // residual, the 16 values of an (i, j) tile are loaded before any is added
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t n = n0 + 32 * j + c;
        if (n >= a.n) {
            continue;
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            float r[16];
            if (a.res != nullptr) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t m = m0 + 32 * i + 8 * q + 4 * hh + e;
                        r[4 * q + e]     = mm_res(a, m < a.m ? m : a.m - 1, n);
                    }
                }
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t m = m0 + 32 * i + 8 * q + 4 * hh + e;
                    if (m < a.m) {
                        const float v = acc[i][j][4 * q + e];
                        *(float *) (a.y + (int64_t) m * a.y1 + (int64_t) n * 4) =
                            a.res != nullptr ? mm_add_res(a, v, r[4 * q + e], n) : v;
                    }
                }
            }
        }
    }
}

// The matrix kernel's key splits added in split order, then the epilogue
// (residual, clamp): one thread per output, consecutive threads along a row.
__global__ void __launch_bounds__(256) k_mmq_reduce(const MmvArgs a) {
    const uint64_t gid = (uint64_t) blockIdx.x * 256u + threadIdx.x;
    const uint32_t m   = (uint32_t) (gid / a.n);
    const uint32_t n   = (uint32_t) (gid - (uint64_t) m * a.n);
    if (m >= a.m) {
        return;
    }
    const float *  pp  = a.part + (size_t) m * a.npad + n;
    const size_t   st  = (size_t) a.mp * a.npad;
    float          v[MI_MMQ_MAX_KSPLIT];
#pragma unroll
    for (int s2 = 0; s2 < MI_MMQ_MAX_KSPLIT; ++s2) {
        v[s2] = pp[(size_t) (s2 < (int) a.splits ? s2 : 0) * st];  // all loads before any add
    }
    float t = v[0];
#pragma unroll
    for (int s2 = 1; s2 < MI_MMQ_MAX_KSPLIT; ++s2) {
        if (s2 < (int) a.splits) {
            t += v[s2];
        }
    }
    *(float *) (a.y + (int64_t) m * a.y1 + (int64_t) n * 4) = mm_epilogue(a, m, n, t);
}

#ifndef MI_MMV_NORED_MIN
#define MI_MMV_NORED_MIN 8  // waves per CU from which key splits stop at one workgroup per row group (0: never)
#endif
#ifndef MI_MMV_WAVES_PER_CU
#define MI_MMV_WAVES_PER_CU 16  // waves to spread one product over, per CU
#endif

// key splits: enough waves to keep the loads of the whole chip in flight; up to
// 8 splits of a row group share a workgroup (reduced in LDS), the rest go
// through the workspace
void mul_mat_q8_0_plan(MmvArgs & a, int cus) {
    a.ng     = (a.n + 63) / 64;
    a.npad   = a.ng * 64;
    a.qbytes = (uint64_t) a.ng * a.nbk * 2048;
    a.mp     = a.m <= 8 ? a.m : (a.m + 127) / 128 * 128;
    if (a.m > 8) {
        // the matrix kernel: key splits (workspace partials, added by
        // k_mmq_reduce) only when its 128 x 128 tiles leave resident workgroup
        // slots empty -- the narrow products (n = H) at prefill sizes
        a.wpg             = 1;
        const uint64_t tl = (uint64_t) ((a.n + 127) / 128) * (a.mp / 128);
        const uint64_t sl = (uint64_t) (cus > 0 ? cus : 256) * MI_MMQ_WG_PER_CU;
        uint64_t       ks = tl < sl ? sl / tl : 1;
        ks                = ks > MI_MMQ_MAX_KSPLIT ? MI_MMQ_MAX_KSPLIT : ks;
        ks                = ks > a.nbk / MI_MMQ_MIN_BPS ? a.nbk / MI_MMQ_MIN_BPS : ks;
        ks                = ks < 1 ? 1 : ks;
        a.bps             = a.nbk == 0 ? 1 : (uint32_t) ((a.nbk + ks - 1) / ks);
        a.splits          = a.nbk == 0 ? 1 : (a.nbk + a.bps - 1) / a.bps;
        return;
    }
    const uint32_t want = (uint32_t) (cus > 0 ? cus : 256) * MI_MMV_WAVES_PER_CU;
    uint32_t       s    = a.ng == 0 || a.ng >= want ? 1 : (want + a.ng - 1) / a.ng;
    // when one workgroup per row group (its splits added in LDS) still gives the
    // grid enough waves, stop there: no partials, no second launch to add them
    if (MI_MMV_NORED_MIN > 0 && s > 8 && (uint64_t) a.ng * 8 >= (uint64_t) (cus > 0 ? cus : 256) * MI_MMV_NORED_MIN) {
        s = 8;
    }
    if (s > a.nbk) {
        s = a.nbk;
    }
    if (s < 1) {
        s = 1;
    }
    a.wpg    = s < 8 ? s : 8;
    a.splits = (s + a.wpg - 1) / a.wpg;                       // workgroups per row group
    a.bps    = a.nbk == 0 ? 1 : (a.nbk + a.splits * a.wpg - 1) / (a.splits * a.wpg);
}

static size_t al256(size_t v) {
    return (v + 255) & ~(size_t) 255;
}

size_t mul_mat_q8_0_workspace(const MmvArgs & a) {
    size_t b = al256((size_t) a.mp * a.k) + al256((size_t) a.mp * a.nbk * 4);
    if (a.splits > 1) {  // partials: [splits][m][npad], or [splits][mp][npad] for the matrix kernel
        b += al256((size_t) a.splits * (a.m > 8 ? a.mp : a.m) * a.npad * 4);
    }
    return b;
}

void mul_mat_q8_0_bind(MmvArgs & a, char * ws) {
    a.xq  = ws;
    a.xd  = (float *) (ws + al256((size_t) a.mp * a.k));
    char * p = (char *) a.xd + al256((size_t) a.mp * a.nbk * 4);
    a.part = a.splits > 1 ? (float *) p : nullptr;
}

int launch_q8_0_repack(const char * src, int64_t nb1, uint32_t k, uint32_t n, char * dst, hipStream_t s) {
    const uint32_t nbk   = k / 32, ng = (n + 63) / 64;
    const uint64_t total = (uint64_t) ng * nbk * 64;
    if (total == 0) {
        return MI_OK;
    }
    MI_LAUNCH(k_q8_0_repack, dim3((uint32_t) ((total + 255) / 256)), dim3(256), 0, s, src, nb1, n, nbk, ng,
                       dst);
    return MI_OK;
}

#ifndef MI_QXN8_MIN_ROWS
#define MI_QXN8_MIN_ROWS 4096  // rows of x from which the norm prologue takes 8 rows per workgroup
#endif
template <bool ADD>
static void launch_quant_x_norm8(const MmvArgs & a, hipStream_t s) {
    const dim3 grid((a.m + 7) / 8);
    if (a.nbk <= 4 * 8) {
        MI_LAUNCH((k_mmv_quant_x_norm8<8, ADD>), grid, dim3(256), 0, s, a);
    } else if (a.nbk <= 4 * 16) {
        MI_LAUNCH((k_mmv_quant_x_norm8<16, ADD>), grid, dim3(256), 0, s, a);
    } else if (a.nbk <= 4 * 24) {
        MI_LAUNCH((k_mmv_quant_x_norm8<24, ADD>), grid, dim3(256), 0, s, a);
    } else {
        MI_LAUNCH((k_mmv_quant_x_norm8<32, ADD>), grid, dim3(256), 0, s, a);
    }
}

int launch_mul_mat_q8_0(const MmvArgs & a, hipStream_t s) {
    if (a.n == 0 || a.m == 0) {
        return MI_OK;
    }
    if (a.nw && a.m >= (uint32_t) MI_QXN8_MIN_ROWS && a.nbk <= 4 * 32) {
        // long x: 8 rows per workgroup, x held in registers (4 * NBW blocks per row at most)
        if (a.ab) {
            launch_quant_x_norm8<true>(a, s);
        } else {
            launch_quant_x_norm8<false>(a, s);
        }
    } else if (a.nw) {
        MI_LAUNCH(k_mmv_quant_x_norm, dim3(a.m), dim3(256), 0, s, a);
    } else {
        const uint64_t threads = ((uint64_t) a.m * a.nbk + MI_QX_U - 1) / MI_QX_U * 8;
        MI_LAUNCH(k_mmv_quant_x, dim3((uint32_t) ((threads + 255) / 256)), dim3(256), 0, s, a);
    }
    if (a.m > 8) {
        MI_LAUNCH(k_mmq_q8_0, dim3((a.n + 127) / 128, a.mp / 128, a.splits), dim3(256), 0, s, a);
        if (a.splits > 1) {
            const uint64_t outs = (uint64_t) a.m * a.n;
            MI_LAUNCH(k_mmq_reduce, dim3((uint32_t) ((outs + 255) / 256)), dim3(256), 0, s, a);
        }
        return MI_OK;
    }
    const dim3   grid(a.ng, a.splits), blk(64 * a.wpg);
    const size_t lds = a.wpg > 1 ? (size_t) a.wpg * a.m * 64 * 4 : 0;
    switch (a.m) {
        case 1: MI_LAUNCH(k_mmv_q8_0<1>, grid, blk, lds, s, a); break;
        case 2: MI_LAUNCH(k_mmv_q8_0<2>, grid, blk, lds, s, a); break;
        case 3: MI_LAUNCH(k_mmv_q8_0<3>, grid, blk, lds, s, a); break;
        case 4: MI_LAUNCH(k_mmv_q8_0<4>, grid, blk, lds, s, a); break;
        case 5: MI_LAUNCH(k_mmv_q8_0<5>, grid, blk, lds, s, a); break;
        case 6: MI_LAUNCH(k_mmv_q8_0<6>, grid, blk, lds, s, a); break;
        case 7: MI_LAUNCH(k_mmv_q8_0<7>, grid, blk, lds, s, a); break;
        case 8: MI_LAUNCH(k_mmv_q8_0<8>, grid, blk, lds, s, a); break;
        default: return MI_ERR_UNSUPPORTED;
    }
    if (a.splits > 1) {
        const dim3 rg((a.m * a.npad + 255) / 256);
        switch (a.m) {
            case 1: MI_LAUNCH(k_mmv_reduce<1>, rg, dim3(256), 0, s, a); break;
            case 2: MI_LAUNCH(k_mmv_reduce<2>, rg, dim3(256), 0, s, a); break;
            case 3: MI_LAUNCH(k_mmv_reduce<3>, rg, dim3(256), 0, s, a); break;
            case 4: MI_LAUNCH(k_mmv_reduce<4>, rg, dim3(256), 0, s, a); break;
            case 5: MI_LAUNCH(k_mmv_reduce<5>, rg, dim3(256), 0, s, a); break;
            case 6: MI_LAUNCH(k_mmv_reduce<6>, rg, dim3(256), 0, s, a); break;
            case 7: MI_LAUNCH(k_mmv_reduce<7>, rg, dim3(256), 0, s, a); break;
            default: MI_LAUNCH(k_mmv_reduce<8>, rg, dim3(256), 0, s, a); break;
        }
    }
    return MI_OK;
}

}  // namespace mi
