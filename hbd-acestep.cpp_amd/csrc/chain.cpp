// chain.cpp -- per-layer drivers: the fused-op sequence of one ACE-Step DiT
// block (dit_ggml_build_layer, dit-graph.h:367-448) and of one Qwen3 decoder
// layer (qw3lm_forward_batch, qwen3-lm.h:630-741), launched back to back on
// one stream. The GEMM / attention outputs those builders produce between
// the fused ops are inputs here (this library does not compute them).
#include "mi_ops.h"
#include "validate.h"

#define MI_TRY(expr)            \
    do {                        \
        const int _rc = (expr); \
        if (_rc != MI_OK) {     \
            return _rc;         \
        }                       \
    } while (0)

namespace {

// ggml_view_1d(adaln, H, i*H*4) of a contiguous F32 [6H] tensor
mi_tensor vec_view(const mi_tensor & v, int64_t H, int i) {
    mi_tensor t = v;
    t.data      = (char *) v.data + (size_t) i * H * 4;
    t.ne[0]     = H;
    t.ne[1] = t.ne[2] = t.ne[3] = 1;
    t.nb[0]                     = 4;
    t.nb[1] = t.nb[2] = t.nb[3] = (uint64_t) H * 4;
    return t;
}

// [D, Nkv, n_tok] -> [D, Nkv, T, B] for a store at B sequence offsets
mi_tensor seq_view(const mi_tensor & x, int64_t B) {
    mi_tensor t = x;
    const int64_t n_tok = x.ne[2] * x.ne[3];
    t.ne[2]             = n_tok / B;
    t.ne[3]             = B;
    t.nb[3]             = x.nb[2] * (uint64_t) t.ne[2];
    return t;
}

}  // namespace

static int dit_block(const mi_dit_block_io * io, mi_stream s) {
    const int64_t H = io->hidden.ne[0];
    const mi_tensor & ad = io->adaln;
    if (ad.type != MI_TYPE_F32 || ad.ne[0] != 6 * H || ad.ne[1] != 1 || ad.ne[2] != 1 || ad.ne[3] != 1 ||
        ad.nb[0] != 4 || !ad.data) {
        return ad.data ? MI_ERR_SHAPE : MI_ERR_NULL;
    }
    // adaln = scale_shift_table + tproj, viewed as 6 vectors (dit-graph.h:391-400)
    const mi_tensor shift_sa = vec_view(ad, H, 0), scale_sa = vec_view(ad, H, 1), gate_sa = vec_view(ad, H, 2);
    const mi_tensor shift_ff = vec_view(ad, H, 3), scale_ff = vec_view(ad, H, 4), gate_ff = vec_view(ad, H, 5);

    // self-attention: RMSNorm*w -> AdaLN (dit-graph.h:404-405)
    MI_TRY(mi_rms_norm_modulate(&io->hidden, &io->sa_norm_w, &scale_sa, &shift_sa, io->eps, &io->norm_sa, s));
    // [QKV GEMM] -> QK-norm -> rope (dit-graph.h:183-198)
    MI_TRY(mi_qk_norm_rope(&io->q, &io->q_w, &io->q_out, &io->k, &io->k_w, &io->k_out, &io->pos, io->eps,
                           io->n_dims, io->rope_freq_base, 1.0f, 1.0f, s));
    // [FA, O-proj] -> gated residual (dit-graph.h:420), fused with the norm
    // that reads it: the cross-attention RMSNorm*w (429) or, without cross
    // attention, the FFN RMSNorm*w -> AdaLN (442-443)
    if (io->use_cross_attn) {
        MI_TRY(mi_add_rms_norm(&io->hidden, &io->sa_out, &gate_sa, 0, 0.0f, 0.0f, &io->ca_norm_w, nullptr, nullptr,
                               io->eps, &io->hidden, &io->norm_ca, s));
        // cross-attention Q-norm and K-norm, per head, no rope (328-331)
        if (io->ca_q.data) {
            MI_TRY(mi_rms_norm(&io->ca_q, &io->ca_q_w, io->eps, &io->ca_q_out, s));
        }
        if (io->ca_k.data) {
            MI_TRY(mi_rms_norm(&io->ca_k, &io->ca_k_w, io->eps, &io->ca_k_out, s));
        }
        // [CA, O-proj] -> residual add (432) fused with the FFN norm (442-443)
        MI_TRY(mi_add_rms_norm(&io->hidden, &io->ca_out, nullptr, 0, 0.0f, 0.0f, &io->ffn_norm_w, &scale_ff,
                               &shift_ff, io->eps, &io->hidden, &io->norm_ffn, s));
    } else {
        MI_TRY(mi_add_rms_norm(&io->hidden, &io->sa_out, &gate_sa, 0, 0.0f, 0.0f, &io->ffn_norm_w, &scale_ff,
                               &shift_ff, io->eps, &io->hidden, &io->norm_ffn, s));
    }
    // [gate_up GEMM] -> SwiGLU (259)
    MI_TRY(mi_swiglu(&io->gate_up, 0, &io->ff, s));
    // [down GEMM] -> gated residual (445)
    MI_TRY(mi_gated_add(&io->hidden, &io->ffn_out, &gate_ff, &io->hidden, s));
    return MI_OK;
}

// Every operand of the chain is validated (a launch-free pass through the
// same entry points) before the first kernel runs, so an error leaves the
// caller's buffers untouched.
extern "C" int mi_dit_block_ops(const mi_dit_block_io * io, mi_stream s) {
    if (!io) {
        return MI_ERR_NULL;
    }
    {
        mi::DryRunScope validate_only;
        MI_TRY(dit_block(io, s));
    }
    return dit_block(io, s);
}

// QK-norm -> rope (qwen3-lm.h:660-667) to q_out / k_out, the V clamp before
// the cache cast (674-677, in place), then the KV store of every sequence, K
// and V, in one launch (682-703)
static int qwen3_rope_and_store(const mi_qwen3_layer_io * io, mi_stream s) {
    const float lim = 65504.0f;
    MI_TRY(mi_qk_norm_rope(&io->q, &io->q_w, &io->q_out, &io->k, &io->k_w, &io->k_out, &io->pos, io->eps,
                           io->n_dims, io->rope_freq_base, 1.0f, 1.0f, s));
    if (io->clamp_fp16 && io->v.data) {
        MI_TRY(mi_add_clamp(&io->v, nullptr, -lim, lim, &io->v, s));
    }
    // KV-cache store: one launch for every sequence, K and V (682-703)
    if (io->k_cache.data) {
        const int64_t B = io->pos0.ne[0];
        const int64_t n_tok = io->k_out.ne[2] * io->k_out.ne[3];
        if (B <= 0 || n_tok % B != 0) {
            return MI_ERR_SHAPE;
        }
        const mi_tensor kk = seq_view(io->k_out, B);
        const mi_tensor vv = io->v.data ? seq_view(io->v, B) : mi_tensor{};
        MI_TRY(mi_kv_store(&kk, &io->k_cache, io->v.data ? &vv : nullptr, io->v.data ? &io->v_cache : nullptr,
                           &io->pos0, io->sets.data ? &io->sets : nullptr, io->kv_rounding, io->d_err, s));
    }
    return MI_OK;
}

static int qwen3_layer(const mi_qwen3_layer_io * io, mi_stream s) {
    const float lim = 65504.0f;
    // pre-attention RMSNorm (qwen3-lm.h:632)
    MI_TRY(mi_rms_norm(&io->hidden, &io->in_norm_w, io->eps, &io->norm, s));
    // [QKV GEMM] -> QK-norm -> rope (660-667), V clamp (674-677) and the KV store
    // (682-703) in one launch when the caller takes K from the cache only
    if (io->k_cache.data && !io->k_out.data) {
        if (!io->v.data) {
            return MI_ERR_NULL;
        }
        MI_TRY(mi_qk_norm_rope_kv_store(&io->q, &io->q_w, &io->q_out, &io->k, &io->k_w, &io->v, &io->pos, io->eps,
                                        io->n_dims,
                                        io->rope_freq_base, 1.0f, 1.0f, io->clamp_fp16, &io->k_cache, &io->v_cache,
                                        &io->pos0, io->sets.data ? &io->sets : nullptr, io->kv_rounding, io->d_err, s));
    } else {
        MI_TRY(qwen3_rope_and_store(io, s));
    }
    // [FA, O-proj] -> residual add (+ clamp) (730-733) fused with the
    // post-attention RMSNorm (736)
    MI_TRY(mi_add_rms_norm(&io->hidden, &io->attn_out, nullptr, io->clamp_fp16, -lim, lim, &io->post_norm_w, nullptr,
                           nullptr, io->eps, &io->hidden, &io->norm2, s));
    // [gate_up GEMM] -> SwiGLU (737)
    MI_TRY(mi_swiglu(&io->gate_up, 0, &io->ff, s));
    // [down GEMM] -> residual add (+ clamp) (738-741)
    if (io->clamp_fp16) {
        MI_TRY(mi_add_clamp(&io->hidden, &io->mlp_out, -lim, lim, &io->hidden, s));
    } else {
        MI_TRY(mi_add(&io->hidden, &io->mlp_out, &io->hidden, s));
    }
    return MI_OK;
}

// validated whole before the first launch, as mi_dit_block_ops
extern "C" int mi_qwen3_layer_ops(const mi_qwen3_layer_io * io, mi_stream s) {
    if (!io) {
        return MI_ERR_NULL;
    }
    {
        mi::DryRunScope validate_only;
        MI_TRY(qwen3_layer(io, s));
    }
    return qwen3_layer(io, s);
}
