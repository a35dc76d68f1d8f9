/* model_qwen.c - maps a qwen35 / qwen3_5 / qwen3 GGUF onto an sg_model.
 *
 * Interface: sg_model_from_gguf / sg_model_free (reference surge.h:345-347).
 * The key names, tensor names and GGUF semantics are the file format's and
 * therefore the same as the reference's mapping (reference
 * src/model_qwen.c:321-621):
 *   - config from <arch>.* keys; head_dim from attention.key_length;
 *     rope_dim from rope.dimension_count (hybrid), full rotary for dense qwen3;
 *   - DeltaNet dims from ssm.{group_count, state_size, time_step_rank,
 *     inner_size, conv_kernel}; head_v_dim = inner_size / time_step_rank;
 *   - vocab = length of tokenizer.ggml.tokens; tied when output.weight is absent;
 *   - per-layer tensors blk.N.*; layer kind by tensor presence;
 *   - GGUF semantics: ssm_a holds -exp(A_log), value heads are tiled,
 *     norms are absolute, every small tensor is F32.
 * Every tensor's dtype and element count is checked against the config.
 */
#include "surge.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static uint64_t elems_of(const sg_tensor *t) {
    uint64_t n = 1;
    for (uint32_t d = 0; d < t->n_dims; d++) n *= t->dims[d];
    return n;
}

typedef struct {
    const sg_gguf *g;
    sg_tensor_type mat;
    char name[160];
    const char *err;
} mapper;

/* Finds blk.<i>.<suffix>; checks dtype and element count when present.
 * Returns NULL when absent (or on a mismatch, with m->err set). */
static const void *tensor(mapper *m, uint32_t layer, const char *suffix,
                          sg_tensor_type want, uint64_t elems) {
    if (m->err) return NULL;
    if (layer == UINT32_MAX) snprintf(m->name, sizeof m->name, "%s", suffix);
    else snprintf(m->name, sizeof m->name, "blk.%u.%s", layer, suffix);
    const sg_tensor *t = sg_gguf_tensor(m->g, m->name);
    if (!t) return NULL;
    if (t->type != want) {
        fprintf(stderr, "model: gguf tensor %s has type %d, expected %d\n", m->name,
                (int)t->type, (int)want);
        m->err = "model: gguf tensor has an unexpected dtype";
        return NULL;
    }
    if (elems_of(t) != elems) {
        fprintf(stderr, "model: gguf tensor %s has %llu elements, expected %llu\n", m->name,
                (unsigned long long)elems_of(t), (unsigned long long)elems);
        m->err = "model: gguf tensor has an unexpected element count";
        return NULL;
    }
    return t->data;
}

void sg_model_free(sg_model *m) {
    if (!m) return;
    free(m->layers);
    memset(m, 0, sizeof *m);
}

sg_err sg_model_from_gguf(const sg_gguf *g, sg_model *m) {
    if (!m) return (sg_err){"model: invalid arguments"};
    memset(m, 0, sizeof *m);
    if (!g) return (sg_err){"model: invalid arguments"};
    const char *arch = NULL;
    if (!sg_gguf_get_str(g, "general.architecture", &arch))
        return (sg_err){"model: gguf missing general.architecture"};
    bool dense = strcmp(arch, "qwen3") == 0;
    if (!dense && strcmp(arch, "qwen35") != 0 && strcmp(arch, "qwen3_5") != 0)
        return (sg_err){"model: unrecognized gguf architecture (expected qwen35, qwen3_5 or qwen3)"};

    sg_cfg c = {0};
    c.attn_output_gate = !dense;
    char key[160];
#define KEY(suffix) (snprintf(key, sizeof key, "%s.%s", arch, suffix), key)
    if (!sg_gguf_get_u32(g, KEY("block_count"), &c.n_layers) ||
        !sg_gguf_get_u32(g, KEY("attention.head_count"), &c.n_heads) ||
        !sg_gguf_get_u32(g, KEY("attention.head_count_kv"), &c.n_kv_heads) ||
        !sg_gguf_get_u32(g, KEY("attention.key_length"), &c.head_dim) ||
        !sg_gguf_get_u32(g, KEY("embedding_length"), &c.hidden) ||
        !sg_gguf_get_u32(g, KEY("feed_forward_length"), &c.ffn_hidden) ||
        !sg_gguf_get_f32(g, KEY("rope.freq_base"), &c.rope_theta) ||
        !sg_gguf_get_f32(g, KEY("attention.layer_norm_rms_epsilon"), &c.rms_eps))
        return (sg_err){"model: gguf missing a required <arch>.* config key"};
    uint32_t vlen = 0;
    if (sg_gguf_get_u32(g, KEY("attention.value_length"), &vlen) && vlen != c.head_dim)
        return (sg_err){"model: gguf value_length differs from key_length"};
    if (dense) {
        c.rope_dim = c.head_dim;
        (void)sg_gguf_get_u32(g, KEY("rope.dimension_count"), &c.rope_dim);
        c.full_attn_interval = 1;
    } else if (!sg_gguf_get_u32(g, KEY("rope.dimension_count"), &c.rope_dim) ||
               !sg_gguf_get_u32(g, KEY("full_attention_interval"), &c.full_attn_interval)) {
        return (sg_err){"model: gguf missing rope.dimension_count or full_attention_interval"};
    }
    uint32_t inner = 0;
    (void)sg_gguf_get_u32(g, KEY("ssm.group_count"), &c.n_k_heads);
    (void)sg_gguf_get_u32(g, KEY("ssm.state_size"), &c.head_k_dim);
    (void)sg_gguf_get_u32(g, KEY("ssm.time_step_rank"), &c.n_v_heads);
    (void)sg_gguf_get_u32(g, KEY("ssm.inner_size"), &inner);
    (void)sg_gguf_get_u32(g, KEY("ssm.conv_kernel"), &c.conv_kernel);
#undef KEY
    if (c.n_v_heads && inner) {
        if (inner % c.n_v_heads) return (sg_err){"model: gguf ssm.inner_size is not a multiple of ssm.time_step_rank"};
        c.head_v_dim = inner / c.n_v_heads;
    }
    sg_gguf_kv_type et;
    uint64_t nvocab = 0;
    if (!sg_gguf_get_arr(g, "tokenizer.ggml.tokens", &et, NULL, &nvocab) || et != SG_GGUF_STR)
        return (sg_err){"model: gguf missing tokenizer.ggml.tokens"};
    if (nvocab == 0 || nvocab > UINT32_MAX) return (sg_err){"model: gguf tokenizer.ggml.tokens has an implausible count"};
    c.vocab = (uint32_t)nvocab;
    if (c.n_layers == 0 || c.n_layers > 100000) return (sg_err){"model: gguf block_count is zero or implausible"};

    const sg_tensor *emb = sg_gguf_tensor(g, "token_embd.weight");
    const sg_tensor *onorm = sg_gguf_tensor(g, "output_norm.weight");
    const sg_tensor *outw = sg_gguf_tensor(g, "output.weight");
    if (!emb) return (sg_err){"model: gguf missing token_embd.weight"};
    if (!onorm) return (sg_err){"model: gguf missing output_norm.weight"};
    if (onorm->type != SG_T_F32) return (sg_err){"model: gguf output_norm.weight is not F32"};
    if (outw && outw->type != emb->type) return (sg_err){"model: gguf output.weight dtype differs from token_embd.weight"};
    c.tied_embeddings = outw == NULL;
    uint64_t H = c.hidden, V = c.vocab;
    if (elems_of(emb) != V * H || elems_of(onorm) != H || (outw && elems_of(outw) != V * H))
        return (sg_err){"model: gguf embedding or output tensor has the wrong element count"};

    uint64_t hd = c.head_dim, attn_w = (uint64_t)c.n_heads * hd, kv_w = (uint64_t)c.n_kv_heads * hd;
    uint64_t q_w = c.attn_output_gate ? 2 * attn_w : attn_w;
    uint64_t key_dim = (uint64_t)c.n_k_heads * c.head_k_dim;
    uint64_t val_dim = (uint64_t)c.n_v_heads * c.head_v_dim;
    uint64_t conv_dim = 2 * key_dim + val_dim, F = c.ffn_hidden, nv = c.n_v_heads;
    bool have_ssm = c.n_k_heads && c.n_v_heads && c.head_k_dim && c.head_v_dim && c.conv_kernel;

    sg_layer_w *ls = calloc(c.n_layers, sizeof *ls);
    if (!ls) return (sg_err){"model: out of memory"};
    mapper mp = { g, emb->type, {0}, NULL };
    sg_tensor_type W = emb->type, F32 = SG_T_F32;
    for (uint32_t i = 0; i < c.n_layers && !mp.err; i++) {
        sg_layer_w *L = &ls[i];
        L->ln1 = tensor(&mp, i, "attn_norm.weight", F32, H);
        L->ln2 = tensor(&mp, i, "post_attention_norm.weight", F32, H);
        if (!L->ln2) L->ln2 = tensor(&mp, i, "ffn_norm.weight", F32, H);
        L->gate_proj = tensor(&mp, i, "ffn_gate.weight", W, F * H);
        L->up_proj = tensor(&mp, i, "ffn_up.weight", W, F * H);
        L->down_proj = tensor(&mp, i, "ffn_down.weight", W, H * F);
        L->q_proj = tensor(&mp, i, "attn_q.weight", W, q_w * H);
        L->k_proj = tensor(&mp, i, "attn_k.weight", W, kv_w * H);
        L->v_proj = tensor(&mp, i, "attn_v.weight", W, kv_w * H);
        L->o_proj = tensor(&mp, i, "attn_output.weight", W, H * attn_w);
        L->q_norm = tensor(&mp, i, "attn_q_norm.weight", F32, hd);
        L->k_norm = tensor(&mp, i, "attn_k_norm.weight", F32, hd);
        if (!have_ssm) {
            snprintf(mp.name, sizeof mp.name, "blk.%u.ssm_a", i);
            if (sg_gguf_tensor(g, mp.name)) mp.err = "model: gguf has linear-attention layers but no <arch>.ssm.* dimensions";
        } else {
            L->ssm_in_qkv = tensor(&mp, i, "attn_qkv.weight", W, conv_dim * H);
            L->ssm_in_z = tensor(&mp, i, "attn_gate.weight", W, val_dim * H);
            L->ssm_in_b = tensor(&mp, i, "ssm_beta.weight", W, nv * H);
            L->ssm_in_a = tensor(&mp, i, "ssm_alpha.weight", W, nv * H);
            L->ssm_a = tensor(&mp, i, "ssm_a", F32, nv);
            L->ssm_dt_bias = tensor(&mp, i, "ssm_dt.bias", F32, nv);
            L->ssm_conv1d = tensor(&mp, i, "ssm_conv1d.weight", F32, conv_dim * c.conv_kernel);
            L->ssm_norm = tensor(&mp, i, "ssm_norm.weight", F32, c.head_v_dim);
            L->ssm_out = tensor(&mp, i, "ssm_out.weight", W, H * val_dim);
        }
        if (mp.err) break;
        if (!L->ln1 || !L->ln2 || !L->gate_proj || !L->up_proj || !L->down_proj) {
            mp.err = "model: gguf layer is missing a norm or MLP tensor";
            break;
        }
        /* Exactly one complete mixer group per layer. */
        const void *a[] = { L->q_proj, L->k_proj, L->v_proj, L->o_proj, L->q_norm, L->k_norm };
        const void *d[] = { L->ssm_in_qkv, L->ssm_in_z, L->ssm_in_b, L->ssm_in_a, L->ssm_a,
                            L->ssm_dt_bias, L->ssm_conv1d, L->ssm_norm, L->ssm_out };
        int na = 0, nd = 0;
        for (int k = 0; k < 6; k++) na += a[k] != NULL;
        for (int k = 0; k < 9; k++) nd += d[k] != NULL;
        if (!((na == 6 && nd == 0) || (na == 0 && nd == 9))) {
            fprintf(stderr, "model: layer %u has %d/6 attention and %d/9 DeltaNet tensors\n", i, na, nd);
            mp.err = "model: gguf layer has an incomplete or mixed tensor group";
        }
    }
    if (mp.err) { free(ls); return (sg_err){mp.err}; }

    m->cfg = c;
    m->tok_emb = emb->data;
    m->out_norm = onorm->data;
    m->lm_head = outw ? outw->data : emb->data;
    m->layers = ls;
    m->wtype = emb->type;
    m->ssm_a_form = SG_SSM_A_NEG_EXP;
    m->v_heads_tiled = true;
    m->ssm_a_type = SG_T_F32;
    m->ssm_norm_type = SG_T_F32;
    m->dense_type = SG_T_F32;
    m->norms_are_residual = false;
    return SG_OK;
}
