/*
 * mxfa_ggml.h -- header-only adapter from ggml GGML_OP_FLASH_ATTN_EXT and
 * GGML_OP_SET_ROWS nodes to the mxfa C ABI (include/mxfa.h).
 *
 * Include it after ggml.h in a ggml backend.  The backend's supports_op and
 * graph_compute, on a node it has already identified as
 * GGML_OP_FLASH_ATTN_EXT (the adapter never looks at node->op, so it does
 * not depend on the numeric value of any GGML_OP_*), call
 *
 *     mxfa_ggml_supports(node)                 -> 1 / 0
 *     mxfa_ggml_flash_attn_ext(node, stream)   -> MXFA_OK / negative status
 *
 * and on a GGML_OP_SET_ROWS node (the KV-cache write before attention)
 *
 *     mxfa_ggml_set_rows_supports(node)        -> 1 / 0
 *     mxfa_ggml_set_rows(node, stream)         -> MXFA_OK / negative status
 *
 * and, where a model hands its pre-attention chain over as one custom node
 * (layout below), mxfa_ggml_qk_norm_rope_supports / mxfa_ggml_qk_norm_rope.
 *
 * The node layout is the one ggml_flash_attn_ext builds (upstream ggml; the
 * reference's call sites are src/qwen3-lm.h:465-469, :789-794,
 * src/dit-graph.h:227-231, :348-352, src/qwen3-enc.h:195-199):
 *   node->src[0..3] = q, k, v, mask (mask may be NULL; src[4], the
 *   attention sinks, must be NULL -- the reference adds none);
 *   node->op_params as float[0] scale, float[1] max_bias,
 *   float[2] logit_softcap, int32[3] prec (ggml_flash_attn_ext_set_prec);
 *   node itself = the F32 output [DV, Nh, Sq, B].
 * ggml type ids and GGML_PREC_* values are used as they are: mxfa uses the
 * same numbers (they are part of the GGUF format).
 *
 * Only the fields type, ne[4], nb[4], data, src[] and op_params of struct
 * ggml_tensor are read, so the adapter also compiles against any struct of
 * that name with those fields (the unit tests use such a mock).
 */
#ifndef MXFA_GGML_H
#define MXFA_GGML_H

#include <string.h>

#include "mxfa.h"

#ifdef __cplusplus
extern "C" {
#endif

struct ggml_tensor;

/* Descriptor of one ggml tensor; a NULL tensor gives a NULL descriptor. */
static inline const mxfa_tensor *mxfa_ggml_desc(const struct ggml_tensor *t, mxfa_tensor *out) {
    int i;
    if (!t) return NULL;
    out->type = (int32_t)t->type;
    for (i = 0; i < 4; i++) {
        out->ne[i] = (int64_t)t->ne[i];
        out->nb[i] = (size_t)t->nb[i];
    }
    out->data = t->data;
    return out;
}

/* op_params of the node: float[0..2] then int32[3]. */
static inline void mxfa_ggml_params(const struct ggml_tensor *node, mxfa_params *p) {
    memcpy(&p->scale, (const char *)node->op_params + 0 * sizeof(float), sizeof(float));
    memcpy(&p->max_bias, (const char *)node->op_params + 1 * sizeof(float), sizeof(float));
    memcpy(&p->logit_softcap, (const char *)node->op_params + 2 * sizeof(float), sizeof(float));
    memcpy(&p->prec, (const char *)node->op_params + 3 * sizeof(float), sizeof(int32_t));
}

/* Fills all descriptors of a flash-attention node.  Returns 0, or
 * MXFA_ERR_UNSUPPORTED when the node carries attention sinks (src[4]). */
static inline int mxfa_ggml_unpack(const struct ggml_tensor *node, mxfa_tensor *q, mxfa_tensor *k, mxfa_tensor *v,
                                   mxfa_tensor *mask, const mxfa_tensor **mask_p, mxfa_tensor *dst,
                                   mxfa_params *p) {
    if (node->src[4] != NULL) return MXFA_ERR_UNSUPPORTED;
    mxfa_ggml_desc(node->src[0], q);
    mxfa_ggml_desc(node->src[1], k);
    mxfa_ggml_desc(node->src[2], v);
    *mask_p = mxfa_ggml_desc(node->src[3], mask);
    mxfa_ggml_desc(node, dst);
    mxfa_ggml_params(node, p);
    return 0;
}

/* supports_op for a GGML_OP_FLASH_ATTN_EXT node (descriptor checks only; the
 * data pointers are not dereferenced). */
static inline int mxfa_ggml_supports(const struct ggml_tensor *node) {
    mxfa_tensor q, k, v, m, d;
    const mxfa_tensor *mp;
    mxfa_params p;
    if (!node || !node->src[0] || !node->src[1] || !node->src[2]) return 0;
    if (mxfa_ggml_unpack(node, &q, &k, &v, &m, &mp, &d, &p) != 0) return 0;
    return mxfa_supports(&q, &k, &v, mp, &p, &d);
}

/* supports_op / graph_compute for a GGML_OP_SET_ROWS node, the KV-cache
 * write (ggml_set_rows(ctx, a, b, c) at src/qwen3-lm.h:453-454, :776-777):
 * the node is a view of the destination `a`, node->src[0] = b (F32 rows),
 * node->src[1] = c (I64 / I32 row ids). */
static inline int mxfa_ggml_set_rows_supports(const struct ggml_tensor *node) {
    mxfa_tensor d, s, r;
    if (!node || !node->src[0] || !node->src[1]) return 0;
    return mxfa_set_rows_supports(mxfa_ggml_desc(node, &d), mxfa_ggml_desc(node->src[0], &s),
                                  mxfa_ggml_desc(node->src[1], &r));
}

static inline int mxfa_ggml_set_rows(const struct ggml_tensor *node, void *hip_stream) {
    mxfa_tensor d, s, r;
    if (!node || !node->src[0] || !node->src[1]) return MXFA_ERR_INVALID;
    mxfa_ggml_desc(node, &d);
    return mxfa_set_rows(&d, mxfa_ggml_desc(node->src[0], &s), mxfa_ggml_desc(node->src[1], &r), hip_stream);
}

/* graph_compute for a GGML_OP_FLASH_ATTN_EXT node on `hip_stream`. */
static inline int mxfa_ggml_flash_attn_ext(const struct ggml_tensor *node, void *hip_stream) {
    mxfa_tensor q, k, v, m, d;
    const mxfa_tensor *mp;
    mxfa_params p;
    int rc;
    if (!node || !node->src[0] || !node->src[1] || !node->src[2]) return MXFA_ERR_INVALID;
    rc = mxfa_ggml_unpack(node, &q, &k, &v, &m, &mp, &d, &p);
    if (rc != 0) return rc;
    return mxfa_flash_attn_ext(&q, &k, &v, mp, &p, &d, hip_stream);
}

/* The pre-attention step (src/qwen3-lm.h:418-454: rms_norm, mul, rope_ext,
 * permute, cont, clamp, and the two set_rows) as one custom node, e.g.
 * ggml_custom_4d with these sources, in this order:
 *   node    = Q out [128, Nh, S, B], F16 or BF16 (attention takes its
 *             permuted view, as it took the rope output's);
 *   src[0..2] = q, k, v: the F32 projections [128, Nh|Nkv, S, B];
 *   src[3], src[4] = q_norm, k_norm: F32 [128];
 *   src[5] = positions: I32 [S] or [S, B];
 *   src[6], src[7] = the K and V cache views written, [128, M, Nkv, B];
 *   src[8] = row ids I64/I32 [S, R], or NULL (row s).
 * eps, rope base and the V clamp are not op_params of a custom node; the
 * caller passes them (from its user data). */
static inline int mxfa_ggml_unpack_norm_rope(const struct ggml_tensor *node, mxfa_tensor *t /* [10] */,
                                             const mxfa_tensor **rows) {
    int i;
    if (!node) return MXFA_ERR_INVALID;
    for (i = 0; i < 8; i++)
        if (!node->src[i]) return MXFA_ERR_INVALID;
    for (i = 0; i < 8; i++) mxfa_ggml_desc(node->src[i], &t[i]);
    mxfa_ggml_desc(node, &t[8]);
    *rows = mxfa_ggml_desc(node->src[8], &t[9]);
    return 0;
}

static inline int mxfa_ggml_qk_norm_rope_supports(const struct ggml_tensor *node, const mxfa_norm_rope_params *p) {
    mxfa_tensor t[10];
    const mxfa_tensor *rows;
    if (mxfa_ggml_unpack_norm_rope(node, t, &rows) != 0) return 0;
    return mxfa_qk_norm_rope_supports(&t[0], &t[1], &t[2], &t[3], &t[4], &t[5], p, &t[8], &t[6], &t[7], rows);
}

static inline int mxfa_ggml_qk_norm_rope(const struct ggml_tensor *node, const mxfa_norm_rope_params *p,
                                         void *hip_stream) {
    mxfa_tensor t[10];
    const mxfa_tensor *rows;
    const int rc = mxfa_ggml_unpack_norm_rope(node, t, &rows);
    if (rc != 0) return rc;
    return mxfa_qk_norm_rope(&t[0], &t[1], &t[2], &t[3], &t[4], &t[5], p, &t[8], &t[6], &t[7], rows, hip_stream);
}

#ifdef __cplusplus
}
#endif

#endif /* MXFA_GGML_H */
