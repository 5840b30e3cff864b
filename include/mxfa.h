/*
 * mxfa.h -- MI355X (gfx950) flash-attention engine, C ABI.
 *
 * The engine implements ggml's GGML_OP_FLASH_ATTN_EXT so that acestep.cpp's
 * attention graphs run unchanged on top of it.  The reference builds every
 * attention node as
 *
 *     attn = ggml_flash_attn_ext(ctx, q, k, v, mask, scale, max_bias, softcap);
 *     ggml_flash_attn_ext_set_prec(attn, GGML_PREC_F32);
 *
 * at src/qwen3-lm.h:465-469 (LM prefill / single decode), :789-794 (batched
 * CFG decode), src/dit-graph.h:227-231 (DiT self-attention), :348-352 (DiT
 * cross-attention) and src/qwen3-enc.h:195-199 (text / lyric / timbre
 * encoders).  The node is executed by whatever ggml backend owns it
 * (src/backend.h:90-145, src/static-graph.h:54-58).  A ggml backend's
 * graph_compute maps such a node onto mxfa_flash_attn_ext() below (see
 * include/mxfa_ggml.h for the header-only adapter from struct ggml_tensor),
 * and its supports_op maps onto mxfa_supports().
 *
 * All tensors are owned by the caller and live in device memory (the ggml
 * backend buffer).  Descriptors carry ggml's own fields: type id, ne[4]
 * (element counts, ne[0] innermost) and nb[4] (byte strides).
 *
 *   q    : F32            [DK, Sq,  Nh,  B ]  any strides, nb[0] = 4
 *   k    : F16|BF16|Q8_0  [DK, Skv, Nkv, Bk]  rows contiguous (nb[0] = type size)
 *   v    : same type as k [DV, Skv, Nkv, Bk]
 *   mask : F16 or NULL    [>=Skv, >=Sq, Nm2, Nm3], additive, broadcast over
 *                         heads (iq2 % Nm2) and batches (iq3 % Nm3);
 *                         -inf entries exclude the key entirely
 *   dst  : F32 contiguous [DV, Nh, Sq, B]   (ggml's permuted FA output)
 *
 * with GQA head map kv_head = q_head / (Nh / Nkv) and batch broadcast
 * kv_batch = b / (B / Bk).  Semantics are those of ggml's CPU kernel
 * (softmax(scale * K.Q [+softcap] + slope * mask) . V, a row with no
 * unmasked key gives 0); accumulation is fp32 throughout.
 */
#ifndef MXFA_H
#define MXFA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (enum ggml_type values; they are stable in the GGUF format). */
#define MXFA_TYPE_F32  0
#define MXFA_TYPE_F16  1
#define MXFA_TYPE_Q8_0 8
#define MXFA_TYPE_BF16 30
#define MXFA_TYPE_I32  26   /* set_rows row ids */
#define MXFA_TYPE_I64  27

/* ggml_prec values (GGML_PREC_DEFAULT / GGML_PREC_F32).  The engine always
 * accumulates in fp32, so both are accepted and treated alike. */
#define MXFA_PREC_DEFAULT 0
#define MXFA_PREC_F32     10

/* Status codes: 0 = success, negative = failure; never exit()/abort(). */
#define MXFA_OK               0
#define MXFA_ERR_INVALID     -1   /* malformed descriptor / NULL pointer      */
#define MXFA_ERR_UNSUPPORTED -2   /* valid op, shape/type not handled here    */
#define MXFA_ERR_HIP         -3   /* HIP runtime error (launch, device)       */
#define MXFA_ERR_NOMEM       -4   /* workspace allocation failed              */

/* One tensor, as ggml describes it (struct ggml_tensor: type, ne, nb, data). */
typedef struct mxfa_tensor {
    int32_t type;
    int64_t ne[4];
    size_t  nb[4];
    void   *data;
} mxfa_tensor;

/* The op parameters of GGML_OP_FLASH_ATTN_EXT: op_params float[0..2] =
 * scale, max_bias, logit_softcap and int32[3] = prec. */
typedef struct mxfa_params {
    float   scale;
    float   max_bias;
    float   logit_softcap;
    int32_t prec;
} mxfa_params;

/* supports_op for GGML_OP_FLASH_ATTN_EXT: returns 1 when
 * mxfa_flash_attn_ext() handles this combination, 0 otherwise (the ggml
 * scheduler then places the node on another backend, as
 * src/static-graph.h:12-19 and :31-52 expect).  Reads descriptors only;
 * no device access.  `dst` may be NULL (then its layout is not checked). */
int mxfa_supports(const mxfa_tensor *q, const mxfa_tensor *k, const mxfa_tensor *v,
                  const mxfa_tensor *mask, const mxfa_params *params, const mxfa_tensor *dst);

/* Execute GGML_OP_FLASH_ATTN_EXT on the current HIP device, ordered on
 * `hip_stream` (a hipStream_t; NULL = the default stream).  Asynchronous:
 * returns after the launches are queued.  The engine owns only a device
 * workspace per (device, stream) for split-KV partials, split tickets and
 * mask tile classes; it is grown on demand and kept until mxfa_release().
 * A grow retires the outgrown buffers without freeing them (work already
 * queued, and HIP graphs captured earlier, keep valid addresses), so it
 * never synchronises.  Calls on different streams use different workspaces
 * and may overlap in time; calls on one stream are ordered by it.  Returns
 * MXFA_OK or a negative status; on failure nothing was launched. */
int mxfa_flash_attn_ext(const mxfa_tensor *q, const mxfa_tensor *k, const mxfa_tensor *v,
                        const mxfa_tensor *mask, const mxfa_params *params, mxfa_tensor *dst,
                        void *hip_stream);

/* Structured masks: GGML_OP_FLASH_ATTN_EXT with the mask given as metadata
 * instead of an F16 tensor.  The reference builds every one of its masks on
 * the host from a few integers and uploads O(Sq*Skv) F16 values per call:
 * causal at src/qwen3-lm.h:597-610 and src/qwen3-enc.h:429-437, per-sequence
 * lengths at src/qwen3-lm.h:872-883 and src/dit-sampler.h:296-309, and the
 * sliding window at src/dit-sampler.h:262-289 and src/cond-enc.h:307-341.
 * Key j is live for query row i (0 <= i < Sq) of batch b iff every flag set
 * holds:
 *   MXFA_MASK_LENGTHS  j < lengths[b % n_lengths]
 *   MXFA_MASK_CAUSAL   j <= pos0 + i
 *   MXFA_MASK_WINDOW   |pos0 + i - j| <= window
 * mxfa_flash_attn_ext_masked(q, k, v, spec, ...) computes exactly what
 * mxfa_flash_attn_ext(q, k, v, mask, ...) computes for the F16 mask
 * [Skv, Sq, 1, B] holding 0 at live keys and -inf elsewhere (flags == 0:
 * no mask).  Nothing is read from device memory for the mask: no mask
 * upload, no mask reads, no mask-classifier pass, and the split-KV decode
 * sizes its splits from the live lengths.  `lengths` is host memory read
 * during the call (n_lengths is 1 or B, at most 64; values >= 0); pos0 >= 0,
 * window >= 0, pos0 + Sq + window < 2^30.
 *
 * MXFA_MASK_DEVICE: `lengths` (and `dev_pos0`, when not NULL, in place of
 * pos0) point to device memory (int32) that the kernels read when they run,
 * not at the call: a launch captured into a HIP graph then follows the
 * values the host writes there between replays, as the reference's static
 * decode graph does with its kv_len / position inputs (src/qwen3-lm.h:864-884).
 * The decode split sizes then come from Skv, not from the live lengths.  The
 * kernels clamp what they read: a negative length to 0, pos0 to [0, 2^30). */
#define MXFA_MASK_CAUSAL  1
#define MXFA_MASK_WINDOW  2
#define MXFA_MASK_LENGTHS 4
#define MXFA_MASK_DEVICE  8

typedef struct mxfa_mask_spec {
    int32_t        flags;      /* MXFA_MASK_* bits */
    int32_t        window;     /* MXFA_MASK_WINDOW */
    int64_t        pos0;       /* absolute position of query row 0 (causal, window) */
    int32_t        n_lengths;  /* MXFA_MASK_LENGTHS: entries of lengths[] */
    const int32_t *lengths;    /* MXFA_MASK_LENGTHS: live key count per batch (device memory with
                                  MXFA_MASK_DEVICE) */
    const int32_t *dev_pos0;   /* MXFA_MASK_DEVICE: device int32 read for pos0, or NULL (use pos0) */
} mxfa_mask_spec;

int mxfa_supports_masked(const mxfa_tensor *q, const mxfa_tensor *k, const mxfa_tensor *v,
                         const mxfa_mask_spec *mask, const mxfa_params *params, const mxfa_tensor *dst);
int mxfa_flash_attn_ext_masked(const mxfa_tensor *q, const mxfa_tensor *k, const mxfa_tensor *v,
                               const mxfa_mask_spec *mask, const mxfa_params *params, mxfa_tensor *dst,
                               void *hip_stream);

/* GGML_OP_SET_ROWS with an F32 source: the KV-cache write the reference
 * issues right before each attention node, ggml_set_rows(ctx, cache, rows_f32,
 * kv_rows) at src/qwen3-lm.h:453-454 ([D, S, Nkv] rows into the
 * [D, max_seq, Nkv] F16 cache, row ids [S] broadcast over Nkv) and :776-777
 * ([D, 1, Nkv, N] rows into N cache sets, row ids [1, 1, N]).  A ggml
 * backend maps the node as (dst = node, src = node->src[0],
 * rows = node->src[1]):
 *
 *   src  : F32             [D, n, ne2, ne3], nb[0] = 4
 *   rows : I64 | I32       [n, R1, R2, 1] with ne2 % R1 == 0, ne3 % R2 == 0
 *   dst  : F32|F16|BF16|Q8_0 [D, M, ne2, ne3] (the cache view)
 *
 *   dst[:, rows[i, i2 % R1, i3 % R2], i2, i3] = convert(src[:, i, i2, i3])
 *
 * convert = ggml's from_float of dst's type: F16 / BF16 round to nearest
 * even, Q8_0 per 32 values d = amax/127 (stored F16), q = round-half-even(
 * x * 127/amax).  Row ids live in device memory and are not read on the
 * host: a row whose id is outside [0, M) is skipped (ggml's CPU backend
 * aborts on it).  Rows that name the same destination row race (ggml leaves
 * that order unspecified too).  Needs D % 4 == 0 (D % 32 for Q8_0), src data
 * and strides 16-byte aligned, dst rows contiguous.  Launches one kernel on
 * `hip_stream`, allocates nothing, returns MXFA_OK or a negative status
 * (nothing launched on failure).  An empty source (n, ne2 or ne3 = 0) is a
 * no-op. */
int mxfa_set_rows_supports(const mxfa_tensor *dst, const mxfa_tensor *src, const mxfa_tensor *rows);
int mxfa_set_rows(mxfa_tensor *dst, const mxfa_tensor *src, const mxfa_tensor *rows, void *hip_stream);

/* Pre-attention fusion: the work between a layer's QKV projections and its
 * attention node, in one pass.  The reference runs it as separate ggml ops
 * (src/qwen3-lm.h:418-454, src/dit-graph.h:177-225):
 *
 *   q = rope_neox(rms_norm(q, eps) * q_norm, positions)
 *   k = rope_neox(rms_norm(k, eps) * k_norm, positions)
 *   v = clamp(v, -65504, 65504)              (only with clamp_v, :438-441)
 *   set_rows(cache_k, cont(permute(k)), kv_rows); likewise v
 *
 * (rope: n_dims = 128, freq_base, freq_scale 1, no YaRN / ext factor; the
 * arithmetic of ggml's CPU ops, see qk_norm_rope.hip) and writes Q already
 * in K's 16-bit type, so that attention (mxfa_flash_attn_ext, Q of K's
 * type) reads half the bytes and converts nothing:
 *
 *   q, k, v   : F32 [128, Nh | Nkv, S, B], nb[0] = 4 (views allowed)
 *   q_norm, k_norm : F32 [128] contiguous
 *   positions : I32 [S] (shared by the batches) or [S, B], contiguous
 *   q_out     : F16 | BF16 [128, Nh, S, B] contiguous (attention takes the
 *               permuted view [128, S, Nh, B], as the reference does)
 *   k_out, v_out : the same type, [128, M, Nkv, B] with nb[0] = 2 (a cache
 *               view); row rows[s, b % R] receives token s of batch b, or
 *               row s when rows is NULL (then M >= S)
 *   rows      : I64 | I32 [S, R] with B % R == 0, or NULL
 *
 * positions == NULL selects DiT cross-attention's chain
 * (src/dit-graph.h:317-346): QK-norm without RoPE (":333 no RoPE for
 * cross-attention") and the K/V casts, with K/V of their own token count
 * Skv (enc_S): k, v are [128, Nkv, Skv, B], k_out / v_out [128, M >= Skv,
 * Nkv, B] (or rows [Skv, R]), while q / q_out keep S tokens.
 *
 * Row ids outside [0, M) are skipped (ggml asserts).  Launches one kernel
 * on `hip_stream`, allocates nothing; MXFA_OK or a negative status. */
typedef struct mxfa_norm_rope_params {
    float   eps;        /* rms_norm epsilon */
    float   freq_base;  /* rope theta */
    int32_t clamp_v;    /* clamp V to +-65504 before the cast */
} mxfa_norm_rope_params;

/* 1 when mxfa_qk_norm_rope would accept these descriptors (checks only,
 * nothing is dereferenced or launched), else 0 with the reason in
 * mxfa_last_error(): the supports_op of the fused step, so that a caller
 * keeps the reference's op chain for what it does not take. */
int mxfa_qk_norm_rope_supports(const mxfa_tensor *q, const mxfa_tensor *k, const mxfa_tensor *v,
                               const mxfa_tensor *q_norm, const mxfa_tensor *k_norm, const mxfa_tensor *positions,
                               const mxfa_norm_rope_params *params, const mxfa_tensor *q_out,
                               const mxfa_tensor *k_out, const mxfa_tensor *v_out, const mxfa_tensor *rows);

int mxfa_qk_norm_rope(const mxfa_tensor *q, const mxfa_tensor *k, const mxfa_tensor *v,
                      const mxfa_tensor *q_norm, const mxfa_tensor *k_norm, const mxfa_tensor *positions,
                      const mxfa_norm_rope_params *params, mxfa_tensor *q_out, mxfa_tensor *k_out,
                      mxfa_tensor *v_out, const mxfa_tensor *rows, void *hip_stream);

/* HIP graph capture / replay.  The reference replays its static decode
 * graph (src/static-graph.h, src/graph-arena.h, src/qwen3-lm.h:36-58): the
 * node arguments stay at fixed addresses and only their contents change
 * between replays (kv_rows, masks, positions).  Every mxfa entry point is
 * capture-safe -- kernels only, no memset, no host synchronisation, split
 * tickets reset by the kernels themselves -- except when the per-device
 * workspace has to grow: that call fails with MXFA_ERR_UNSUPPORTED while
 * `hip_stream` is being captured.  mxfa_reserve() grows the workspace of
 * `hip_stream` on the current device for the given FA call without
 * launching anything (beyond the one-time zero fill of a new ticket
 * buffer); so does any eager call of the same shapes on that stream.  A
 * graph keeps the workspace addresses of the stream it was captured on:
 * a later grow of that workspace retires the old buffers but keeps them
 * allocated until mxfa_release(), so the graph stays valid.  Replays must
 * not overlap in time with other mxfa calls on the capture stream.  A
 * structured mask's host-side values (pos0, window, lengths) are captured
 * with the launch: for lengths or positions that change between replays,
 * set MXFA_MASK_DEVICE (they are then read from device memory at run time)
 * or use the dense mask.  (No counterpart in ggml: a backend calls
 * mxfa_reserve from its graph set-up.) */
int mxfa_reserve(const mxfa_tensor *q, const mxfa_tensor *k, const mxfa_tensor *v, const mxfa_tensor *mask,
                 const mxfa_params *params, void *hip_stream);

/* One mask classification per graph.  The reference builds each mask once
 * per graph as an input tensor and hands the same tensor to every layer's
 * attention node: the LM's causal mask (src/qwen3-lm.h:515-517, used at
 * :541-543 by all 36 layers of the 4B model), the DiT's sliding-window and
 * cross-attention masks (src/dit-graph.h:522-528, used at :574-576).  The
 * engine's prefill path first sorts every (128-query x 64-key) tile of a
 * dense mask into all -inf / all zero / mixed (one classifier launch);
 * after mxfa_graph_begin(stream), a mask that several FA nodes on that
 * stream share -- the same data pointer, ne, nb, and the same Sq and Skv --
 * is classified once, at its first node, and the later nodes reuse the
 * classes, until mxfa_graph_end(stream).  A ggml backend brackets each
 * graph_compute with the two calls (no counterpart in ggml; like
 * mxfa_reserve they are backend-level): between them the contents of a
 * mask that FA nodes read must not change, and after mxfa_graph_end the
 * stream classifies per call again.  A second mxfa_graph_begin without an
 * end starts a new graph (earlier classes are forgotten).  Under HIP
 * graph capture the classifier launch is recorded at the mask's first node,
 * so every replay reclassifies the mask's current contents before the
 * nodes that read the classes.  The classes of one graph live in a
 * per-(device, stream) arena grown on demand (64 KiB holds the classes of
 * hundreds of masks of the reference's shapes); a graph that would grow it
 * fails with MXFA_ERR_UNSUPPORTED while being captured (compute it eagerly
 * once first).  Host-side only: launches nothing, allocates nothing.
 * mxfa_flash_attn_ext_noalloc always classifies per call. */
int mxfa_graph_begin(void *hip_stream);
int mxfa_graph_end(void *hip_stream);

/* Allocation-free variant of mxfa_flash_attn_ext (no counterpart in the
 * reference or in ggml).  For callers that cannot allocate device memory:
 * code under HIP graph capture, tight serving loops, hosts that forbid
 * hipMalloc.  Same arguments, semantics and kernels as mxfa_flash_attn_ext,
 * but the split-KV partials, split tickets and mask tile classes live in a
 * fixed array of 8 MiB per GPU (65536 tickets plus 8 MiB - 256 KiB of
 * partials/classes), held until the process ends; no hipMalloc, hipFree or
 * allocating library call is made.  A call that needs more (decode with
 * many query rows per KV head at long context; prefill masks with very
 * many planes) fails with MXFA_ERR_UNSUPPORTED and launches nothing.  The
 * first call on a device looks up the array and zero-fills its tickets
 * (one kernel on `hip_stream`); it must not be captured.  Every call on a
 * device shares that device's array, so calls that overlap in time on one
 * GPU (on different streams, or a replayed graph next to an eager call)
 * race; calls ordered on one stream do not. */
int mxfa_flash_attn_ext_noalloc(const mxfa_tensor *q, const mxfa_tensor *k, const mxfa_tensor *v,
                                const mxfa_tensor *mask, const mxfa_params *params, mxfa_tensor *dst,
                                void *hip_stream);

/* Free the workspaces of every device and stream, retired buffers
 * included (synchronises each device first).  Graphs captured before the
 * call must not be replayed after it. */
void mxfa_release(void);

/* Diagnostics (no counterpart in ggml): bytes of the live workspaces
 * (partials, classes and tickets of every device and stream) and the number
 * of outgrown buffers kept for earlier captures.  MXFA_OK or
 * MXFA_ERR_INVALID. */
int mxfa_workspace_info(int64_t *live_bytes, int64_t *retired_buffers);

/* Human-readable text for a status code; last error detail for MXFA_ERR_HIP
 * and MXFA_ERR_UNSUPPORTED (thread-local). */
const char *mxfa_status_string(int status);
const char *mxfa_last_error(void);

/* Library version: major*10000 + minor*100 + patch. */
int mxfa_version(void);

/* Per-kernel timing (a profiling aid; no counterpart in ggml).  With
 * mxfa_timing_enable(n), n >= 1, every kernel the engine launches is run n
 * times back to back (each launch rewrites its outputs from its inputs, so
 * the result is unchanged) between two HIP events recorded on its launch
 * stream, counted as n launches: with n large the average is the kernel's
 * own duration, with no event overhead per launch.  mxfa_timing_read()
 * waits for the recorded events, returns the summed duration (ms) and
 * launch count of one kernel family ("fa_prefill", "mask_classify",
 * "fa_decode", "set_rows", "qk_norm_rope") since the last reset, and
 * mxfa_timing_reset() clears all counters.  n = 0 (the default) turns
 * timing off. */
void mxfa_timing_enable(int on);
int  mxfa_timing_read(const char *kernel, double *total_ms, int64_t *launches);
void mxfa_timing_reset(void);

#ifdef __cplusplus
}
#endif

#endif /* MXFA_H */
