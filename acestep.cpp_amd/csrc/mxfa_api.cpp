// mxfa_api.cpp -- host side of the C ABI declared in include/mxfa.h.
//
// Validates ggml-style descriptors (the same contract ggml_flash_attn_ext
// asserts), picks a kernel and launches it on the caller's stream:
//   * split-KV decode kernel (fa_decode.hip) when few query rows share a
//     KV head: decode (Sq = 1) and short prompts, and every Q8_0 K/V call;
//   * MFMA prefill kernel (fa_mfma.hip) for long query runs (prefill, DiT),
//     preceded by the mask tile classifier when a mask is given;
// and GGML_OP_SET_ROWS, the KV-cache write before each attention node
// (set_rows.hip).
// The only memory the engine owns is per (device, stream) and grow-only: a
// workspace (split partials, mask tile classes) and the split tickets.  A
// grow retires the old buffers instead of freeing them -- kernels still
// queued, or a HIP graph captured earlier, may hold their addresses -- and
// mxfa_release() frees everything.  Calls on different streams use
// different workspaces and may overlap in time.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "mxfa.h"
#include "mxfa_internal.h"

namespace {

using namespace mxfa;

thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

// One dense mask's tile classes within a graph (mxfa_graph_begin): the
// classes depend only on the mask's bytes inside [0, Skv) x [0, Sq) of each
// plane, so (data, ne, nb, Sq, Skv) identifies them while the mask's
// contents stay fixed, as they do during one ggml graph computation.
struct ClassEntry {
    const void *data = nullptr;
    int64_t ne[4] = {0, 0, 0, 0};
    size_t nb[4] = {0, 0, 0, 0};
    int64_t Sq = 0, Skv = 0;
    size_t bytes = 0;   // the block's layout (classes, with or without liveness words)
    uint8_t *cls = nullptr;
};

struct Workspace {
    int device = 0;
    hipStream_t stream = nullptr;
    void *ptr = nullptr;
    size_t size = 0;
    int *tickets = nullptr;   // zero between calls
    int64_t n_tickets = 0;
    std::vector<void *> retired;   // outgrown buffers, freed by mxfa_release()
    // mask tile classes of the current graph: epoch 0 = no graph begun on
    // this stream (every call classifies its own mask into `ptr`)
    uint64_t epoch = 0;
    uint8_t *arena = nullptr;
    size_t arena_size = 0, arena_used = 0;
    std::vector<ClassEntry> entries;
};
std::mutex g_ws_mu;
std::vector<Workspace> g_ws;  // one per (device, stream) that has needed one

// Query-run length from which the MFMA prefill kernel is used.
constexpr int64_t kPrefillMinSq = 64;
// Build option MXFA_WIDE=0 keeps every prefill call on the 32-query kernel
// (for same-box comparisons of the two).
#ifndef MXFA_WIDE
#define MXFA_WIDE 1
#endif
constexpr bool kPfWide = MXFA_WIDE != 0;
// Masked calls take it up to this many key tiles: a causal mask over long
// rows would make 192-query jobs the critical path (the host cannot tell a
// dense causal mask from a window or padding mask, and a structured mask
// follows the same rule as its dense form).
constexpr int64_t kPfWideMaskedMaxKt = 4;
// Workgroups the decode kernel aims for before it splits the KV range.
// (build option for A/B runs; 512 = two workgroups per CU measured best:
// 256, 384, 640, 768, 1024 and 2048 were slower on C3 / C5)
#ifndef MXFA_SPLIT_TARGET
#define MXFA_SPLIT_TARGET 512
#endif
constexpr int64_t kSplitTargetWgs = MXFA_SPLIT_TARGET;
constexpr int kSplitKeyQuantum = 128;  // register kernel: 4 waves x 32 keys
constexpr int kSplitKeyQuantumLds = 64;  // LDS kernel: 4 waves x 16 keys
constexpr int64_t kMaxDecodeSplits = 64;   // merge capacity of the decode kernel
constexpr int kMaxLiveListTiles = 64;      // (batch, row tile) streams a live-split grid may list
constexpr int64_t kDecCus = 256;           // MI355X compute units
#ifndef MXFA_DEC_PAIR_NUM
#define MXFA_DEC_PAIR_NUM 10
#endif
constexpr int64_t kDecPairNum = MXFA_DEC_PAIR_NUM;   // even split's share of a pair, in eighths of a chunk x 2 / 2

bool is_aligned(const void *p, size_t a) { return ((uintptr_t)p % a) == 0; }

size_t elem_row_bytes(int type, int64_t ne0) {
    switch (type) {
        case MXFA_TYPE_F32: return 4 * (size_t)ne0;
        case MXFA_TYPE_F16:
        case MXFA_TYPE_BF16: return 2 * (size_t)ne0;
        case MXFA_TYPE_Q8_0: return (size_t)(ne0 / 32) * 34;
        default: return 0;
    }
}

size_t type_block_bytes(int type) {
    switch (type) {
        case MXFA_TYPE_F32: return 4;
        case MXFA_TYPE_F16:
        case MXFA_TYPE_BF16: return 2;
        case MXFA_TYPE_Q8_0: return 34;
        default: return 0;
    }
}

// Validation of a GGML_OP_SET_ROWS node (the shape asserts of ggml_set_rows
// plus this kernel's layout needs).  Fills `a` when `a` is given.
int check_set_rows(const mxfa_tensor *dst, const mxfa_tensor *src, const mxfa_tensor *rows, SetRowsArgs *a) {
    if (!dst || !src || !rows) return fail(MXFA_ERR_INVALID, "dst, src and rows are required");
    for (const mxfa_tensor *t : {dst, src, rows})
        for (int i = 0; i < 4; i++)
            if (t->ne[i] < 0) return fail(MXFA_ERR_INVALID, "ne[%d] = %lld is negative", i, (long long)t->ne[i]);
    if (src->type != MXFA_TYPE_F32) return fail(MXFA_ERR_UNSUPPORTED, "set_rows source must be F32 (type %d)", src->type);
    if (rows->type != MXFA_TYPE_I64 && rows->type != MXFA_TYPE_I32)
        return fail(MXFA_ERR_INVALID, "row ids must be I64 or I32 (type %d)", rows->type);
    if (dst->ne[0] != src->ne[0] || dst->ne[2] != src->ne[2] || dst->ne[3] != src->ne[3])
        return fail(MXFA_ERR_INVALID, "dst and src differ in ne[0], ne[2] or ne[3]");
    if (src->ne[1] != rows->ne[0]) return fail(MXFA_ERR_INVALID, "src->ne[1] != rows->ne[0]");
    if (rows->ne[1] < 1 || rows->ne[2] < 1 || rows->ne[3] != 1)
        return fail(MXFA_ERR_INVALID, "rows must be [n, R1 >= 1, R2 >= 1, 1]");
    if (src->ne[2] % rows->ne[1] || src->ne[3] % rows->ne[2])
        return fail(MXFA_ERR_INVALID, "row ids do not broadcast over src->ne[2] / ne[3]");
    const int dt = dst->type;
    if (dt != MXFA_TYPE_F32 && dt != MXFA_TYPE_F16 && dt != MXFA_TYPE_BF16 && dt != MXFA_TYPE_Q8_0)
        return fail(MXFA_ERR_UNSUPPORTED, "set_rows destination type %d (F32, F16, BF16, Q8_0)", dt);
    const int64_t D = src->ne[0];
    if (dt == MXFA_TYPE_Q8_0 ? D % 32 != 0 : D % 4 != 0)
        return fail(MXFA_ERR_UNSUPPORTED, "row length %lld (needs a multiple of %d)", (long long)D,
                    dt == MXFA_TYPE_Q8_0 ? 32 : 4);
    if (src->nb[0] != 4 || dst->nb[0] != type_block_bytes(dt))
        return fail(MXFA_ERR_UNSUPPORTED, "src/dst rows must be contiguous");
    if (rows->nb[0] != (rows->type == MXFA_TYPE_I64 ? 8u : 4u))
        return fail(MXFA_ERR_INVALID, "row ids must be contiguous along ne[0]");
    const int64_t n_rows = src->ne[1] * src->ne[2] * src->ne[3];
    if (n_rows == 0 || D == 0) {
        if (a) *a = SetRowsArgs{};
        return MXFA_OK;   // empty source: nothing to write
    }
    if (!dst->data || !src->data || !rows->data) return fail(MXFA_ERR_INVALID, "NULL data pointer");
    if (!is_aligned(src->data, 16) || src->nb[1] % 16 || src->nb[2] % 16 || src->nb[3] % 16)
        return fail(MXFA_ERR_UNSUPPORTED, "src data/strides must be 16-byte aligned");
    const size_t da = dt == MXFA_TYPE_F32 ? 16 : dt == MXFA_TYPE_Q8_0 ? 2 : 8;
    if (!is_aligned(dst->data, da) || dst->nb[1] % da || dst->nb[2] % da || dst->nb[3] % da)
        return fail(MXFA_ERR_UNSUPPORTED, "dst data/strides must be %zu-byte aligned", da);
    const size_t ia = rows->nb[0];
    if (!is_aligned(rows->data, ia) || rows->nb[1] % ia || rows->nb[2] % ia)
        return fail(MXFA_ERR_INVALID, "row ids misaligned");
    if (n_rows * (D / 4) >= ((int64_t)1 << 31))
        return fail(MXFA_ERR_UNSUPPORTED, "set_rows source too large for one launch");
    if (a) {
        SetRowsArgs &r = *a;
        r = SetRowsArgs{};
        r.src = (const char *)src->data;
        r.rows = (const char *)rows->data;
        r.dst = (char *)dst->data;
        r.cpr = (uint32_t)(D / 4);
        r.ne01 = (uint32_t)src->ne[1];
        r.ne02 = (uint32_t)src->ne[2];
        r.n_rows = (uint32_t)n_rows;
        r.r_ne1 = (uint32_t)rows->ne[1];
        r.r_ne2 = (uint32_t)rows->ne[2];
        r.s_nb1 = (int64_t)src->nb[1];
        r.s_nb2 = (int64_t)src->nb[2];
        r.s_nb3 = (int64_t)src->nb[3];
        r.r_nb0 = (int64_t)rows->nb[0];
        r.r_nb1 = (int64_t)rows->nb[1];
        r.r_nb2 = (int64_t)rows->nb[2];
        r.d_nb1 = (int64_t)dst->nb[1];
        r.d_nb2 = (int64_t)dst->nb[2];
        r.d_nb3 = (int64_t)dst->nb[3];
        r.dst_ne1 = dst->ne[1];
        r.rows_i64 = rows->type == MXFA_TYPE_I64;
    }
    return MXFA_OK;
}

// Validation of a pre-attention fusion call; fills `a` (and *out_type).
int check_norm_rope(const mxfa_tensor *q, const mxfa_tensor *k, const mxfa_tensor *v, const mxfa_tensor *qw,
                    const mxfa_tensor *kw, const mxfa_tensor *pos, const mxfa_norm_rope_params *p,
                    const mxfa_tensor *qo, const mxfa_tensor *ko, const mxfa_tensor *vo, const mxfa_tensor *rows,
                    NormRopeArgs *a, int *out_type) {
    if (!q || !k || !v || !qw || !kw || !p || !qo || !ko || !vo)
        return fail(MXFA_ERR_INVALID, "q, k, v, norms, params and outputs are required");
    for (const mxfa_tensor *t : {q, k, v, qw, kw, pos, qo, ko, vo, rows}) {
        if (!t) continue;
        for (int i = 0; i < 4; i++)
            if (t->ne[i] <= 0) return fail(MXFA_ERR_INVALID, "ne[%d] = %lld must be positive", i, (long long)t->ne[i]);
        if (!t->data) return fail(MXFA_ERR_INVALID, "NULL data pointer");
    }
    for (const mxfa_tensor *t : {q, k, v})
        if (t->type != MXFA_TYPE_F32 || t->ne[0] != kD || t->nb[0] != 4 || !is_aligned(t->data, 16) ||
            t->nb[1] % 16 || t->nb[2] % 16 || t->nb[3] % 16)
            return fail(MXFA_ERR_UNSUPPORTED, "q/k/v must be F32 rows of 128 values, 16-byte aligned");
    // positions == NULL: no RoPE (DiT cross-attention); K/V may then have
    // their own token count
    const int64_t Nh = q->ne[1], Nkv = k->ne[1], S = q->ne[2], B = q->ne[3], Skv = k->ne[2];
    if (v->ne[1] != Nkv || v->ne[2] != Skv || k->ne[3] != B || v->ne[3] != B || (pos && Skv != S))
        return fail(MXFA_ERR_INVALID, "q/k/v shapes disagree");
    for (const mxfa_tensor *t : {qw, kw})
        if (t->type != MXFA_TYPE_F32 || t->ne[0] != kD || t->ne[1] * t->ne[2] * t->ne[3] != 1 || t->nb[0] != 4)
            return fail(MXFA_ERR_INVALID, "norm weights must be F32 [128]");
    for (const mxfa_tensor *t : {qw, kw})
        if (!is_aligned(t->data, 16)) return fail(MXFA_ERR_UNSUPPORTED, "norm weights must be 16-byte aligned");
    if (pos && (pos->type != MXFA_TYPE_I32 || pos->ne[0] != S || (pos->ne[1] != 1 && pos->ne[1] != B) ||
                pos->ne[2] != 1 || pos->ne[3] != 1 || pos->nb[0] != 4 ||
                (pos->ne[1] > 1 && pos->nb[1] != 4 * (size_t)S) || !is_aligned(pos->data, 4)))
        return fail(MXFA_ERR_INVALID, "positions must be I32 [S] or [S, B], contiguous");
    const int ot = qo->type;
    if (ot != MXFA_TYPE_F16 && ot != MXFA_TYPE_BF16)
        return fail(MXFA_ERR_UNSUPPORTED, "outputs must be F16 or BF16 (type %d)", ot);
    if (qo->ne[0] != kD || qo->ne[1] != Nh || qo->ne[2] != S || qo->ne[3] != B || qo->nb[0] != 2 ||
        qo->nb[1] != 2 * (size_t)kD || qo->nb[2] != qo->nb[1] * Nh || qo->nb[3] != qo->nb[2] * S ||
        !is_aligned(qo->data, 8))
        return fail(MXFA_ERR_INVALID, "q_out must be contiguous [128, Nh, S, B]");
    for (const mxfa_tensor *t : {ko, vo})
        if (t->type != ot || t->ne[0] != kD || t->ne[2] != Nkv || t->ne[3] != B || t->nb[0] != 2 ||
            !is_aligned(t->data, 8) || t->nb[1] % 8 || t->nb[2] % 8 || t->nb[3] % 8)
            return fail(MXFA_ERR_INVALID, "k_out/v_out must be [128, M, Nkv, B] of q_out's type, 8-byte aligned rows");
    if (ko->ne[1] != vo->ne[1] || ko->nb[1] != vo->nb[1] || ko->nb[2] != vo->nb[2] || ko->nb[3] != vo->nb[3])
        return fail(MXFA_ERR_INVALID, "k_out and v_out layouts differ");
    if (rows) {
        const size_t es = rows->type == MXFA_TYPE_I64 ? 8 : 4;
        if ((rows->type != MXFA_TYPE_I64 && rows->type != MXFA_TYPE_I32) || rows->ne[0] != Skv || B % rows->ne[1] ||
            rows->ne[2] != 1 || rows->ne[3] != 1 || rows->nb[0] != es || !is_aligned(rows->data, es) ||
            rows->nb[1] % es)
            return fail(MXFA_ERR_INVALID, "rows must be I64/I32 [Skv, R] with B %% R == 0");
    } else if (ko->ne[1] < Skv) {
        return fail(MXFA_ERR_INVALID, "without rows, k_out/v_out need at least one row per K/V token");
    }
    if (!(p->eps >= 0.0f) || !std::isfinite(p->eps) || !(p->freq_base > 0.0f) || !std::isfinite(p->freq_base))
        return fail(MXFA_ERR_INVALID, "eps / freq_base invalid");
    if ((Nh + 2 * Nkv) * std::max(S, Skv) * B >= ((int64_t)1 << 40) || std::max(S, Skv) * B >= ((int64_t)1 << 31) ||
        Nh + 2 * Nkv > 4096)
        return fail(MXFA_ERR_UNSUPPORTED, "too many rows");
    if (a) {
        NormRopeArgs &r = *a;
        r = NormRopeArgs{};
        r.q = (const char *)q->data;
        r.k = (const char *)k->data;
        r.v = (const char *)v->data;
        for (int i = 0; i < 3; i++) {
            r.q_nb[i] = (int64_t)q->nb[i + 1];
            r.k_nb[i] = (int64_t)k->nb[i + 1];
            r.v_nb[i] = (int64_t)v->nb[i + 1];
        }
        r.q_w = (const float *)qw->data;
        r.k_w = (const float *)kw->data;
        r.pos = pos ? (const int32_t *)pos->data : nullptr;
        r.pos_per_batch = pos && pos->ne[1] > 1;
        r.rope = pos != nullptr;
        r.Skv = (int32_t)Skv;
        r.eps = p->eps;
        r.theta_scale = std::pow(p->freq_base, -2.0f / (float)kD);
        r.clamp_v = p->clamp_v != 0;
        r.q_out = (char *)qo->data;
        r.k_out = (char *)ko->data;
        r.v_out = (char *)vo->data;
        r.kv_nb1 = (int64_t)ko->nb[1];
        r.kv_nb2 = (int64_t)ko->nb[2];
        r.kv_nb3 = (int64_t)ko->nb[3];
        r.kv_rows = ko->ne[1];
        if (rows) {
            r.rows = (const char *)rows->data;
            r.r_nb0 = (int64_t)rows->nb[0];
            r.r_nb1 = (int64_t)rows->nb[1];
            r.r_ne1 = (int32_t)rows->ne[1];
            r.rows_i64 = rows->type == MXFA_TYPE_I64;
        }
        r.Nh = (int32_t)Nh;
        r.Nkv = (int32_t)Nkv;
        r.S = (int32_t)S;
        r.B = (int32_t)B;
    }
    if (out_type) *out_type = ot;
    return MXFA_OK;
}

struct Plan {
    bool prefill = false;
    size_t cls_block = 0;   // prefill under a dense mask: tile classes, then (bits_off > 0) liveness words
    size_t bits_off = 0;
    bool wide = false;   // prefill on the 48-query-per-wave kernel (fa_wide.hip)
    FaArgs args{};
    int ktype = 0;
    int n_planes = 0;
    size_t ws_bytes = 0;
    int64_t n_tickets = 0;
    // prefill over a Q8_0 cache: K/V staged in F16 in the workspace, after
    // the tile classes (stage.ks/vs are set in run)
    bool q8_stage = false;
    Q8StageArgs stage{};
    size_t stage_off = 0;
};

// Full validation.  Returns MXFA_OK, MXFA_ERR_INVALID (malformed) or
// MXFA_ERR_UNSUPPORTED (well-formed but not handled by these kernels).
int check(const mxfa_tensor *q, const mxfa_tensor *k, const mxfa_tensor *v, const mxfa_tensor *mask,
          const mxfa_params *p, const mxfa_tensor *dst) {
    if (!q || !k || !v || !p) return fail(MXFA_ERR_INVALID, "q, k, v and params are required");
    for (const mxfa_tensor *t : {q, k, v, mask, dst}) {
        if (!t) continue;
        for (int i = 0; i < 4; i++)
            if (t->ne[i] <= 0) return fail(MXFA_ERR_INVALID, "ne[%d] = %lld must be positive", i, (long long)t->ne[i]);
    }
    // Q is F32 (ggml's FA input), or already in K's 16-bit type (F16 / BF16
    // K; the fused pre-attention kernel writes it so): ggml converts Q to
    // K's type before the KQ product, so both give the same operands.
    const bool q16 = (q->type == MXFA_TYPE_F16 || q->type == MXFA_TYPE_BF16) && q->type == k->type;
    if (q->type != MXFA_TYPE_F32 && !q16)
        return fail(MXFA_ERR_UNSUPPORTED, "q must be F32 or K's 16-bit type (q type %d, k type %d)", q->type, k->type);
    if (k->type != MXFA_TYPE_F16 && k->type != MXFA_TYPE_BF16 && k->type != MXFA_TYPE_Q8_0)
        return fail(MXFA_ERR_UNSUPPORTED, "k type %d not supported (F16, BF16, Q8_0)", k->type);
    if (v->type != k->type) return fail(MXFA_ERR_UNSUPPORTED, "k and v types differ (%d, %d)", k->type, v->type);
    if (q->ne[0] != k->ne[0]) return fail(MXFA_ERR_INVALID, "q->ne[0] != k->ne[0]");
    if (k->ne[1] != v->ne[1]) return fail(MXFA_ERR_INVALID, "k->ne[1] != v->ne[1]");
    if (q->ne[0] != kD || v->ne[0] != kD) return fail(MXFA_ERR_UNSUPPORTED, "head size %lld/%lld (only 128)",
                                                       (long long)q->ne[0], (long long)v->ne[0]);
    if (k->ne[2] != v->ne[2] || k->ne[3] != v->ne[3])
        return fail(MXFA_ERR_UNSUPPORTED, "k and v head/batch counts differ");
    if (q->ne[2] % k->ne[2]) return fail(MXFA_ERR_INVALID, "Nh %% Nkv != 0");
    if (q->ne[3] % k->ne[3]) return fail(MXFA_ERR_INVALID, "B %% Bk != 0");
    const int64_t lim = (int64_t)1 << 30;
    if (q->ne[1] > lim || q->ne[2] > 65535 || q->ne[3] > 65535 || k->ne[1] > lim)
        return fail(MXFA_ERR_UNSUPPORTED, "dimension too large");
    if (q->nb[0] != (q16 ? 2u : 4u)) return fail(MXFA_ERR_UNSUPPORTED, "q rows must be contiguous");
    if (k->nb[0] != type_block_bytes(k->type) || v->nb[0] != type_block_bytes(v->type))
        return fail(MXFA_ERR_UNSUPPORTED, "k/v rows must be contiguous");
    if (!q->data || !k->data || !v->data) return fail(MXFA_ERR_INVALID, "NULL data pointer");
    if (!is_aligned(q->data, 16) || q->nb[1] % 16 || q->nb[2] % 16 || q->nb[3] % 16)
        return fail(MXFA_ERR_UNSUPPORTED, "q data/strides must be 16-byte aligned");
    const size_t kv_align = k->type == MXFA_TYPE_Q8_0 ? 4 : 16;
    for (const mxfa_tensor *t : {k, v})
        if (!is_aligned(t->data, kv_align) || t->nb[1] % kv_align || t->nb[2] % kv_align || t->nb[3] % kv_align)
            return fail(MXFA_ERR_UNSUPPORTED, "k/v data/strides must be %zu-byte aligned", kv_align);
    if (mask) {
        if (mask->type != MXFA_TYPE_F16) return fail(MXFA_ERR_UNSUPPORTED, "mask must be F16");
        if (!mask->data) return fail(MXFA_ERR_INVALID, "NULL mask data");
        if (mask->nb[0] != 2) return fail(MXFA_ERR_UNSUPPORTED, "mask rows must be contiguous");
        if (mask->ne[0] < k->ne[1]) return fail(MXFA_ERR_INVALID, "mask->ne[0] < Skv");
        if (mask->ne[1] < q->ne[1]) return fail(MXFA_ERR_INVALID, "mask->ne[1] < Sq");
        if (q->ne[2] % mask->ne[2] || q->ne[3] % mask->ne[3])
            return fail(MXFA_ERR_INVALID, "mask does not broadcast over heads/batches");
        if (!is_aligned(mask->data, 2) || mask->nb[1] % 2 || mask->nb[2] % 2 || mask->nb[3] % 2)
            return fail(MXFA_ERR_INVALID, "mask misaligned");
    }
    if (!(p->scale == p->scale) || !std::isfinite(p->scale)) return fail(MXFA_ERR_INVALID, "scale not finite");
    if (p->max_bias < 0.0f || !std::isfinite(p->max_bias)) return fail(MXFA_ERR_INVALID, "max_bias invalid");
    if (!std::isfinite(p->logit_softcap)) return fail(MXFA_ERR_INVALID, "logit_softcap not finite");
    if (p->prec != MXFA_PREC_DEFAULT && p->prec != MXFA_PREC_F32) return fail(MXFA_ERR_INVALID, "prec %d", p->prec);
    if (dst) {
        if (dst->type != MXFA_TYPE_F32) return fail(MXFA_ERR_UNSUPPORTED, "dst must be F32");
        if (dst->ne[0] != v->ne[0] || dst->ne[1] != q->ne[2] || dst->ne[2] != q->ne[1] || dst->ne[3] != q->ne[3])
            return fail(MXFA_ERR_INVALID, "dst shape must be [DV, Nh, Sq, B]");
        const size_t nb1 = 4 * (size_t)dst->ne[0], nb2 = nb1 * dst->ne[1], nb3 = nb2 * dst->ne[2];
        if (dst->nb[0] != 4 || dst->nb[1] != nb1 || dst->nb[2] != nb2 || dst->nb[3] != nb3)
            return fail(MXFA_ERR_UNSUPPORTED, "dst must be contiguous");
        if (!dst->data || !is_aligned(dst->data, 16)) return fail(MXFA_ERR_INVALID, "dst data NULL or misaligned");
    }
    return MXFA_OK;
}

// Validation of a structured mask (mxfa_mask_spec) for q's shape.
int check_spec(const mxfa_mask_spec *sm, const mxfa_tensor *q) {
    if (!sm) return fail(MXFA_ERR_INVALID, "mask spec is required");
    if (sm->flags & ~(MXFA_MASK_CAUSAL | MXFA_MASK_WINDOW | MXFA_MASK_LENGTHS | MXFA_MASK_DEVICE))
        return fail(MXFA_ERR_INVALID, "unknown mask flags 0x%x", sm->flags);
    const bool dev = (sm->flags & MXFA_MASK_DEVICE) != 0;
    const int64_t lim = (int64_t)1 << 30;
    const int64_t w = (sm->flags & MXFA_MASK_WINDOW) ? sm->window : 0;
    if (w < 0 || w >= lim) return fail(MXFA_ERR_INVALID, "window %d out of range", sm->window);
    if (sm->pos0 < 0 || sm->pos0 + q->ne[1] + w >= lim) return fail(MXFA_ERR_INVALID, "pos0 / window out of range");
    if (dev && q->ne[1] + w >= lim) return fail(MXFA_ERR_INVALID, "Sq + window out of range");
    if (sm->flags & MXFA_MASK_LENGTHS) {
        if (!sm->lengths) return fail(MXFA_ERR_INVALID, "MXFA_MASK_LENGTHS without lengths");
        if (sm->n_lengths != 1 && sm->n_lengths != q->ne[3])
            return fail(MXFA_ERR_INVALID, "n_lengths %d must be 1 or B = %lld", sm->n_lengths, (long long)q->ne[3]);
        if (sm->n_lengths > kSmMaxLen)
            return fail(MXFA_ERR_UNSUPPORTED, "n_lengths %d > %d", sm->n_lengths, kSmMaxLen);
        if (!dev)   // (device lengths are read, and clamped, by the kernels)
            for (int i = 0; i < sm->n_lengths; i++)
                if (sm->lengths[i] < 0) return fail(MXFA_ERR_INVALID, "lengths[%d] = %d < 0", i, sm->lengths[i]);
    }
    return MXFA_OK;
}

// ws_cap: workspace bytes the call may use (the allocation-free entry
// point's fixed scratch); a prompt over a Q8_0 cache whose F16 staging does
// not fit takes the decode kernel instead, which stages nothing.
void make_plan(const mxfa_tensor *q, const mxfa_tensor *k, const mxfa_tensor *v, const mxfa_tensor *mask,
               const mxfa_params *p, mxfa_tensor *dst, Plan &pl, const mxfa_mask_spec *sm = nullptr,
               size_t ws_cap = SIZE_MAX) {
    FaArgs &a = pl.args;
    const bool sm_dev = sm && (sm->flags & MXFA_MASK_DEVICE);
    if (sm && (sm->flags & ~MXFA_MASK_DEVICE)) {
        a.sm_flags = sm->flags;
        a.sm_window = (sm->flags & MXFA_MASK_WINDOW) ? sm->window : 0;
        a.sm_pos0 = (int32_t)sm->pos0;
        a.sm_nlen = 1;
        if (sm_dev) a.sm_pos0_dev = sm->dev_pos0;
        if (sm->flags & MXFA_MASK_LENGTHS) {
            a.sm_nlen = sm->n_lengths;
            if (sm_dev) {
                a.sm_len_dev = sm->lengths;
            } else {
                for (int i = 0; i < sm->n_lengths; i++)
                    a.sm_len[i] = (int32_t)std::min<int64_t>(sm->lengths[i], k->ne[1]);
            }
        }
    }
    a.q = (const char *)q->data;
    a.k = (const char *)k->data;
    a.v = (const char *)v->data;
    a.mask = mask ? (const char *)mask->data : nullptr;
    a.dst = dst ? (float *)dst->data : nullptr;
    a.q_nb1 = (int64_t)q->nb[1]; a.q_nb2 = (int64_t)q->nb[2]; a.q_nb3 = (int64_t)q->nb[3];
    a.q16 = q->type != MXFA_TYPE_F32;
    a.k_nb1 = (int64_t)k->nb[1]; a.k_nb2 = (int64_t)k->nb[2]; a.k_nb3 = (int64_t)k->nb[3];
    a.v_nb1 = (int64_t)v->nb[1]; a.v_nb2 = (int64_t)v->nb[2]; a.v_nb3 = (int64_t)v->nb[3];
    if (mask) {
        a.m_nb1 = (int64_t)mask->nb[1]; a.m_nb2 = (int64_t)mask->nb[2]; a.m_nb3 = (int64_t)mask->nb[3];
        a.m_ne2 = (int32_t)mask->ne[2]; a.m_ne3 = (int32_t)mask->ne[3];
    } else {
        a.m_ne2 = 1; a.m_ne3 = 1;
    }
    a.Sq = (int32_t)q->ne[1];
    a.Nh = (int32_t)q->ne[2];
    a.B = (int32_t)q->ne[3];
    a.Skv = (int32_t)k->ne[1];
    a.Nkv = (int32_t)k->ne[2];
    a.G = a.Nh / a.Nkv;
    a.rk3 = (int32_t)(q->ne[3] / k->ne[3]);
    a.M = a.Sq * a.G;
    a.scale = p->scale;
    a.softcap = p->logit_softcap;
    a.max_bias = p->max_bias;
    // ALiBi constants as ggml computes them (per-head slopes).
    const uint32_t n_head = (uint32_t)a.Nh;
    a.n_head_log2 = 1u << (uint32_t)std::floor(std::log2((double)n_head));
    const float m0 = std::pow(2.0f, -(p->max_bias) / (float)a.n_head_log2);
    const float m1 = std::pow(2.0f, -(p->max_bias / 2.0f) / (float)a.n_head_log2);
    a.l2m0 = (float)std::log2((double)m0);
    a.l2m1 = (float)std::log2((double)m1);
    a.softcap_in = p->logit_softcap != 0.0f ? p->scale / p->logit_softcap : 0.0f;
    pl.ktype = k->type;

    auto mask_rows_aligned = [&](size_t al) {
        return mask && is_aligned(mask->data, al) && mask->nb[1] % al == 0 && mask->nb[2] % al == 0 &&
               mask->nb[3] % al == 0;
    };
    a.mask_al8 = mask_rows_aligned(8);
    a.mask_al16 = mask_rows_aligned(16);
    a.mask_vec4 = a.mask_al8 && mask->ne[0] >= ((k->ne[1] + 3) & ~(int64_t)3);
    a.mask_vec16 = a.mask_vec4 && mask->ne[0] >= 16;
    // prefill: mask rows are read in 8-byte groups of 4 keys (rows 8-byte
    // aligned) through a buffer resource over one mask plane, addressed
    // with 32-bit offsets.  With ne0 % 4 == 0 every group that starts below
    // Skv lies wholly inside its row, so no load that carries a live key
    // crosses the end of the plane (a contiguous 8-byte aligned mask has
    // ne0 % 4 == 0 anyway; other strided views go to the decode kernel).
    if (mask) {
        const uint64_t plane = (uint64_t)(mask->ne[1] - 1) * mask->nb[1] + 2 * (uint64_t)mask->ne[0];
        a.m_plane_bytes = plane <= 0x7FFFFFFFull ? (uint32_t)plane : 0;
    }
    const bool mask_vec_ok = !mask || (a.mask_al8 && a.m_plane_bytes != 0 && mask->ne[0] % 4 == 0);
    const int64_t n_kt = (a.Skv + kPfBN - 1) / kPfBN;
    // the prefill kernel addresses one (batch, kv head)'s K and V rows with
    // 32-bit offsets from a buffer base: every row of every key tile must
    // lie within 4 GiB of it
    // A Q8_0 cache goes to the prefill kernel through F16 staging of K/V
    // (q8_stage.hip): contiguous rows of 256 bytes.
    const bool q8 = k->type == MXFA_TYPE_Q8_0;
    const uint64_t row_bytes = q8 ? 256 : (uint64_t)std::max(k->nb[1], v->nb[1]);
    const bool offsets_32 = (uint64_t)n_kt * kPfBN * row_bytes <= 0xFFFFFFFFull;
    const int64_t n_kv_rows = k->ne[1] * k->ne[2] * k->ne[3];
    const bool stage_ok = !q8 || 32 * n_kv_rows < ((int64_t)1 << 31);
    // (classes of every mask plane, then 256 B of F16 staging per K and per
    // V row; bounds as in the prefill branch below)
    const uint64_t n_qt_pf = (uint64_t)(a.Sq + kPfBM - 1) / kPfBM, n_kt_pad_pf = ((uint64_t)n_kt + 3) & ~3ull;
    const uint64_t cls_pf = mask ? (uint64_t)a.m_ne2 * a.m_ne3 * n_qt_pf * n_kt_pad_pf : 0;
    const bool stage_fits = !q8 || ((cls_pf + 255) & ~255ull) + 512ull * (uint64_t)n_kv_rows <= ws_cap;
    // the liveness words of class-3 tiles (8 bytes per query row and key
    // tile) follow the classes when the workspace can hold them; otherwise
    // the classifier labels such tiles 2
    const uint64_t bits_pf = mask ? (uint64_t)a.m_ne2 * a.m_ne3 * n_qt_pf * kPfBM * (uint64_t)n_kt * 8 : 0;
    const uint64_t with_bits = ((cls_pf + 255) & ~255ull) + ((bits_pf + 255) & ~255ull);
    // (Q8_0 calls keep reading mask values: their prefill instance has no
    // word path)
    const bool bits_fit = mask && !q8 && with_bits <= ws_cap;
    pl.prefill = (k->type == MXFA_TYPE_F16 || k->type == MXFA_TYPE_BF16 || q8) && a.Sq >= kPrefillMinSq &&
                 mask_vec_ok && offsets_32 && stage_ok && stage_fits && (!mask || n_kt <= kPfMaxKeyTiles);
    if (pl.prefill) {
        a.n_qt = (a.Sq + kPfBM - 1) / kPfBM;
        a.n_kt = (int32_t)n_kt;
        a.n_kt_pad = (a.n_kt + 3) & ~3;
        // F16 calls without a mask (the DiT's self-attention: the reference
        // casts K/V to F16 first) or with a dense mask over few key tiles
        // (the DiT's cross-attention) take the kernel with 48 queries per
        // wave: 192-query workgroups, each LDS operand read once for three
        // MFMAs.  Same-box A/B against the 32-query kernel: C4 self 149.0
        // against 164.0 us, C4 cross 35.1-35.6 against 37.5-37.6 us.  (BF16
        // stays on the 32-query kernel: its P hi/lo pair does not fit the
        // wide kernel's registers without spills.)
        // The same rule holds for a dense mask and its structured form, so
        // that the two stay on one kernel (bit-identical outputs).
        pl.wide = kPfWide && k->type == MXFA_TYPE_F16 && a.softcap == 0.0f &&
                  ((!mask && a.sm_flags == 0) || n_kt <= kPfWideMaskedMaxKt);
        a.n_qt_w = pl.wide ? (a.Sq + kPfWideBM - 1) / kPfWideBM : 0;
        pl.n_planes = mask ? a.m_ne2 * a.m_ne3 : 0;
        pl.ws_bytes = mask ? (size_t)pl.n_planes * a.n_qt * a.n_kt_pad : 0;
        if (bits_fit) {
            pl.bits_off = (pl.ws_bytes + 255) & ~(size_t)255;
            pl.ws_bytes = (size_t)with_bits;
        }
        pl.cls_block = pl.ws_bytes;
        a.n_splits = 1;
        a.chunk = a.Skv;
        if (q8) {
            Q8StageArgs &st = pl.stage;
            st.k = a.k; st.v = a.v;
            st.k_nb1 = a.k_nb1; st.k_nb2 = a.k_nb2; st.k_nb3 = a.k_nb3;
            st.v_nb1 = a.v_nb1; st.v_nb2 = a.v_nb2; st.v_nb3 = a.v_nb3;
            st.Skv = (uint32_t)a.Skv; st.Nkv = (uint32_t)a.Nkv;
            st.n_kv = (uint32_t)n_kv_rows;   // (Q: quantised to Q8_0 by the prefill kernel on load)
            pl.q8_stage = true;
            pl.stage_off = (pl.ws_bytes + 255) & ~(size_t)255;
            pl.ws_bytes = pl.stage_off + 256 * (size_t)(2 * n_kv_rows);
            // the prefill reads the staged F16 K and V rows [128, Skv, Nkv, Bk]
            a.k_nb1 = a.v_nb1 = 256;
            a.k_nb2 = a.v_nb2 = 256 * (int64_t)a.Skv;
            a.k_nb3 = a.v_nb3 = a.k_nb2 * a.Nkv;
        }
        return;
    }
    a.row_tiles = (a.M + 15) / 16;
    const int64_t base = (int64_t)a.B * a.Nkv * a.row_tiles;
    // Splits are whole steps of the kernel that runs them: 64 keys for the
    // LDS kernel (F16/BF16 with no dense mask or one of 16-byte rows; a
    // structured call has no dense mask: 4 waves x 16 keys), 128 for the
    // register kernel (4 x 32).  Short windows then split finer: C1's 512
    // keys into 8 splits per KV head instead of 4, 9.67 -> 8.95 us per call,
    // the 28-layer decode token 377.5 -> 355.3 us replayed; structured
    // splits of equal live work come closer to it: c3m 36.5-36.8 -> 35.9-36.0
    // us (same box each).
    const bool lds_kernel = k->type != MXFA_TYPE_Q8_0 && (!mask || a.mask_vec16);
    const int64_t quantum = lds_kernel ? kSplitKeyQuantumLds : kSplitKeyQuantum;
    const int64_t max_splits = (a.Skv + quantum - 1) / quantum;
    int64_t n_splits = 1, chunk = 0;
    auto round_q = [&](int64_t x) { return (x + quantum - 1) / quantum * quantum; };
    if (a.sm_flags && !sm_dev) {
        // Structured mask: every (batch, kv head, row tile) stream covers
        // the keys its rows see; one chunk size for all of them, from the
        // total live work, so that every split carries the same work.
        int64_t total = 0, max_len = 0;
        std::vector<int64_t> lens((size_t)a.B * a.row_tiles);
        for (int b = 0; b < a.B; b++)
            for (int rt = 0; rt < a.row_tiles; rt++) {
                const int r0 = rt * 16, nr = std::min(16, a.M - r0);
                int lo_f, hi_f, lo_l, hi_l;
                sm_row_range(a, b, r0 / a.G, lo_f, hi_f);
                sm_row_range(a, b, (r0 + nr - 1) / a.G, lo_l, hi_l);
                const int64_t len = std::max(0, hi_l - lo_f);
                lens[(size_t)b * a.row_tiles + rt] = len;
                total += len * a.Nkv;
                max_len = std::max(max_len, len);
            }
        chunk = round_q(std::max<int64_t>({(total + kSplitTargetWgs - 1) / kSplitTargetWgs,
                                           (max_len + kMaxDecodeSplits - 1) / kMaxDecodeSplits, 1}));
        // the grid is the list of live splits, (b, rt, split) major, kv head
        // minor, in the order the kernel walks them (each workgroup walks
        // the (b, rt) list to find its split: short lists only)
        int64_t live = 0;
        for (int64_t len : lens) {
            const int64_t ns = std::max<int64_t>(1, (len + chunk - 1) / chunk);
            n_splits = std::max<int64_t>(n_splits, ns);
            live += ns * a.Nkv;
        }
        if (lens.size() <= (size_t)kMaxLiveListTiles) a.dec_live = (int32_t)live;
    } else {
        if (base < kSplitTargetWgs)
            n_splits = std::min<int64_t>({max_splits, (kSplitTargetWgs + base - 1) / base, kMaxDecodeSplits});
        chunk = round_q((a.Skv + n_splits - 1) / n_splits);
        n_splits = (a.Skv + chunk - 1) / chunk;
    }
    a.n_splits = (int32_t)n_splits;
    a.chunk = (int32_t)chunk;
    // Paired splits (fa_decode.hip, make_tile): a dense grid of exactly two
    // workgroups per CU whose first half runs ahead of its second; the even
    // split of each pair (first half) takes kDecPairNum/8 of the pair's
    // 2 chunks / 2, rounded to the key quantum.
    if (!a.sm_flags && kDecPairNum > 8 && n_splits % 2 == 0 && base * n_splits == 2 * kDecCus) {
        const int64_t want = (chunk * kDecPairNum / 8 + kSplitKeyQuantum / 2) / kSplitKeyQuantum * kSplitKeyQuantum;
        if (want > chunk && want < 2 * chunk) a.dec_pair = (int32_t)want;
    }
    if (n_splits > 1) {
        const size_t rows = (size_t)a.B * a.Nkv * a.M * n_splits;
        pl.ws_bytes = rows * kD * sizeof(float) + rows * 2 * sizeof(float);
        pl.n_tickets = (int64_t)a.B * a.Nkv * a.row_tiles;
    }
}

// Workspace of (current device, stream), created on first use (g_ws_mu held).
int workspace_of(hipStream_t stream, Workspace **out) {
    int dev = 0;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(MXFA_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
    for (Workspace &w : g_ws)
        if (w.device == dev && w.stream == stream) {
            *out = &w;
            return MXFA_OK;
        }
    g_ws.push_back(Workspace{});
    g_ws.back().device = dev;
    g_ws.back().stream = stream;
    *out = &g_ws.back();
    return MXFA_OK;
}

// Tile classes of a dense mask within the stream's current graph.  Sets
// *cls to NULL when no graph has begun on the stream (the call classifies
// into its workspace as before); else to the mask's class bytes in the
// stream's arena, with *fresh = true when this call is the mask's first use
// in the graph (it must run the classifier) and false when an earlier node
// of the graph already did.  The arena grows (the old one is retired, as
// workspaces are) except under capture.
int graph_classes(const mxfa_tensor *mask, int64_t Sq, int64_t Skv, size_t bytes, hipStream_t stream, uint8_t **cls,
                  bool *fresh) {
    *cls = nullptr;
    *fresh = false;
    std::lock_guard<std::mutex> lock(g_ws_mu);
    Workspace *w = nullptr;
    const int rc = workspace_of(stream, &w);
    if (rc != MXFA_OK) return rc;
    if (w->epoch == 0) return MXFA_OK;
    for (const ClassEntry &c : w->entries) {
        bool same = c.data == mask->data && c.Sq == Sq && c.Skv == Skv && c.bytes == bytes;
        for (int i = 0; i < 4 && same; i++) same = c.ne[i] == mask->ne[i] && c.nb[i] == mask->nb[i];
        if (same) {
            *cls = c.cls;
            return MXFA_OK;
        }
    }
    const size_t need = (w->arena_used + bytes + 255) & ~(size_t)255;
    if (need > w->arena_size) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
            return fail(MXFA_ERR_UNSUPPORTED,
                        "the graph's mask class arena must grow (%zu bytes) while the stream is being captured; "
                        "compute the graph once eagerly before capturing it",
                        need);
        const size_t want = std::max<size_t>((size_t)64 << 10, 2 * need);
        void *p = nullptr;
        const hipError_t e = hipMalloc(&p, want);
        if (e != hipSuccess) return fail(MXFA_ERR_NOMEM, "hipMalloc(%zu): %s", want, hipGetErrorString(e));
        if (w->arena) w->retired.push_back(w->arena);
        w->arena = (uint8_t *)p;
        w->arena_size = want;
        w->arena_used = 0;   // (entries of this graph keep their bytes in the retired arena)
    }
    ClassEntry c;
    c.data = mask->data;
    for (int i = 0; i < 4; i++) {
        c.ne[i] = mask->ne[i];
        c.nb[i] = mask->nb[i];
    }
    c.Sq = Sq;
    c.Skv = Skv;
    c.bytes = bytes;
    c.cls = w->arena + w->arena_used;
    w->arena_used = (w->arena_used + bytes + 255) & ~(size_t)255;
    w->entries.push_back(c);
    *cls = c.cls;
    *fresh = true;
    return MXFA_OK;
}

int ensure_workspace(size_t bytes, int64_t n_tickets, hipStream_t stream, void **out, int **tickets) {
    *out = nullptr;
    *tickets = nullptr;
    if (bytes == 0 && n_tickets == 0) return MXFA_OK;
    std::lock_guard<std::mutex> lock(g_ws_mu);
    Workspace *found = nullptr;
    const int rc = workspace_of(stream, &found);
    if (rc != MXFA_OK) return rc;
    Workspace &ws = *found;
    hipError_t e;
    if (ws.size < bytes || ws.n_tickets < n_tickets) {
        // Growing allocates, which a stream under HIP graph capture cannot
        // do: the first call of a shape must run eagerly (or through
        // mxfa_reserve) before a graph containing it is captured.
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
            return fail(MXFA_ERR_UNSUPPORTED,
                        "workspace must grow (%zu bytes, %lld tickets) while the stream is being captured; "
                        "run the call once eagerly or call mxfa_reserve() before capture",
                        bytes, (long long)n_tickets);
    }
    // An outgrown buffer is retired, not freed: kernels queued on the
    // stream, and graphs captured earlier, keep using its address.
    if (ws.size < bytes) {
        // at least double: a prompt continued over a growing cache (Q8_0
        // staging grows with Skv) regrows O(log) times, and the retired
        // chain stays below the final size
        size_t want = std::max(bytes + bytes / 4, 2 * ws.size);
        want = (want + 4095) & ~(size_t)4095;
        void *p = nullptr;
        e = hipMalloc(&p, want);
        if (e != hipSuccess) return fail(MXFA_ERR_NOMEM, "hipMalloc(%zu): %s", want, hipGetErrorString(e));
        if (ws.ptr) ws.retired.push_back(ws.ptr);
        ws.ptr = p;
        ws.size = want;
    }
    if (ws.n_tickets < n_tickets) {
        const int64_t want = std::max<int64_t>(1024, n_tickets + n_tickets / 4);
        int *p = nullptr;
        e = hipMalloc((void **)&p, (size_t)want * sizeof(int));
        if (e != hipSuccess) return fail(MXFA_ERR_NOMEM, "hipMalloc(tickets): %s", hipGetErrorString(e));
        e = launch_fill_zero(p, want, stream);
        if (e != hipSuccess) {
            (void)hipFree(p);
            return fail(MXFA_ERR_HIP, "ticket fill: %s", hipGetErrorString(e));
        }
        if (ws.tickets) ws.retired.push_back(ws.tickets);
        ws.tickets = p;
        ws.n_tickets = want;
    }
    *out = ws.ptr;
    *tickets = ws.tickets;
    return MXFA_OK;
}

// -- per-kernel timing ---------------------------------------------------------
struct TimedLaunch {
    std::string family;
    hipEvent_t start = nullptr, stop = nullptr;
    int launches = 1;   // back-to-back launches between the two events
};
struct FamilyStats {
    double ms = 0.0;
    int64_t launches = 0;
};
std::atomic<int> g_timing{0};   // launches per bracket (0: timing off)
std::mutex g_timing_mu;
std::vector<TimedLaunch *> g_pending;
std::vector<std::pair<std::string, FamilyStats>> g_stats;

FamilyStats &stats_of(const std::string &f) {
    for (auto &kv : g_stats)
        if (kv.first == f) return kv.second;
    g_stats.emplace_back(f, FamilyStats{});
    return g_stats.back().second;
}

// Waits for and folds every pending event pair into the per-family totals.
void drain_pending() {
    for (TimedLaunch *t : g_pending) {
        float ms = 0.0f;
        if (t->stop && hipEventSynchronize(t->stop) == hipSuccess &&
            hipEventElapsedTime(&ms, t->start, t->stop) == hipSuccess) {
            FamilyStats &st = stats_of(t->family);
            st.ms += ms;
            st.launches += t->launches;
        }
        if (t->start) (void)hipEventDestroy(t->start);
        if (t->stop) (void)hipEventDestroy(t->stop);
        delete t;
    }
    g_pending.clear();
}

// -- the allocation-free variant's scratch ------------------------------------
// A fixed device array per GPU (this code object's copy on each device)
// stands in for the grow-only workspace: the tickets at its start, the split
// partials or mask tile classes after them.  Host code never passes the
// array's name to a kernel: it looks up each device's address once
// (hipGetSymbolAddress) and uses that.
constexpr size_t kScratchBytes = (size_t)8 << 20;      // 8 MiB per GPU, held until the process ends
constexpr int64_t kScratchTickets = 65536;             // 256 KiB of split tickets
constexpr size_t kScratchTicketBytes = (size_t)kScratchTickets * sizeof(int);
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

struct Scratch {
    void *ws = nullptr;       // partials / classes
    size_t ws_bytes = 0;
    int *tickets = nullptr;
    int64_t n_tickets = 0;
};
std::mutex g_scratch_mu;
std::vector<void *> g_scratch_ptr;   // per device: the array's address, nullptr until set up

// Set-up on the current device (first call there): the array's device
// address, and one zero fill of its tickets (a kernel on `stream`; the
// kernels leave every ticket at zero after that).  Refused while `stream`
// is being captured.
int scratch_of_device(hipStream_t stream, Scratch *out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(MXFA_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if ((size_t)dev >= g_scratch_ptr.size()) g_scratch_ptr.resize(dev + 1, nullptr);
    if (!g_scratch_ptr[dev]) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
            return fail(MXFA_ERR_UNSUPPORTED,
                        "the first mxfa_flash_attn_ext_noalloc call on a device sets up its scratch and must "
                        "not be captured: call it once eagerly first");
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return fail(MXFA_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        e = launch_fill_zero((int *)ptr, kScratchTickets, stream);
        if (e != hipSuccess) return fail(MXFA_ERR_HIP, "scratch ticket fill: %s", hipGetErrorString(e));
        g_scratch_ptr[dev] = ptr;
    }
    uint8_t *base = (uint8_t *)g_scratch_ptr[dev];
    out->tickets = (int *)base;
    out->n_tickets = kScratchTickets;
    out->ws = base + kScratchTicketBytes;
    out->ws_bytes = kScratchBytes - kScratchTicketBytes;
    return MXFA_OK;
}

// Plans and launches one validated call (dense `mask` or structured `sm`).
// `fixed`: use that scratch instead of the stream's grow-only workspace
// (the allocation-free entry point); a call that needs more fails.
int run(const mxfa_tensor *q, const mxfa_tensor *k, const mxfa_tensor *v, const mxfa_tensor *mask,
        const mxfa_params *params, mxfa_tensor *dst, void *hip_stream, const mxfa_mask_spec *sm,
        const Scratch *fixed = nullptr) {
    hipStream_t stream = (hipStream_t)hip_stream;
    Plan pl;
    make_plan(q, k, v, mask, params, dst, pl, sm, fixed ? fixed->ws_bytes : SIZE_MAX);
    void *ws = nullptr;
    if (!pl.prefill && (int64_t)pl.args.Nkv * pl.args.row_tiles > 65535)
        return fail(MXFA_ERR_UNSUPPORTED, "too many query rows per KV head for the decode kernel");
    int *tickets = nullptr;
    if (fixed) {
        if (pl.ws_bytes > fixed->ws_bytes || pl.n_tickets > fixed->n_tickets)
            return fail(MXFA_ERR_UNSUPPORTED,
                        "call needs %zu bytes of partials/classes and %lld tickets; the allocation-free scratch "
                        "holds %zu bytes and %lld tickets",
                        pl.ws_bytes, (long long)pl.n_tickets, fixed->ws_bytes, (long long)fixed->n_tickets);
        ws = fixed->ws;
        tickets = fixed->tickets;
    } else {
        const int rc = ensure_workspace(pl.ws_bytes, pl.n_tickets, stream, &ws, &tickets);
        if (rc != MXFA_OK) return rc;
    }
    FaArgs &a = pl.args;
    hipError_t e;
    if (pl.prefill) {
        if (pl.q8_stage) {
            char *base = (char *)ws + pl.stage_off;
            Q8StageArgs &st = pl.stage;
            st.ks = base;
            st.vs = st.ks + 256 * (size_t)st.n_kv;
            a.k = st.ks;
            a.v = st.vs;
            e = timed_launch("q8_stage", stream, [&] { return launch_q8_stage(st, stream); });
            if (e != hipSuccess) return fail(MXFA_ERR_HIP, "q8 stage launch: %s", hipGetErrorString(e));
        }
        if (a.mask) {
            // within a graph (mxfa_graph_begin) a mask is classified at its
            // first node only; otherwise every call classifies its own
            uint8_t *cls = (uint8_t *)ws;
            bool classify = true;
            if (!fixed) {
                uint8_t *gc = nullptr;
                const int rc = graph_classes(mask, a.Sq, a.Skv, pl.cls_block, stream, &gc, &classify);
                if (rc != MXFA_OK) return rc;
                if (gc) cls = gc;
                else classify = true;
            }
            a.tile_class = cls;
            a.tile_bits = pl.bits_off ? (uint64_t *)(cls + pl.bits_off) : nullptr;
            if (classify) {
                e = timed_launch("mask_classify", stream,
                                 [&] { return launch_mask_classify(a, pl.n_planes, cls, stream); });
                if (e != hipSuccess) return fail(MXFA_ERR_HIP, "mask classify launch: %s", hipGetErrorString(e));
            }
        }
        e = timed_launch("fa_prefill", stream, [&] {
            return pl.wide ? launch_fa_wide(a, pl.ktype, stream) : launch_fa_prefill(a, pl.ktype, stream);
        });
        if (e != hipSuccess) return fail(MXFA_ERR_HIP, "prefill launch: %s", hipGetErrorString(e));
        return MXFA_OK;
    }
    if (a.n_splits > 1) {
        const size_t rows = (size_t)a.B * a.Nkv * a.M * a.n_splits;
        a.part_o = (float *)ws;
        a.part_ml = a.part_o + rows * kD;
        a.tickets = tickets;
    }
    e = launch_fa_decode(a, pl.ktype, stream);
    if (e != hipSuccess) return fail(MXFA_ERR_HIP, "decode launch: %s", hipGetErrorString(e));
    return MXFA_OK;
}

}  // namespace

namespace mxfa {

int timing_mode() { return g_timing.load(std::memory_order_relaxed); }

void timing_begin(const char *family, hipStream_t stream, void **token) {
    TimedLaunch *t = new TimedLaunch;
    t->family = family;
    if (hipEventCreate(&t->start) != hipSuccess || hipEventRecord(t->start, stream) != hipSuccess) {
        if (t->start) (void)hipEventDestroy(t->start);
        delete t;
        *token = nullptr;
        return;
    }
    *token = t;
}

void timing_end(void *token, hipStream_t stream, int launches) {
    TimedLaunch *t = (TimedLaunch *)token;
    if (!t) return;
    t->launches = launches;
    if (hipEventCreate(&t->stop) != hipSuccess || hipEventRecord(t->stop, stream) != hipSuccess) {
        if (t->stop) (void)hipEventDestroy(t->stop);
        t->stop = nullptr;
    }
    std::lock_guard<std::mutex> lock(g_timing_mu);
    g_pending.push_back(t);
}

}  // namespace mxfa

extern "C" {

int mxfa_supports(const mxfa_tensor *q, const mxfa_tensor *k, const mxfa_tensor *v, const mxfa_tensor *mask,
                  const mxfa_params *params, const mxfa_tensor *dst) {
    const int rc = check(q, k, v, mask, params, dst);
    if (rc != MXFA_OK) return 0;
    Plan pl;
    make_plan(q, k, v, mask, params, nullptr, pl);
    if (!pl.prefill && (int64_t)pl.args.Nkv * pl.args.row_tiles > 65535) {
        fail(MXFA_ERR_UNSUPPORTED, "too many query rows per KV head for the decode kernel");
        return 0;
    }
    return 1;
}

int mxfa_flash_attn_ext(const mxfa_tensor *q, const mxfa_tensor *k, const mxfa_tensor *v, const mxfa_tensor *mask,
                        const mxfa_params *params, mxfa_tensor *dst, void *hip_stream) {
    if (!dst) return fail(MXFA_ERR_INVALID, "dst is required");
    const int rc = check(q, k, v, mask, params, dst);
    if (rc != MXFA_OK) return rc;
    return run(q, k, v, mask, params, dst, hip_stream, nullptr);
}

int mxfa_flash_attn_ext_noalloc(const mxfa_tensor *q, const mxfa_tensor *k, const mxfa_tensor *v,
                                const mxfa_tensor *mask, const mxfa_params *params, mxfa_tensor *dst,
                                void *hip_stream) {
    if (!dst) return fail(MXFA_ERR_INVALID, "dst is required");
    int rc = check(q, k, v, mask, params, dst);
    if (rc != MXFA_OK) return rc;
    Scratch sc;
    rc = scratch_of_device((hipStream_t)hip_stream, &sc);
    if (rc != MXFA_OK) return rc;
    return run(q, k, v, mask, params, dst, hip_stream, nullptr, &sc);
}

int mxfa_reserve(const mxfa_tensor *q, const mxfa_tensor *k, const mxfa_tensor *v, const mxfa_tensor *mask,
                 const mxfa_params *params, void *hip_stream) {
    const int rc = check(q, k, v, mask, params, nullptr);
    if (rc != MXFA_OK) return rc;
    Plan pl;
    make_plan(q, k, v, mask, params, nullptr, pl);
    void *ws = nullptr;
    int *tickets = nullptr;
    return ensure_workspace(pl.ws_bytes, pl.n_tickets, (hipStream_t)hip_stream, &ws, &tickets);
}

int mxfa_graph_begin(void *hip_stream) {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    Workspace *w = nullptr;
    const int rc = workspace_of((hipStream_t)hip_stream, &w);
    if (rc != MXFA_OK) return rc;
    w->epoch++;
    w->arena_used = 0;
    w->entries.clear();
    return MXFA_OK;
}

int mxfa_graph_end(void *hip_stream) {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    Workspace *w = nullptr;
    const int rc = workspace_of((hipStream_t)hip_stream, &w);
    if (rc != MXFA_OK) return rc;
    w->epoch = 0;
    w->arena_used = 0;
    w->entries.clear();
    return MXFA_OK;
}

int mxfa_supports_masked(const mxfa_tensor *q, const mxfa_tensor *k, const mxfa_tensor *v, const mxfa_mask_spec *mask,
                         const mxfa_params *params, const mxfa_tensor *dst) {
    if (check(q, k, v, nullptr, params, dst) != MXFA_OK || check_spec(mask, q) != MXFA_OK) return 0;
    Plan pl;
    make_plan(q, k, v, nullptr, params, nullptr, pl, mask);
    if (!pl.prefill && (int64_t)pl.args.Nkv * pl.args.row_tiles > 65535) {
        fail(MXFA_ERR_UNSUPPORTED, "too many query rows per KV head for the decode kernel");
        return 0;
    }
    return 1;
}

int mxfa_flash_attn_ext_masked(const mxfa_tensor *q, const mxfa_tensor *k, const mxfa_tensor *v,
                               const mxfa_mask_spec *mask, const mxfa_params *params, mxfa_tensor *dst,
                               void *hip_stream) {
    if (!dst) return fail(MXFA_ERR_INVALID, "dst is required");
    int rc = check(q, k, v, nullptr, params, dst);
    if (rc != MXFA_OK) return rc;
    rc = check_spec(mask, q);
    if (rc != MXFA_OK) return rc;
    return run(q, k, v, nullptr, params, dst, hip_stream, mask);
}

int mxfa_qk_norm_rope(const mxfa_tensor *q, const mxfa_tensor *k, const mxfa_tensor *v, const mxfa_tensor *q_norm,
                      const mxfa_tensor *k_norm, const mxfa_tensor *positions, const mxfa_norm_rope_params *params,
                      mxfa_tensor *q_out, mxfa_tensor *k_out, mxfa_tensor *v_out, const mxfa_tensor *rows,
                      void *hip_stream) {
    NormRopeArgs a;
    int ot = 0;
    const int rc = check_norm_rope(q, k, v, q_norm, k_norm, positions, params, q_out, k_out, v_out, rows, &a, &ot);
    if (rc != MXFA_OK) return rc;
    hipStream_t stream = (hipStream_t)hip_stream;
    const hipError_t e =
        timed_launch("qk_norm_rope", stream, [&] { return launch_qk_norm_rope(a, ot, stream); });
    if (e != hipSuccess) return fail(MXFA_ERR_HIP, "qk_norm_rope launch: %s", hipGetErrorString(e));
    return MXFA_OK;
}

int mxfa_qk_norm_rope_supports(const mxfa_tensor *q, const mxfa_tensor *k, const mxfa_tensor *v,
                               const mxfa_tensor *q_norm, const mxfa_tensor *k_norm, const mxfa_tensor *positions,
                               const mxfa_norm_rope_params *params, const mxfa_tensor *q_out,
                               const mxfa_tensor *k_out, const mxfa_tensor *v_out, const mxfa_tensor *rows) {
    return check_norm_rope(q, k, v, q_norm, k_norm, positions, params, q_out, k_out, v_out, rows, nullptr,
                           nullptr) == MXFA_OK
               ? 1
               : 0;
}

int mxfa_set_rows_supports(const mxfa_tensor *dst, const mxfa_tensor *src, const mxfa_tensor *rows) {
    return check_set_rows(dst, src, rows, nullptr) == MXFA_OK ? 1 : 0;
}

int mxfa_set_rows(mxfa_tensor *dst, const mxfa_tensor *src, const mxfa_tensor *rows, void *hip_stream) {
    SetRowsArgs a;
    const int rc = check_set_rows(dst, src, rows, &a);
    if (rc != MXFA_OK) return rc;
    if (a.n_rows == 0) return MXFA_OK;
    hipStream_t stream = (hipStream_t)hip_stream;
    const hipError_t e = timed_launch("set_rows", stream, [&] { return launch_set_rows(a, dst->type, stream); });
    if (e != hipSuccess) return fail(MXFA_ERR_HIP, "set_rows launch: %s", hipGetErrorString(e));
    return MXFA_OK;
}

void mxfa_release(void) {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    int cur = 0;
    const bool have_cur = hipGetDevice(&cur) == hipSuccess;
    for (Workspace &w : g_ws) {
        if (hipSetDevice(w.device) != hipSuccess) continue;
        (void)hipDeviceSynchronize();
        if (w.ptr) (void)hipFree(w.ptr);
        if (w.tickets) (void)hipFree(w.tickets);
        if (w.arena) (void)hipFree(w.arena);
        for (void *p : w.retired) (void)hipFree(p);
    }
    g_ws.clear();
    if (have_cur) (void)hipSetDevice(cur);
}

int mxfa_workspace_info(int64_t *live_bytes, int64_t *retired_buffers) {
    if (!live_bytes || !retired_buffers) return fail(MXFA_ERR_INVALID, "NULL argument");
    std::lock_guard<std::mutex> lock(g_ws_mu);
    int64_t live = 0, ret = 0;
    for (const Workspace &w : g_ws) {
        live += (int64_t)w.size + w.n_tickets * (int64_t)sizeof(int) + (int64_t)w.arena_size;
        ret += (int64_t)w.retired.size();
    }
    *live_bytes = live;
    *retired_buffers = ret;
    return MXFA_OK;
}

const char *mxfa_status_string(int status) {
    switch (status) {
        case MXFA_OK: return "ok";
        case MXFA_ERR_INVALID: return "invalid argument";
        case MXFA_ERR_UNSUPPORTED: return "unsupported";
        case MXFA_ERR_HIP: return "HIP error";
        case MXFA_ERR_NOMEM: return "out of device memory";
        default: return "unknown status";
    }
}

const char *mxfa_last_error(void) { return g_last_error.c_str(); }

void mxfa_timing_enable(int on) { g_timing.store(on < 0 ? 0 : std::min(on, 1000)); }

int mxfa_timing_read(const char *kernel, double *total_ms, int64_t *launches) {
    if (!kernel || !total_ms || !launches) return fail(MXFA_ERR_INVALID, "NULL argument");
    std::lock_guard<std::mutex> lock(g_timing_mu);
    drain_pending();
    const FamilyStats &st = stats_of(kernel);
    *total_ms = st.ms;
    *launches = st.launches;
    return MXFA_OK;
}

void mxfa_timing_reset(void) {
    std::lock_guard<std::mutex> lock(g_timing_mu);
    drain_pending();
    g_stats.clear();
}

int mxfa_version(void) { return 100; }

}  // extern "C"
