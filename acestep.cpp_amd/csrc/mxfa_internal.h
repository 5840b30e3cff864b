// mxfa_internal.h -- launchers shared between the kernel translation units
// and the host API (mxfa_api.cpp).  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>

#include "mxfa_common.h"

namespace mxfa {

// Split-KV decode kernel, F16/BF16/Q8_0 K/V.  With a.n_splits > 1 it needs
// a.part_o / a.part_ml and a.tickets (B*Nkv*row_tiles ints, zero on entry;
// left zero on exit).
hipError_t launch_fa_decode(const FaArgs &a, int ktype, hipStream_t stream);

// Zero-fills n ints (ticket buffer set-up).
hipError_t launch_fill_zero(int *p, int64_t n, hipStream_t stream);

// MFMA prefill kernel geometry.
constexpr int kPfBM = 128;   // query rows per workgroup (4 waves x 32)
constexpr int kPfBN = 64;    // keys per K/V tile

// Mask tile classifier: writes a.tile_class[plane][qt][kt] (row stride
// a.n_kt_pad bytes) for every (mask plane, kPfBM-query tile, kPfBN-key
// tile): 0 = all -inf, 1 = all zero, 2 = anything else, 3 = a mix of 0 and
// -inf only (with a.tile_bits set): then the tile's liveness goes to
// a.tile_bits[((plane * n_qt + qt) * n_kt + kt) * kPfBM + row], bit k for key
// k of the tile (keys past Skv: 0).
constexpr int kPfMaxKeyTiles = 512;   // class rows held in two registers per lane
hipError_t launch_mask_classify(const FaArgs &a, int n_planes, uint8_t *classes, hipStream_t stream);

// MFMA prefill / DiT kernel.  ktype: T_F16/T_BF16, or T_Q8_0 for K/V
// staged in F16 by launch_q8_stage (Q, F32, quantised to Q8_0 on load).
hipError_t launch_fa_prefill(const FaArgs &a, int ktype, hipStream_t stream);

// MFMA prefill with 48 queries per wave (fa_wide.hip): kPfWideBM-query
// workgroups over a.n_qt_w tiles; F16 K/V, no softcap, dense mask or none
// (tile classes as for launch_fa_prefill, over kPfBM-query tiles).
constexpr int kPfWideBM = 192;   // query rows per workgroup (4 waves x 48)
hipError_t launch_fa_wide(const FaArgs &a, int ktype, hipStream_t stream);

// F16 staging of a prefill over a Q8_0 cache (q8_stage.hip): the Q8_0 K/V
// rows, dequantised, into contiguous [128, Skv, Nkv, Bk] F16 buffers (the
// prefill kernel quantises Q itself: launch_fa_prefill with T_Q8_0).  K and
// V have the same shape, rows 4-byte aligned; 32 n_kv < 2^31.
struct Q8StageArgs {
    const char *k, *v;
    int64_t k_nb1, k_nb2, k_nb3, v_nb1, v_nb2, v_nb3;
    char *ks, *vs;
    uint32_t Skv, Nkv;
    uint32_t n_kv;   // K rows = V rows (Skv Nkv Bk)
};
hipError_t launch_q8_stage(const Q8StageArgs &a, hipStream_t stream);

// KV-cache write (GGML_OP_SET_ROWS, F32 source).  Source row r of the
// flattened [ne01, ne02, ne03] row space goes to destination row
// rows[r % ne01, i02 % r_ne1, i03 % r_ne2] of plane (i02, i03).
struct SetRowsArgs {
    const char *src;            // F32 rows
    const char *rows;           // I64 (rows_i64) or I32 row ids
    char *dst;                  // destination rows (dst_ne1 per plane)
    uint32_t cpr;               // 4-value chunks per row (ne0 / 4)
    uint32_t ne01, ne02, n_rows;                // n_rows = ne01*ne02*ne03 (< 2^31 chunks total)
    uint32_t r_ne1, r_ne2;                      // row-id broadcast extents
    int64_t s_nb1, s_nb2, s_nb3;                // source strides (bytes)
    int64_t r_nb0, r_nb1, r_nb2;                // row-id strides
    int64_t d_nb1, d_nb2, d_nb3, dst_ne1;       // destination strides, rows per plane
    int rows_i64;
};

// ne0 % 4 == 0 (F32/F16/BF16) or ne0 % 32 == 0 (Q8_0); source rows 16-byte
// aligned, F16/BF16 destination rows 8-byte aligned, F32 16-byte, Q8_0 2-byte;
// n_rows * cpr < 2^31.
hipError_t launch_set_rows(const SetRowsArgs &a, int dtype, hipStream_t stream);

// Pre-attention fusion (QK-RMSNorm, NEOX RoPE, 16-bit cast, KV-cache
// write); see qk_norm_rope.hip.  Q/K/V rows are F32 [128, H, S | Skv, B]
// with strides {head, token, batch}; Q goes to [128, Nh, S, B] contiguous,
// K/V to row rows[s, b % r_ne1] (or s) of their [128, kv_rows, Nkv, B]
// views.  rope == 0: no rotation (pos unused) and K/V may have Skv != S
// tokens (cross-attention); with RoPE, Skv == S.
struct NormRopeArgs {
    const char *q, *k, *v;
    int64_t q_nb[3], k_nb[3], v_nb[3];
    const float *q_w, *k_w;
    const int32_t *pos;
    int32_t pos_per_batch;
    float eps, theta_scale;
    int32_t clamp_v;
    char *q_out, *k_out, *v_out;
    int64_t kv_nb1, kv_nb2, kv_nb3, kv_rows;
    const char *rows;
    int64_t r_nb0, r_nb1;
    int32_t r_ne1, rows_i64;
    int32_t Nh, Nkv, S, B;
    int32_t Skv, rope;
};
hipError_t launch_qk_norm_rope(const NormRopeArgs &a, int out_type, hipStream_t stream);

// Per-kernel timing: with timing mode n > 0, timed_launch() runs `launch`
// n times back to back (every launch of the engine is idempotent: it
// rewrites its outputs from its inputs) between two events on `stream`, and
// files the pair under `family` as n launches.
int timing_mode();
void timing_begin(const char *family, hipStream_t stream, void **token);
void timing_end(void *token, hipStream_t stream, int launches);

template <typename F>
hipError_t timed_launch(const char *family, hipStream_t stream, F launch) {
    const int n = timing_mode();
    if (n <= 0) return launch();
    void *tok = nullptr;
    timing_begin(family, stream, &tok);
    hipError_t e = launch();
    int done = 1;
    for (; done < n && e == hipSuccess; done++) e = launch();
    timing_end(tok, stream, done);
    return e;
}

}  // namespace mxfa
