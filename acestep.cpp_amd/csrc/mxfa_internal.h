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
// tile): 0 = all -inf, 1 = all zero, 2 = anything else.
constexpr int kPfMaxKeyTiles = 512;   // class rows held in two registers per lane
hipError_t launch_mask_classify(const FaArgs &a, int n_planes, uint8_t *classes, hipStream_t stream);

// MFMA prefill / DiT kernel.  ktype: T_F16/T_BF16.
hipError_t launch_fa_prefill(const FaArgs &a, int ktype, hipStream_t stream);

// Per-kernel timing: when enabled, timed_launch() brackets `launch` with
// two events on `stream` and files them under `family`.
bool timing_enabled();
void timing_begin(const char *family, hipStream_t stream, void **token);
void timing_end(void *token, hipStream_t stream);

template <typename F>
hipError_t timed_launch(const char *family, hipStream_t stream, F launch) {
    if (!timing_enabled()) return launch();
    void *tok = nullptr;
    timing_begin(family, stream, &tok);
    const hipError_t e = launch();
    timing_end(tok, stream);
    return e;
}

}  // namespace mxfa
