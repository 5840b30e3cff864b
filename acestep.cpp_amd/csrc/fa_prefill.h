// fa_prefill.h -- pieces shared by the two MFMA prefill kernels
// (fa_mfma.hip: 32 queries per wave; fa_wide.hip: 48 queries per wave):
// LDS tile geometry, the XCD-aware job order, tile classes held in
// registers, and cross-lane pair reductions.
#pragma once

#include "mxfa_common.h"
#include "mxfa_internal.h"

namespace mxfa {

constexpr int kTileBytes = 16384;            // K or V rows of one 64-key tile
constexpr int kStageBytes = 2 * kTileBytes;  // K + V
constexpr int kPfLds = 2 * kStageBytes;      // double buffered: 64 KB
constexpr uint32_t kXcds = 8;                // MI355X: workgroups go round-robin to 8 XCDs
constexpr uint32_t kCusPerXcd = 32;          // 256 CUs

// Job of this workgroup among n_qt * Nh * B (query tile, q head, batch)
// jobs.  Workgroup ids go round-robin to the XCDs; each XCD gets a
// contiguous block of the job list, which is ordered by (batch, kv head),
// then by query tile from the last (longest under a causal mask) down, then
// by q head within the GQA group: the q tiles that share K/V rows run on one
// XCD and share its L2.  Within an XCD the order snakes over rounds of
// kCusPerXcd: the XCD's dispatcher gives each CU one workgroup per round, so
// odd rounds run reversed and a CU pairs a long causal tile with a short
// one.  `second`: the workgroup is the CU's second of the first pair (every
// CU of the XCD holds a pair).
__device__ __forceinline__ void pf_job(const FaArgs &a, int n_qt, int &qt, int &head, int &b, bool &second) {
    const uint32_t L = __builtin_amdgcn_workgroup_id_x();
    const uint32_t N = (uint32_t)(n_qt * a.Nh * a.B);
    const uint32_t nq = N / kXcds, nr = N % kXcds, x = L % kXcds, s0 = L / kXcds;
    const uint32_t n_x = x < nr ? nq + 1 : nq;
    const uint32_t rnd = s0 / kCusPerXcd, w = s0 % kCusPerXcd;
    const uint32_t cnt = min(kCusPerXcd, n_x - rnd * kCusPerXcd);
    const uint32_t s = (rnd & 1) ? rnd * kCusPerXcd + (cnt - 1 - w) : s0;
    const uint32_t J = x < nr ? x * (nq + 1) + s : nr * (nq + 1) + (x - nr) * nq + s;
    const uint32_t per_u = (uint32_t)(a.G * n_qt);
    const uint32_t u = J / per_u, r = J % per_u;
    qt = __builtin_amdgcn_readfirstlane(n_qt - 1 - (int)(r / (uint32_t)a.G));
    b = __builtin_amdgcn_readfirstlane((int)(u / (uint32_t)a.Nkv));
    head = __builtin_amdgcn_readfirstlane((int)(u % (uint32_t)a.Nkv) * a.G + (int)(r % (uint32_t)a.G));
    second = rnd == 1 && n_x >= 2 * kCusPerXcd;
}

// Tile classes of one (plane, query tile) row live in registers: lane l
// holds the class bytes of key tiles 4l..4l+3 (w0: tiles < 256, w1: tiles
// 256..511), read with v_readlane (uniform, no memory wait in the loop).
struct TileClasses {
    uint32_t w0, w1;
    bool present;
    __device__ __forceinline__ int at(int kt) const {
        if (!present) return 1;
        const uint32_t w = kt < 256 ? __builtin_amdgcn_readlane(w0, (kt >> 2) & 63)
                                    : __builtin_amdgcn_readlane(w1, ((kt - 256) >> 2) & 63);
        return (int)((w >> (8 * (kt & 3))) & 0xFFu);
    }
    // (readfirstlane: the result is wave-uniform, and the compiler must
    // know it to keep the tile loop on scalar branches)
    __device__ __forceinline__ int next_live(int kt, int n) const {
        if (!present) return kt;
        while (kt < n && at(kt) == 0) kt++;
        return __builtin_amdgcn_readfirstlane(kt);
    }
};

// Class bytes (0 all -inf, 1 all zero, 2 mixed) of the union of two row
// ranges' tiles, four at a time: equal classes stand, different ones make
// the tile mixed.
__device__ __forceinline__ uint32_t class_union4(uint32_t x, uint32_t y) {
    const uint32_t d = x ^ y;
    const uint32_t nz = (((d & 0x7F7F7F7Fu) + 0x7F7F7F7Fu) | d) & 0x80808080u;   // bit 7: byte differs
    const uint32_t m = (nz >> 7) * 0xFFu;
    return (x & ~m) | (0x02020202u & m);
}

// Max / sum of a lane's value and the same register of lane l ^ 32 (one
// v_permlane32_swap) or l ^ 16 (v_permlane16_swap).
__device__ __forceinline__ float max_pair32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                    false, false);
    return fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}
__device__ __forceinline__ float sum_pair32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                    false, false);
    return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}
__device__ __forceinline__ float sum_pair16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                    false, false);
    return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}

}  // namespace mxfa
