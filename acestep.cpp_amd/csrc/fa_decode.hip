// fa_decode.hip -- split-KV flash attention for gfx950: decode and short
// query runs, over F16, BF16 or Q8_0 K/V.
//
// Serves the decode call sites of the reference: single-sequence decode
// (src/qwen3-lm.h:465, n_tokens = 1) and batched CFG decode
// (src/qwen3-lm.h:789-794, q [D,1,Nh,N] against a 4D KV-cache view with a
// per-sequence padding mask built at :872-883), the Q8_0 KV cache, and any
// shape the MFMA prefill kernel does not take.  The op is HBM-bound: the
// design is about keeping K/V bytes in flight and reading each byte once.
//
// Work decomposition.  One workgroup = 4 waves = one (batch b, KV head,
// 16-row tile, KV split).  A row is one (query, q head) pair; the G = Nh/Nkv
// q heads of a KV head (and the Sq queries) are packed as MFMA columns, so
// each K/V byte streamed from HBM serves all of them (GQA reuse).
//
//  1. Live range.  The workgroup scans the mask rows of its 16 rows over
//     its split and clips the split to [first live key, last live key]:
//     keys past a sequence's length (the reference pads the window to 256
//     keys and masks the tail, qwen3-lm.h:496-500, :875-881) are never
//     read, and splits that lie wholly past it exit at once.  Holes inside
//     the range are handled per element.
//  2. Streaming, two kernels:
//     fa_decode_lds_kernel (F16/BF16 with a vector-readable mask or none):
//       each wave owns a ring of NST stages in LDS, one 16-key block per
//       stage (K 4 KB, V 4 KB, the tile's mask 512 B), filled by HBM->LDS
//       DMA (global_load_lds) NST-1 blocks ahead of the block being
//       computed, with explicit vmcnt waits; no K/V byte passes through
//       VGPRs.  The first stages are issued before the live-range scan
//       returns (they are right whenever the range starts at the split
//       start, as it does for every live split of a padding mask).
//       S^T = K . Q^T with v_mfma_f32_16x16x32_{f16,bf16} (K rows from
//       LDS, XOR-swizzled); O^T += V^T . P^T with
//       v_mfma_f32_16x16x16_{f16,bf16}, V^T read with the gfx950 LDS
//       transpose read (ds_read_b64_tr_b16) from the row-major V stage.
//     fa_decode_reg_kernel (Q8_0, or a mask that is not 8-byte aligned):
//       each wave keeps two 32-key blocks in registers (block n+1 loading
//       while block n is computed).  Q8_0: Q is quantised to Q8_0 in the
//       prologue exactly as ggml quantises it; S^T uses
//       v_mfma_i32_16x16x32_i8, one MFMA per 32-value block, exact int32
//       block sums scaled by d_k * d_q; V is dequantised to f16 and staged
//       transposed into a per-wave LDS tile for the 16-bit MFMA.
//     Both: online softmax in fp32 registers (exp2 domain).
//  3. The 4 waves merge (m, l, O) through LDS.  One split: the workgroup
//     writes the normalised output.  Several: it writes an unnormalised
//     partial plus (m, l), and the last workgroup of the tile to finish (a
//     device-scope ticket counter, reset by that workgroup) merges the
//     splits with a log-sum-exp reduction -- no second launch.
//
// Masked keys never contribute: a score whose mask entry is -inf is
// replaced by -inf (not added to), and V values of keys dead for every row
// of the tile are zeroed before the PV product, so non-finite data in
// masked cache slots cannot leak into the output (ggml's CPU kernel skips
// such keys entirely, ggml-cpu/ops.cpp flash_attn_ext_f16_one_chunk).

#include <type_traits>

#include "mxfa_common.h"
#include "mxfa_internal.h"
#include "once_per_device.h"

namespace mxfa {

constexpr int kDecWaves = 4;
constexpr int kVtStride = 36;  // halfs per V^T row of the register kernel: 32 keys + 4 pad

// Mask access modes (template argument MM).
constexpr int kMaskNone = 0;     // no mask
constexpr int kMaskVec = 1;      // 8-byte aligned rows of >= round_up(Skv, 4) entries (LDS
                                 // kernel: and >= 16)
constexpr int kMaskScalar = 2;   // anything else
constexpr int kMaskStruct = 3;   // structured mask (a.sm_*): no mask reads

// Per-lane coordinates of a decode workgroup.
struct Tile {
    int tid, lane, wave, c16, g16;
    int split, kvh, rt, b, bk;
    int r;          // row owned as MFMA column c16
    bool row_ok;
    int iq1, head;
};

// Splits of the (batch b, row tile rt) streams under a structured mask:
// a.chunk keys each from the first key any row of the tile sees to the last
// one (at least one split, which writes zeros when nothing is live).
__device__ __forceinline__ void sm_tile_keys(const FaArgs &a, int b, int rt, int &lo, int &len) {
    const int r0 = rt * 16, nr = min(16, a.M - r0);
    int lo_f, hi_f, lo_l, hi_l;
    sm_row_range(a, b, r0 / a.G, lo_f, hi_f);
    sm_row_range(a, b, (r0 + nr - 1) / a.G, lo_l, hi_l);
    lo = lo_f;
    len = max(0, hi_l - lo_f);
}
__device__ __forceinline__ int sm_tile_splits(const FaArgs &a, int len) { return max(1, (len + a.chunk - 1) / a.chunk); }

template <int MM>
__device__ __forceinline__ Tile make_tile(const FaArgs &a) {
    Tile t;
    t.tid = threadIdx.x;
    t.lane = t.tid & 63;
    t.wave = __builtin_amdgcn_readfirstlane(t.tid >> 6);   // wave-uniform
    t.c16 = t.lane & 15;
    t.g16 = t.lane >> 4;
    if (MM == kMaskStruct && a.dec_live > 0) {
        // Live-split list (host lengths): workgroup i = j * Nkv + kv head,
        // j running over the splits of (b, rt) in order, so that every
        // workgroup streams live keys and none waits behind dead ones.
        const int i = (int)blockIdx.x;
        t.kvh = i % a.Nkv;
        int j = i / a.Nkv, b = 0, rt = 0;
        for (;;) {
            int lo, len;
            sm_tile_keys(a, b, rt, lo, len);
            const int ns = sm_tile_splits(a, len);
            if (j < ns || (b == a.B - 1 && rt == a.row_tiles - 1)) break;
            j -= ns;
            if (++rt == a.row_tiles) { rt = 0; b++; }
        }
        t.split = __builtin_amdgcn_readfirstlane(j);
        t.rt = __builtin_amdgcn_readfirstlane(rt);
        t.b = __builtin_amdgcn_readfirstlane(b);
    } else if (a.dec_pair > 0) {
        // Paired splits (two workgroups per CU): the grid's first half is
        // dispatched one workgroup per CU and runs ahead of the second half
        // (its waves are older), so every stream takes its even splits from
        // the first half and its odd splits from the second, and the even
        // split of each pair streams a.dec_pair keys, more than half.  The
        // second half starts ~1 us late (s_sleep 32: 32 x 64 clocks), so
        // that the two halves' first loads do not share one burst
        // (measured: C5 27.0 -> 26.3 us, C3 39.8 -> 39.3 us).
        const int L = (int)(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z));
        const int half = (int)(gridDim.x * gridDim.y * gridDim.z) / 2, hs = (int)gridDim.x / 2;
        const bool first = L < half;
        if (!first) __builtin_amdgcn_s_sleep(32);
        const int Lh = first ? L : L - half;
        const int stream = Lh / hs;
        t.split = __builtin_amdgcn_readfirstlane(2 * (Lh % hs) + (first ? 0 : 1));
        t.kvh = __builtin_amdgcn_readfirstlane((stream % (int)gridDim.y) / a.row_tiles);
        t.rt = __builtin_amdgcn_readfirstlane((stream % (int)gridDim.y) % a.row_tiles);
        t.b = __builtin_amdgcn_readfirstlane(stream / (int)gridDim.y);
    } else {
        t.split = blockIdx.x;
        t.kvh = blockIdx.y / a.row_tiles;
        t.rt = blockIdx.y % a.row_tiles;
        t.b = blockIdx.z;
    }
    t.bk = t.b / a.rk3;
    t.r = t.rt * 16 + t.c16;
    t.row_ok = t.r < a.M;
    t.iq1 = t.row_ok ? t.r / a.G : 0;
    t.head = t.kvh * a.G + (t.row_ok ? t.r % a.G : 0);
    return t;
}

// Key range [k0, k1) of this workgroup's split, and the number of splits
// `ns` of its (batch, kv head, row tile) stream.  Dense masks: splits of
// a.chunk keys from 0 (a.n_splits of them).  Structured masks: splits of
// a.chunk keys from the first key any row of the tile sees, up to the last
// one (the host sized a.chunk from the live lengths, so splits carry equal
// work).  With host lengths the grid lists exactly those splits
// (a.dec_live); with device lengths it is the dense grid and workgroups
// past their stream's last split do nothing (skip).
struct SplitRange {
    int k0, k1, ns;
    bool skip;
};
template <int MM>
__device__ __forceinline__ SplitRange split_range(const FaArgs &a, const Tile &t) {
    SplitRange sr;
    if constexpr (MM == kMaskStruct) {
        int lo, len;
        sm_tile_keys(a, t.b, t.rt, lo, len);
        sr.ns = sm_tile_splits(a, len);
        sr.skip = t.split >= sr.ns;
        sr.k0 = len ? lo + t.split * a.chunk : 0;
        sr.k1 = len ? min(lo + len, sr.k0 + a.chunk) : 0;
    } else if (a.dec_pair > 0) {
        // pair p = keys [2p chunk, (2p + 2) chunk): a.dec_pair for the even
        // split, the rest for the odd one
        sr.ns = a.n_splits;
        sr.skip = false;
        const int base = (t.split >> 1) * 2 * a.chunk;
        sr.k0 = min(a.Skv, base + ((t.split & 1) ? a.dec_pair : 0));
        sr.k1 = min(a.Skv, (t.split & 1) ? base + 2 * a.chunk : base + a.dec_pair);
    } else {
        sr.ns = a.n_splits;
        sr.skip = false;
        sr.k0 = t.split * a.chunk;
        sr.k1 = min(a.Skv, sr.k0 + a.chunk);
    }
    return sr;
}

__device__ __forceinline__ const float *q_row(const FaArgs &a, const Tile &t) {
    return (const float *)(a.q + (int64_t)t.iq1 * a.q_nb1 + (int64_t)t.head * a.q_nb2 + (int64_t)t.b * a.q_nb3);
}

// Q^T operand of the 16x16x32 MFMA: lane holds Q[row][32s + 8*g16 + e],
// converted like ggml converts Q to K's vec-dot type (round to nearest even),
// or loaded as it is when Q is already stored in that type (a.q16).
// Q as Q8_0 (ggml quantize_row_q8_0: d = fp16(amax/127), q = rint(x*127/amax)
// per 32-value block), laid out as the B operand of the i8 MFMA.
// Q of the register kernel in two halves: q_issue loads the lane's raw Q
// (F32, or 16-bit when a.q16), q_convert turns it into the MFMA operands
// (the 16-bit type of the PV product, or Q8_0 as ggml quantises Q for a
// Q8_0 K).  Between them the kernel issues its first K/V loads, so Q's
// conversion waits for Q's own loads alone.
struct QRaw {
    f32x4 x[8];
};
__device__ __forceinline__ QRaw q_issue(const FaArgs &a, const Tile &t) {
    QRaw r;
#pragma unroll
    for (int i = 0; i < 8; i++) r.x[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (!t.row_ok) return r;
    if (a.q16) {
        const uint16_t *qh = (const uint16_t *)(a.q + (int64_t)t.iq1 * a.q_nb1 + (int64_t)t.head * a.q_nb2 +
                                                (int64_t)t.b * a.q_nb3);
#pragma unroll
        for (int s = 0; s < 4; s++) r.x[2 * s] = __builtin_bit_cast(f32x4, *(const u16x8 *)(qh + 32 * s + 8 * t.g16));
    } else {
        const float *qp = q_row(a, t);
#pragma unroll
        for (int s = 0; s < 4; s++) {
            r.x[2 * s] = *(const f32x4 *)(qp + 32 * s + 8 * t.g16);
            r.x[2 * s + 1] = *(const f32x4 *)(qp + 32 * s + 8 * t.g16 + 4);
        }
    }
    return r;
}
template <int T>
__device__ __forceinline__ void q_convert16(const FaArgs &a, const QRaw &r, typename Mfma16<T>::v8 (&qb)[4]) {
#pragma unroll
    for (int s = 0; s < 4; s++)
        qb[s] = a.q16 ? __builtin_bit_cast(typename Mfma16<T>::v8, r.x[2 * s])
                      : __builtin_bit_cast(typename Mfma16<T>::v8, cvt8<T>(r.x[2 * s], r.x[2 * s + 1]));
}
__device__ __forceinline__ void q_convert8(const QRaw &r, long (&qq)[4], float (&dq)[4]) {
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const f32x4 x0 = r.x[2 * s], x1 = r.x[2 * s + 1];
        float amax = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; e++) amax = fmaxf(amax, fmaxf(fabsf(x0[e]), fabsf(x1[e])));
        amax = fmaxf(amax, __shfl_xor(amax, 16));
        amax = fmaxf(amax, __shfl_xor(amax, 32));
        dq[s] = (float)(_Float16)(amax / 127.0f);
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        uint32_t w0 = 0u, w1 = 0u;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            w0 |= ((uint32_t)(int)__builtin_rintf(x0[e] * id) & 0xFFu) << (8 * e);
            w1 |= ((uint32_t)(int)__builtin_rintf(x1[e] * id) & 0xFFu) << (8 * e);
        }
        qq[s] = (long)(((uint64_t)w1 << 32) | w0);
    }
}

__device__ __forceinline__ const uint16_t *mask_row(const FaArgs &a, int iq1, int head, int b) {
    return (const uint16_t *)(a.mask + (int64_t)iq1 * a.m_nb1 + (int64_t)(head % a.m_ne2) * a.m_nb2 +
                              (int64_t)(b % a.m_ne3) * a.m_nb3);
}

// Live key range [lo, hi) of [k0, k1) over the mask rows of the tile's
// rows (empty when nothing is live).  Called by the whole workgroup.
// Workgroup-wide [first, last] of the per-thread live ranges -> [lo, hi).
__device__ void range_reduce(const Tile &t, int first, int last, int *range_lds, int &lo, int &hi) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        first = min(first, __shfl_xor(first, off));
        last = max(last, __shfl_xor(last, off));
    }
    if (t.lane == 0) {
        range_lds[t.wave] = first;
        range_lds[kDecWaves + t.wave] = last;
    }
    __syncthreads();
    first = INT32_MAX;
    last = -1;
#pragma unroll
    for (int w = 0; w < kDecWaves; w++) {
        first = min(first, range_lds[w]);
        last = max(last, range_lds[kDecWaves + w]);
    }
    lo = first;
    hi = last + 1;
}

// Mask rows scanned for a tile: the tile's queries (one row each when the
// mask has one head plane) or its rows.
struct ScanRows {
    int q_first, r0, n_scan;
};
__device__ __forceinline__ ScanRows scan_rows(const FaArgs &a, const Tile &t) {
    ScanRows sr;
    sr.r0 = t.rt * 16;
    const int nr = min(16, a.M - sr.r0);
    sr.q_first = sr.r0 / a.G;
    const int q_last = (sr.r0 + nr - 1) / a.G;
    sr.n_scan = a.m_ne2 == 1 ? q_last - sr.q_first + 1 : nr;
    return sr;
}
__device__ __forceinline__ const uint16_t *scan_row(const FaArgs &a, const Tile &t, const ScanRows &sr, int si) {
    const int sq1 = a.m_ne2 == 1 ? sr.q_first + si : (sr.r0 + si) / a.G;
    const int sh = a.m_ne2 == 1 ? 0 : t.kvh * a.G + (sr.r0 + si) % a.G;
    return mask_row(a, sq1, sh, t.b);
}

// Live range [lo, hi) of keys in [k0, k1) under a dense mask: keys whose
// entry is -inf in every scanned row are dead.
__device__ void live_range(const FaArgs &a, const Tile &t, int k0, int k1, int *range_lds, int &lo, int &hi) {
    const ScanRows sr = scan_rows(a, t);
    const int n8 = (k1 - k0 + 7) >> 3;
    int first = INT32_MAX, last = -1;
    for (int it = t.tid; it < sr.n_scan * n8; it += 256) {
        const int si = it / n8, k8 = k0 + 8 * (it - si * n8);
        const uint16_t *row = scan_row(a, t, sr, si);
        uint32_t livebits = 0;
        if (a.mask_al16 && k8 + 8 <= k1) {
            const u16x8 mv = *(const u16x8 *)(row + k8);
#pragma unroll
            for (int e = 0; e < 8; e++) livebits |= (mv[e] != 0xFC00u ? 1u : 0u) << e;
        } else {
            for (int e = 0; e < 8 && k8 + e < k1; e++) livebits |= (row[k8 + e] != 0xFC00u ? 1u : 0u) << e;
        }
        if (livebits) {
            first = min(first, k8 + __builtin_ctz(livebits));
            last = max(last, k8 + 31 - __builtin_clz(livebits));
        }
    }
    range_reduce(t, first, last, range_lds, lo, hi);
}

// The same scan in two halves, so that its loads go out ahead of a
// kernel's first K/V loads and the reduction waits for them alone:
// scan_issue loads each thread's 8-key group when one aligned 16-byte load
// per thread covers the scan (16-byte aligned rows, k1 - k0 a multiple of
// 8, at most 256 groups); otherwise scan_finish runs live_range.
struct ScanPre {
    u16x8 mv;
    int k8;
    bool one;
};
__device__ __forceinline__ ScanPre scan_issue(const FaArgs &a, const Tile &t, int k0, int k1) {
    ScanPre p;
    p.mv = u16x8{0xFC00u, 0xFC00u, 0xFC00u, 0xFC00u, 0xFC00u, 0xFC00u, 0xFC00u, 0xFC00u};
    p.k8 = 0;
    const ScanRows sr = scan_rows(a, t);
    const int n8 = (k1 - k0) >> 3;
    p.one = a.mask_al16 && ((k1 - k0) & 7) == 0 && sr.n_scan * n8 <= 256;   // uniform
    if (p.one && t.tid < sr.n_scan * n8) {
        const int si = t.tid / n8;
        p.k8 = k0 + 8 * (t.tid - si * n8);
        p.mv = *(const u16x8 *)(scan_row(a, t, sr, si) + p.k8);
    }
    return p;
}
__device__ __forceinline__ void scan_finish(const FaArgs &a, const Tile &t, const ScanPre &p, int k0, int k1,
                                            int *range_lds, int &lo, int &hi) {
    if (!p.one) {
        live_range(a, t, k0, k1, range_lds, lo, hi);
        return;
    }
    uint32_t livebits = 0;
#pragma unroll
    for (int e = 0; e < 8; e++) livebits |= (p.mv[e] != 0xFC00u ? 1u : 0u) << e;
    const int first = livebits ? p.k8 + __builtin_ctz(livebits) : INT32_MAX;
    const int last = livebits ? p.k8 + 31 - __builtin_clz(livebits) : -1;
    range_reduce(t, first, last, range_lds, lo, hi);
}

// 16 bytes stored at agent scope: global_store_dwordx4 with sc1, the
// encoding a relaxed agent-scope atomic store of each element gets on this
// architecture (written through past the XCD's L2), in one transaction
// instead of four.  Complete at device scope once vmcnt drains.
__device__ __forceinline__ void st_agent16(float *p, f32x4 v) {
    asm volatile("global_store_dwordx4 %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}

__device__ __forceinline__ float ld_dev(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Log-sum-exp merge of the ns partials of the tile's nr rows (run by the
// last workgroup of the tile; partial row pr0 + r, partial slots a.n_splits
// apart).  Thread -> dim t.tid % 128 of rows t.tid / 128 + 2j.  The O
// partials of the first two rows of a thread (every row when nr <= 4, as in
// decode) are loaded up front together with every (m, l) pair, so the merge
// waits for one memory round trip; phase A turns (m, l) into weights in
// LDS, phase B accumulates in split order (larger nr / ns load the rest in
// batches of 16).
constexpr int kMaxSplits = 64;
__device__ void merge_splits(const FaArgs &a, const Tile &t, int64_t pr0, int nr, int ns, float *lds) {
    const int stride = a.n_splits;           // partial slots per row
    float *wm = lds;                         // [16][kMaxSplits]: m, then weights
    float *wl = wm + 16 * kMaxSplits;        // [16][kMaxSplits]: l
    float *Linv = wl + 16 * kMaxSplits;      // [16]
    const int d = t.tid & (kD - 1);
    const int rA = t.tid >> 7, rB = rA + 2;
    // The first 16 partials of rows rA and rB and the first 1024 (m, l)
    // pairs go out together: one memory round trip.  (The workgroup's LDS
    // is free here: its own merge data was read before the ticket's
    // barriers, and a barrier would also wait for these loads.)
    float pa[16], pb[16];
    float mv0[4], lv0[4];
    {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = t.tid + 256 * u;
            const int r = i / ns, sp = i - r * ns;
            const float *pm = a.part_ml + ((pr0 + r) * stride + sp) * 2;
            mv0[u] = i < nr * ns ? ld_dev(pm) : 0.0f;
            lv0[u] = i < nr * ns ? ld_dev(pm + 1) : 0.0f;
        }
        const float *poA = a.part_o + (pr0 + rA) * stride * kD + d;
        const float *poB = a.part_o + (pr0 + rB) * stride * kD + d;
#pragma unroll
        for (int u = 0; u < 16; u++) {
            pa[u] = (rA < nr && u < ns) ? ld_dev(poA + (int64_t)u * kD) : 0.0f;
            pb[u] = (rB < nr && u < ns) ? ld_dev(poB + (int64_t)u * kD) : 0.0f;
        }
    }
    for (int i0 = 0; i0 < nr * ns; i0 += 256 * 4) {
        float mv[4], lv[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = i0 + t.tid + 256 * u;
            const int r = i / ns, sp = i - r * ns;
            const float *pm = a.part_ml + ((pr0 + r) * stride + sp) * 2;
            mv[u] = i0 == 0 ? mv0[u] : (i < nr * ns ? ld_dev(pm) : 0.0f);
            lv[u] = i0 == 0 ? lv0[u] : (i < nr * ns ? ld_dev(pm + 1) : 0.0f);
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = i0 + t.tid + 256 * u;
            if (i < nr * ns) {
                const int r = i / ns, sp = i - r * ns;
                wm[r * kMaxSplits + sp] = mv[u];
                wl[r * kMaxSplits + sp] = lv[u];
            }
        }
    }
    __syncthreads();
    if (t.tid < nr) {
        const int r = t.tid;
        float ms_all = -INFINITY;
        for (int sp = 0; sp < ns; sp++) ms_all = fmaxf(ms_all, wm[r * kMaxSplits + sp]);
        float Lt = 0.0f;
        for (int sp = 0; sp < ns; sp++) {
            const float ms = wm[r * kMaxSplits + sp];
            const float f = (ms == -INFINITY) ? 0.0f : fast_exp2(ms - ms_all);
            wm[r * kMaxSplits + sp] = f;
            Lt = fmaf(f, wl[r * kMaxSplits + sp], Lt);
        }
        Linv[r] = (Lt == 0.0f) ? 0.0f : 1.0f / Lt;
    }
    __syncthreads();
    // phase B: row r of this thread, the first 16 partials from `pre`
    auto accum_row = [&](int r, const float (&pre)[16], bool have_pre) {
        const float *po = a.part_o + (pr0 + r) * stride * kD + d;
        float acc = 0.0f;
        for (int s0 = 0; s0 < ns; s0 += 16) {
            // (the 16 weights are read together, past ns too: a row holds
            // kMaxSplits of them, and those past ns are not used)
            float ov[16], wv[16];
#pragma unroll
            for (int u = 0; u < 16; u++) wv[u] = wm[r * kMaxSplits + s0 + u];
#pragma unroll
            for (int u = 0; u < 16; u++)
                ov[u] = (s0 == 0 && have_pre) ? pre[u] : (s0 + u < ns ? ld_dev(po + (int64_t)(s0 + u) * kD) : 0.0f);
#pragma unroll
            for (int u = 0; u < 16; u++)
                if (s0 + u < ns) acc = fmaf(wv[u], ov[u], acc);
        }
        const int rg = t.rt * 16 + r;
        const int iq1o = rg / a.G, heado = t.kvh * a.G + rg % a.G;
        a.dst[(((int64_t)t.b * a.Sq + iq1o) * a.Nh + heado) * kD + d] = acc * Linv[r];
    };
    if (rA < nr) accum_row(rA, pa, true);
    if (rB < nr) accum_row(rB, pb, true);
    for (int r = rA + 4; r < nr; r += 2) accum_row(r, pa, false);
}

// Merges the 4 waves' (m, l, O^T) of the tile and writes the output (one
// split) or the split's partial; with several splits, the tile's last
// workgroup to finish merges all partials.  `lds` must hold 33 KB, free
// once every wave has passed the first barrier.  o[dt][i] =
// O^T[16dt + 4*g16 + i][row c16] (unnormalised), m2 in the exp2 domain,
// lsum the lane's share of the row sum.
__device__ void finish_tile(const FaArgs &a, const Tile &t, int ns, const f32x4 (&o)[8], float m2, float lsum,
                            float *lds, int *last_lds) {
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
    __syncthreads();
    float *mo = lds;                             // [wave][d][16 rows]
    float *mm = mo + kDecWaves * kD * 16;        // [wave][16] max
    float *ml = mm + kDecWaves * 16;             // [wave][16] sum
#pragma unroll
    for (int dt = 0; dt < 8; dt++)
#pragma unroll
        for (int i = 0; i < 4; i++) mo[(t.wave * kD + 16 * dt + 4 * t.g16 + i) * 16 + t.c16] = o[dt][i];
    if (t.g16 == 0) {
        mm[t.wave * 16 + t.c16] = m2;
        ml[t.wave * 16 + t.c16] = lsum;
    }
    __syncthreads();

    const int rr = t.tid & 15;
    const int dd0 = (t.tid >> 4) * 8;
    const int rglob = t.rt * 16 + rr;
    const bool out_row = rglob < a.M;
    float mw[kDecWaves];
    float mstar = -INFINITY;
#pragma unroll
    for (int w = 0; w < kDecWaves; w++) {
        mw[w] = mm[w * 16 + rr];
        mstar = fmaxf(mstar, mw[w]);
    }
    float fw[kDecWaves];
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < kDecWaves; w++) {
        fw[w] = (mw[w] == -INFINITY) ? 0.0f : fast_exp2(mw[w] - mstar);
        L += fw[w] * ml[w * 16 + rr];
    }
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        float sacc = 0.0f;
#pragma unroll
        for (int w = 0; w < kDecWaves; w++) sacc += fw[w] * mo[(w * kD + dd0 + e) * 16 + rr];
        acc[e] = sacc;
    }
    const int iq1o = rglob / a.G, heado = t.kvh * a.G + rglob % a.G;
    float *dp = a.dst + (((int64_t)t.b * a.Sq + iq1o) * a.Nh + heado) * kD + dd0;
    if (ns == 1) {
        if (!out_row) return;
        const float inv = (L == 0.0f) ? 0.0f : 1.0f / L;
        *(f32x4 *)dp = f32x4{acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
        *(f32x4 *)(dp + 4) = f32x4{acc[4] * inv, acc[5] * inv, acc[6] * inv, acc[7] * inv};
        return;
    }

    // Several splits: partial out, then the tile's last workgroup merges.
    // Every value that crosses workgroups is itself an agent-scope atomic
    // access: the partials go out as agent-scope stores (global_store ... sc1,
    // the encoding of a relaxed agent-scope atomic store on this
    // architecture, written through to the device coherence point), the
    // ticket is an agent-scope atomic add, and the merge reads the partials
    // with agent-scope atomic loads (sc1, served from the coherence point,
    // never from a stale L2 line).  A store counts in vmcnt until the
    // coherence point has acknowledged it, so `s_waitcnt vmcnt(0)` in every
    // wave, then the barrier, put every partial at the coherence point before
    // thread 0 issues its ticket add; the workgroup that draws the last
    // ticket issues its loads after that add has returned.  The compiler
    // keeps this order: the waitcnt is an asm statement with a "memory"
    // clobber, which no memory access may cross; the merge's loads are
    // atomic (never speculated) and sit behind the ticket's value, which
    // reaches every wave through LDS and a barrier.  The compiler's
    // release/acquire fences at agent scope would add a whole-L2 write-back
    // (buffer_wbl2) per wave and an L2 invalidate (buffer_inv) per ticket --
    // measured: C3 44.7 -> 140 us, C5 31 -> 57 us -- to cover ordinary
    // stores, which this protocol does not publish.
    const int64_t tile = ((int64_t)t.b * a.Nkv + t.kvh) * a.row_tiles + t.rt;
    const int64_t pr0 = ((int64_t)t.b * a.Nkv + t.kvh) * a.M + t.rt * 16;   // first row of the tile
    if (out_row) {
        float *po = a.part_o + ((pr0 + rr) * a.n_splits + t.split) * kD + dd0;
        st_agent16(po, f32x4{acc[0], acc[1], acc[2], acc[3]});
        st_agent16(po + 4, f32x4{acc[4], acc[5], acc[6], acc[7]});
        if (dd0 == 0) {
            float *pm = a.part_ml + ((pr0 + rr) * a.n_splits + t.split) * 2;
            __hip_atomic_store(pm, mstar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(pm + 1, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (t.tid == 0) {
        const int prev = __hip_atomic_fetch_add(&a.tickets[tile], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *last_lds = prev == ns - 1;
    }
    __syncthreads();
    if (!*last_lds) return;
    if (t.tid == 0) __hip_atomic_store(&a.tickets[tile], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    merge_splits(a, t, pr0, min(16, a.M - t.rt * 16), ns, lds);
}

// ---------------------------------------------------------------------------
// LDS-streaming kernel (F16 / BF16).
// ---------------------------------------------------------------------------

// MFMA 16x16x16 for the PV product of 16-key blocks (4 k-values per lane).
template <int T> struct Mfma16k16;
template <> struct Mfma16k16<T_F16> {
    typedef _Float16 v4 __attribute__((ext_vector_type(4)));
    static __device__ __forceinline__ f32x4 run(u16x4 a, u16x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(v4, a), __builtin_bit_cast(v4, b), c, 0, 0,
                                                     0);
    }
};
template <> struct Mfma16k16<T_BF16> {
    typedef short v4 __attribute__((ext_vector_type(4)));
    static __device__ __forceinline__ f32x4 run(u16x4 a, u16x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(v4, a), __builtin_bit_cast(v4, b), c, 0,
                                                         0, 0);
    }
};

// One stage: K [16 keys][256 B], V [16 keys][256 B], mask [16 rows][16 keys].
constexpr int kStK = 0, kStV = 4096, kStM = 8192, kStBytes = 8704;

// 16-byte chunk c of V row k (k < 16 within the stage) sits at slot
// c ^ swz_dv(k): the transpose reads of one half-wave (8 keys x 2 chunks x
// 2 halves) then cover all 64 banks once.  K rows use swz_k (k & 15).
__device__ __forceinline__ int swz_dv(int k) { return 2 * (k & 7); }

template <int NST> constexpr int lds_bytes_lds_kernel() { return NST * kDecWaves * kStBytes; }

// Waits until at most n stages of DMA (of PER instructions each) are in
// flight.
template <int PER, int NST>
__device__ __forceinline__ void wait_stages(int n) {
    static_assert(PER * (NST - 1) <= 63, "vmcnt range");
    if constexpr (NST > 3) {
        if (n >= 3) { MXFA_WAIT_VMCNT(3 * PER); return; }
    }
    if constexpr (NST > 2) {
        if (n == 2) { MXFA_WAIT_VMCNT(2 * PER); return; }
    }
    if (n == 1) { MXFA_WAIT_VMCNT(PER); return; }
    MXFA_WAIT_VMCNT(0);
}

template <int KT, int MM, int NST>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
fa_decode_lds_kernel(const FaArgs a) {
    static_assert(MM == kMaskNone || MM == kMaskVec || MM == kMaskStruct, "mask mode");
    static_assert(NST >= 2 && NST <= 4, "stages");
    using MF = Mfma16<KT>;
    using V8 = typename MF::v8;
    using PV = Mfma16k16<KT>;
    constexpr int kPer = 8 + (MM == kMaskVec ? 2 : 0);   // DMA instructions per stage
    static_assert(kD == 128, "kernel is written for D = 128");

    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ int range_lds[2 * kDecWaves];
    __shared__ int last_lds;

    const Tile t = make_tile<MM>(a);
    const SplitRange sr = split_range<MM>(a, t);
    if (sr.skip) return;   // past the stream's last split (uniform: no waits, no LDS, no ticket)
    // the live-range scan's loads go out first (dense mask), then Q's
    ScanPre scan{};
    if constexpr (MM == kMaskVec) scan = scan_issue(a, t, sr.k0, sr.k1);
    const QRaw qraw = q_issue(a, t);
    const int lane = t.lane, c16 = t.c16, g16 = t.g16;
    V8 qb[4];
    const float slope_l2 = alibi_slope(a, t.head) * kLog2e;
    const char *kbase = a.k + (int64_t)t.kvh * a.k_nb2 + (int64_t)t.bk * a.k_nb3;
    const char *vbase = a.v + (int64_t)t.kvh * a.v_nb2 + (int64_t)t.bk * a.v_nb3;
    const float sl2 = a.scale * kLog2e;
    const bool use_softcap = a.softcap != 0.0f;
    const float sc_in = a.softcap_in;
    const int skv4 = (a.Skv + 3) & ~3;
    const int k0 = sr.k0, k1 = sr.k1;
    uint8_t *ring = smem + t.wave * NST * kStBytes;
    // structured mask: the live keys of this lane's row
    int rlo = 0, rhi = 0;
    if constexpr (MM == kMaskStruct) sm_row_range(a, t.b, t.iq1, rlo, rhi);

    // DMA lane geometry.  K/V: instruction j covers keys 4j..4j+3 of the
    // stage, lane -> (key 4j + lane/16, slot lane%16).  Mask: instruction i
    // covers rows 8i..8i+7, lane -> (row 8i + lane/8, keys 2(lane%8), +1);
    // rows past M read row 0 of the tile (unused).
    const int dkey = lane >> 4, dslot = lane & 15;
    const int mpair = 2 * (lane & 7);
    const uint16_t *mdma[2] = {nullptr, nullptr};
    if constexpr (MM == kMaskVec) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            int rr = t.rt * 16 + 8 * i + (lane >> 3);
            if (rr >= a.M) rr = t.rt * 16;
            mdma[i] = mask_row(a, rr / a.G, t.kvh * a.G + rr % a.G, t.b);
        }
    }
    auto issue = [&](int kb, int slot) {
        uint8_t *st = ring + slot * kStBytes;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int kr = 4 * j + dkey;
            const int key = min(kb + kr, a.Skv - 1);
            dma16(kbase + (int64_t)key * a.k_nb1 + 16 * (dslot ^ swz_k(kr)), st + kStK + 1024 * j);
            dma16(vbase + (int64_t)key * a.v_nb1 + 16 * (dslot ^ swz_dv(kr)), st + kStV + 1024 * j);
        }
        if constexpr (MM == kMaskVec) {
            // key pairs at or past round_up(Skv, 4) (keys >= Skv, never
            // used) re-read the last pair of the row
            const int kp = min(kb + mpair, skv4 - 2);
#pragma unroll
            for (int i = 0; i < 2; i++) dma4(mdma[i] + kp, st + kStM + 256 * i);
        }
    };

    // Speculative fill: the first stages of [k0, k1) -- the whole ring -- go
    // out before the live range is known, so that the wait below (which the
    // scan needs anyway) does not leave the ring empty behind it.
    const int kbw_spec = k0 + 16 * t.wave;
    const int nblk_spec = kbw_spec < k1 ? (k1 - kbw_spec + 63) / 64 : 0;
    // (one stage under a dense mask: a split that the scan finds wholly past
    // its sequence's end then wastes one stage of K/V reads, not a ring)
    const int n_spec = min(MM == kMaskVec ? 1 : NST, nblk_spec);
    for (int s = 0; s < n_spec; s++) issue(kbw_spec + 64 * s, s);

    q_convert16<KT>(a, qraw, qb);
    int lo = k0, hi = k1;
    if constexpr (MM == kMaskVec) scan_finish(a, t, scan, k0, k1, range_lds, lo, hi);
    // the speculative stages have landed (they drain with Q's and the scan's
    // loads: one memory latency for all three)
    MXFA_WAIT_VMCNT(0);

    const int base = lo < hi ? k0 + ((lo - k0) & ~63) : k0;
    const int kbw = base + 16 * t.wave;
    const int n_blk = (lo < hi && kbw < hi) ? (hi - kbw + 63) / 64 : 0;
    const int done_upto = base == k0 ? min(n_spec, n_blk) : 0;   // stages already in LDS

    f32x4 o[8];
#pragma unroll
    for (int dt = 0; dt < 8; dt++) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m2 = -INFINITY;   // running max of this lane's row (exp2 domain)
    float lsum = 0.0f;      // this lane's share of the row sum

    // transpose-read geometry of the V^T operand: this lane addresses the
    // 8-byte chunk (key 4*g16 + c16/4, dims 16dt + 4(c16%4) .. +4); lane j
    // of the 16-lane group then receives V[4*g16 + e][16dt + j], e = 0..3
    const int tr_key = 4 * g16 + (c16 >> 2);
    const int tr_chunk = (c16 & 3) >> 1, tr_half = c16 & 1;

    auto compute = [&](int kb, int slot) {
        const uint8_t *st = ring + slot * kStBytes;
        // mask entries of (row c16, keys kb + 4*g16 + i)
        float mk[4];
        int live = 0;
        u16x4 mw = {0, 0, 0, 0};
        if constexpr (MM == kMaskVec) mw = *(const u16x4 *)(st + kStM + c16 * 32 + 8 * g16);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int key = kb + 4 * g16 + i;
            float mv = -INFINITY;
            const bool in_row = MM != kMaskStruct || (key >= rlo && key < rhi);
            if (t.row_ok && key < hi && in_row) mv = MM == kMaskVec ? h2f_bits(mw[i]) * slope_l2 : 0.0f;
            mk[i] = mv;
            live |= (mv != -INFINITY);
        }
        if (!__any(live)) return;
        // keys dead for every row of the tile (AND over the 16 rows)
        uint32_t dead = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) dead |= (mk[i] == -INFINITY ? 1u : 0u) << i;
        dead = and_rows16(dead);

        // S^T[key 4*g16 + i][row c16] = K . Q^T
        f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const u16x8 av = *(const u16x8 *)(st + kStK + c16 * 256 + 16 * ((4 * q + g16) ^ swz_k(c16)));
            s = MF::run(__builtin_bit_cast(V8, av), qb[q], s);
        }
        // online softmax (exp2 domain, lazy rescale: the reference max is
        // raised only when some row's new max exceeds it by more than 8, so
        // p <= 2^8; O and l share the reference, the softmax is unchanged)
        float xs[4];
        float bmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float xv;
            if (use_softcap) xv = (a.softcap * tanhf(s[i] * sc_in)) * kLog2e + mk[i];
            else xv = fmaf(s[i], sl2, mk[i]);
            xv = (mk[i] == -INFINITY) ? -INFINITY : xv;
            xs[i] = xv;
            bmax = fmaxf(bmax, xv);
        }
        bmax = max_half32(max_pair16(bmax));
        if (__any(bmax > m2 + 8.0f)) {
            const float mnew = fmaxf(m2, bmax);
            const float alpha = (mnew == -INFINITY) ? 1.0f : fast_exp2(m2 - mnew);
            m2 = mnew;
            lsum *= alpha;
#pragma unroll
            for (int dt = 0; dt < 8; dt++) o[dt] *= alpha;
        }
        const float m_use = (m2 == -INFINITY) ? 0.0f : m2;
        f32x4 p;
#pragma unroll
        for (int i = 0; i < 4; i++) p[i] = fast_exp2(xs[i] - m_use);   // exp2(-inf) = 0
        const u16x8 pb8 = cvt8<KT>(p, f32x4{0.f, 0.f, 0.f, 0.f});
        lsum = sum8<KT>(pb8, lsum);
        const u16x4 pb = {pb8[0], pb8[1], pb8[2], pb8[3]};
        // bf16: the lo parts of P for a second PV product (bf16_lo)
        u16x4 pl = {0, 0, 0, 0};
        if constexpr (KT == T_BF16) {
            const u16x8 pl8 = bf16_lo8(p, f32x4{0.f, 0.f, 0.f, 0.f}, pb8);
            lsum = sum8<KT>(pl8, lsum);
            pl = u16x4{pl8[0], pl8[1], pl8[2], pl8[3]};
        }

        // O^T[d][row] += V^T[d][keys 4*g16 + e] . P^T; V values of dead
        // keys are masked to zero (operand element e <-> key 4*g16 + e)
        uint64_t vmask = ~(uint64_t)0;
#pragma unroll
        for (int e = 0; e < 4; e++)
            if (dead & (1u << e)) vmask &= ~((uint64_t)0xFFFF << (16 * e));
        const bool any_dead = __any(dead != 0);
#pragma unroll
        for (int dt = 0; dt < 8; dt++) {
            const int c = 2 * dt + tr_chunk;
            u16x4 av = lds_read_tr16(st + kStV + tr_key * 256 + 16 * (c ^ swz_dv(tr_key)) + 8 * tr_half);
            if (any_dead) av = __builtin_bit_cast(u16x4, __builtin_bit_cast(uint64_t, av) & vmask);
            o[dt] = PV::run(av, pb, o[dt]);
            if constexpr (KT == T_BF16) o[dt] = PV::run(av, pl, o[dt]);
        }
    };

    // NST-stage ring: stage n lives in slot n % NST; stage n + NST - 1 is
    // issued before stage n is computed (its slot was read by stage n - 1).
    int issued = done_upto;
    while (issued < min(n_blk, NST - 1)) {
        issue(kbw + 64 * issued, issued % NST);
        issued++;
    }
    for (int n = 0; n < n_blk; n++) {
        if (issued < n_blk && issued <= n + NST - 1) {
            issue(kbw + 64 * issued, issued % NST);
            issued++;
        }
        if (n >= done_upto) wait_stages<kPer, NST>(issued - 1 - n);
        compute(kbw + 64 * n, n % NST);
        MXFA_WAIT_LGKMCNT0();   // this slot's LDS reads are done before it is refilled
    }
    MXFA_WAIT_VMCNT(0);
    finish_tile(a, t, sr.ns, o, m2, lsum, (float *)smem, &last_lds);
}

// ---------------------------------------------------------------------------
// Register-streaming kernel (Q8_0, and F16/BF16 with an unaligned mask).
// ---------------------------------------------------------------------------

// Q8_0 row of 128 values: 4 blocks of {fp16 d, int8 qs[32]} = 136 bytes.
// A lane reads the 8 qs bytes at offset o = 34t + 2 + 8j of block t through
// a 12-byte window starting at the 4-byte aligned a0 = 34t + 8j - 2(t & 1):
// the bytes sit at window offset 2 (t even) or 4 (t odd).  For j = 0 the
// window also holds the block's d: low half of word 0 (t even) or high
// half (t odd).  Every window lies inside its row.
struct W3 {
    uint32_t w0, w1, w2;
};

__device__ __forceinline__ W3 load_w3(const char *p) {
    const uint32_t *q = (const uint32_t *)p;   // 4-byte aligned
    return W3{q[0], q[1], q[2]};
}

// Register image of one lane's share of a 32-key block.
struct BlkF {          // F16 / BF16
    u16x8 k[2][4];     // K: key 16sb + c16, dims 32t + 8g16 .. +8
    u16x8 v[2][4];     // V: key 4g16 + 16j + kk, dims 8c16 .. +8
    u16x4 m[2];        // mask: row c16, keys 16sb + 4g16 .. +4
};
struct BlkQ {          // Q8_0 windows
    W3 k[2][4];        // K: key 16sb + c16, block t, qs 8g16 .. +8
    W3 v[2][4];        // V: key 4g16 + 16j + kk, block c16/4, qs 8(c16%4) .. +8
    u16x4 m[2];
};

// Dequantises 8 int8 values (two words) times d to 8 f16 bit patterns.
// (q ^ 0x80) placed under the f16 exponent of 1024 reads as 1152 + q
// exactly; subtracting 1152 gives q exactly, and one f16 multiply by d
// rounds q*d once, as the fp32 product rounded to f16 would.
__device__ __forceinline__ u16x8 dequant8(uint32_t lo, uint32_t hi, _Float16 d) {
    const uint32_t x0 = lo ^ 0x80808080u, x1 = hi ^ 0x80808080u;
    const uint32_t e[4] = {__builtin_amdgcn_perm(0x64646464u, x0, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, x0, 0x04030402u),
                           __builtin_amdgcn_perm(0x64646464u, x1, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, x1, 0x04030402u)};
    const f16x2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    const f16x2 dd = {d, d};
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const f16x2 v = (__builtin_bit_cast(f16x2, e[i]) - bias) * dd;
        r[i] = __builtin_bit_cast(uint32_t, v);
    }
    return __builtin_bit_cast(u16x8, r);
}

template <int KT, int MM>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
fa_decode_reg_kernel(const FaArgs a) {
    constexpr bool kQ8 = KT == T_Q8_0;
    constexpr int TV = kQ8 ? T_F16 : KT;        // format of the PV product
    using MF = Mfma16<TV>;
    using V8 = typename MF::v8;
    using Blk = std::conditional_t<kQ8, BlkQ, BlkF>;
    static_assert(kD == 128, "kernel is written for D = 128");

    __shared__ __attribute__((aligned(16))) uint16_t vt_lds[kDecWaves * kD * kVtStride];
    __shared__ int range_lds[2 * kDecWaves];
    __shared__ int last_lds;

    const Tile t = make_tile<MM>(a);
    const SplitRange sr = split_range<MM>(a, t);
    if (sr.skip) return;   // past the stream's last split (uniform: no waits, no LDS, no ticket)
    constexpr bool kDense = MM == kMaskVec || MM == kMaskScalar;   // a dense mask is read
    // the live-range scan's loads go out first (dense masks)
    ScanPre scan{};
    if constexpr (kDense) scan = scan_issue(a, t, sr.k0, sr.k1);
    const QRaw qraw = q_issue(a, t);
    const int c16 = t.c16, g16 = t.g16;
    V8 qb[4];
    long qq[4];
    float dq[4];
    const float slope_l2 = alibi_slope(a, t.head) * kLog2e;
    const uint16_t *mrow = kDense ? mask_row(a, t.iq1, t.head, t.b) : nullptr;
    const int skv4 = (a.Skv + 3) & ~3;
    const char *kbase = a.k + (int64_t)t.kvh * a.k_nb2 + (int64_t)t.bk * a.k_nb3;
    const char *vbase = a.v + (int64_t)t.kvh * a.v_nb2 + (int64_t)t.bk * a.v_nb3;
    const float sl2 = a.scale * kLog2e;
    const bool use_softcap = a.softcap != 0.0f;
    const float sc_in = a.softcap_in;

    const int k0 = sr.k0, k1 = sr.k1;
    int lo = k0, hi = k1;   // live range (dense masks: scanned below)
    int rlo = 0, rhi = 0;
    if constexpr (MM == kMaskStruct) sm_row_range(a, t.b, t.iq1, rlo, rhi);

    f32x4 o[8];
#pragma unroll
    for (int dt = 0; dt < 8; dt++) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m2 = -INFINITY;
    float lsum = 0.0f;
    uint16_t *vt = vt_lds + t.wave * kD * kVtStride;

    // Q8_0 V: lane c16 covers block tv = c16/4, qs bytes 8(c16%4) .. +8
    const int tv = c16 >> 2;
    const bool tv_odd = tv & 1;
    const int v_off = 34 * tv + 8 * (c16 & 3) - 2 * (tv & 1);

    // loads of one block into registers.  Keys past Skv are clamped to a
    // valid row (their scores are -inf and their V values zeroed).
    auto load = [&](int kb, Blk &x) {
#pragma unroll
        for (int sb = 0; sb < 2; sb++) {
            const int key = min(kb + 16 * sb + c16, a.Skv - 1);
            const char *kp = kbase + (int64_t)key * a.k_nb1;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                if constexpr (kQ8) x.k[sb][q] = load_w3(kp + 34 * q + 8 * g16 - 2 * (q & 1));
                else x.k[sb][q] = *(const u16x8 *)(kp + 16 * g16 + 64 * q);
            }
        }
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                const int key = min(kb + 4 * g16 + 16 * j + kk, a.Skv - 1);
                const char *vp = vbase + (int64_t)key * a.v_nb1;
                if constexpr (kQ8) x.v[j][kk] = load_w3(vp + v_off);
                else x.v[j][kk] = *(const u16x8 *)(vp + 16 * c16);
            }
        if constexpr (MM == kMaskVec) {
            // rows hold >= round_up(Skv, 4) entries: groups at or past that
            // are clamped to the last group (their keys are >= Skv, unused)
#pragma unroll
            for (int sb = 0; sb < 2; sb++)
                x.m[sb] = *(const u16x4 *)(mrow + min(kb + 16 * sb + 4 * g16, skv4 - 4));
        } else if constexpr (MM == kMaskScalar) {
#pragma unroll
            for (int sb = 0; sb < 2; sb++)
#pragma unroll
                for (int i = 0; i < 4; i++) x.m[sb][i] = mrow[min(kb + 16 * sb + 4 * g16 + i, a.Skv - 1)];
        }
    };

    auto compute = [&](int kb, const Blk &x) {
        float mk[2][4];
        int live = 0;
#pragma unroll
        for (int sb = 0; sb < 2; sb++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int key = kb + 16 * sb + 4 * g16 + i;
                float mv = -INFINITY;
                const bool in_row = MM != kMaskStruct || (key >= rlo && key < rhi);
                if (t.row_ok && key < hi && in_row) mv = kDense ? h2f_bits(x.m[sb][i]) * slope_l2 : 0.0f;
                mk[sb][i] = mv;
                live |= (mv != -INFINITY);
            }
        if (!__any(live)) return;

        uint32_t dead = 0;
#pragma unroll
        for (int sb = 0; sb < 2; sb++)
#pragma unroll
            for (int i = 0; i < 4; i++) dead |= (mk[sb][i] == -INFINITY ? 1u : 0u) << (4 * sb + i);
        dead = and_rows16(dead);

        // S^T tile: lane holds S^T[key 16sb+4g16+i][row c16]
        f32x4 s[2];
#pragma unroll
        for (int sb = 0; sb < 2; sb++) {
            if constexpr (!kQ8) {
                s[sb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int q = 0; q < 4; q++) s[sb] = MF::run(__builtin_bit_cast(V8, x.k[sb][q]), qb[q], s[sb]);
            } else {
                i32x4 is[4];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const W3 &w = x.k[sb][q];
                    const uint32_t ql = (q & 1) ? w.w1 : __builtin_amdgcn_alignbyte(w.w1, w.w0, 2);
                    const uint32_t qh = (q & 1) ? w.w2 : __builtin_amdgcn_alignbyte(w.w2, w.w1, 2);
                    const long ka = (long)(((uint64_t)qh << 32) | ql);
                    is[q] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ka, qq[q], i32x4{0, 0, 0, 0}, 0, 0, 0);
                }
                // d_k of key c16 sits in the g16 = 0 lanes' windows (blocks
                // 0, 2: low half of word 0; blocks 1, 3: high half)
                const uint32_t p01 = (x.k[sb][0].w0 & 0xFFFFu) | (x.k[sb][1].w0 & 0xFFFF0000u);
                const uint32_t p23 = (x.k[sb][2].w0 & 0xFFFFu) | (x.k[sb][3].w0 & 0xFFFF0000u);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t d01 = (uint32_t)__shfl((int)p01, 4 * g16 + i);
                    const uint32_t d23 = (uint32_t)__shfl((int)p23, 4 * g16 + i);
                    const float dk[4] = {h2f_bits((uint16_t)d01), h2f_bits((uint16_t)(d01 >> 16)),
                                         h2f_bits((uint16_t)d23), h2f_bits((uint16_t)(d23 >> 16))};
                    float acc = 0.0f;
#pragma unroll
                    for (int q = 0; q < 4; q++) acc = fmaf(dk[q] * dq[q], (float)is[q][i], acc);
                    s[sb][i] = acc;
                }
            }
        }

        float xs[2][4];
        float bmax = -INFINITY;
#pragma unroll
        for (int sb = 0; sb < 2; sb++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float xv;
                if (use_softcap) xv = (a.softcap * tanhf(s[sb][i] * sc_in)) * kLog2e + mk[sb][i];
                else xv = fmaf(s[sb][i], sl2, mk[sb][i]);
                xv = (mk[sb][i] == -INFINITY) ? -INFINITY : xv;
                xs[sb][i] = xv;
                bmax = fmaxf(bmax, xv);
            }
        bmax = max_half32(max_pair16(bmax));
        if (__any(bmax > m2 + 8.0f)) {
            const float mnew = fmaxf(m2, bmax);
            const float alpha = (mnew == -INFINITY) ? 1.0f : fast_exp2(m2 - mnew);
            m2 = mnew;
            lsum *= alpha;
#pragma unroll
            for (int dt = 0; dt < 8; dt++) o[dt] *= alpha;
        }
        const float m_use = (m2 == -INFINITY) ? 0.0f : m2;
        f32x4 p0, p1;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            p0[i] = fast_exp2(xs[0][i] - m_use);
            p1[i] = fast_exp2(xs[1][i] - m_use);
        }
        const u16x8 pbits = cvt8<TV>(p0, p1);
        lsum = sum8<TV>(pbits, lsum);
        const V8 pb = __builtin_bit_cast(V8, pbits);
        // bf16: the lo parts of P for a second PV product (bf16_lo)
        V8 pl = {};
        if constexpr (TV == T_BF16) {
            const u16x8 lbits = bf16_lo8(p0, p1, pbits);
            lsum = sum8<TV>(lbits, lsum);
            pl = __builtin_bit_cast(V8, lbits);
        }

        // V^T into this wave's LDS tile.  Chunk kc (4 keys) of row d is
        // stored at chunk slot kc ^ ((d >> 4) & 7).
#pragma unroll
        for (int j = 0; j < 2; j++) {
            u16x8 vr[4];
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                if constexpr (kQ8) {
                    const W3 &w = x.v[j][kk];
                    const uint32_t ql = tv_odd ? w.w1 : __builtin_amdgcn_alignbyte(w.w1, w.w0, 2);
                    const uint32_t qh = tv_odd ? w.w2 : __builtin_amdgcn_alignbyte(w.w2, w.w1, 2);
                    // d of the block is in the window of the quad's first lane
                    const uint32_t dsrc = tv_odd ? (w.w0 >> 16) : (w.w0 & 0xFFFFu);
                    const uint32_t dbits = (uint32_t)__builtin_amdgcn_mov_dpp((int)dsrc, 0x00, 0xF, 0xF, false);
                    vr[kk] = dequant8(ql, qh, __builtin_bit_cast(_Float16, (uint16_t)dbits));
                } else {
                    vr[kk] = x.v[j][kk];
                }
                if (dead & (1u << (4 * j + kk))) vr[kk] = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
            }
            const int kc = g16 + 4 * j;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int d = 8 * c16 + e;
                u16x4 w = {vr[0][e], vr[1][e], vr[2][e], vr[3][e]};
                *(u16x4 *)(vt + d * kVtStride + 4 * (kc ^ ((d >> 4) & 7))) = w;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        // O^T[d][row] += V^T[d][keys] . P^T[keys][row]
#pragma unroll
        for (int dt = 0; dt < 8; dt++) {
            const int d = 16 * dt + c16;
            const uint16_t *row = vt + d * kVtStride;
            u16x4 vlo = *(const u16x4 *)(row + 4 * (g16 ^ dt));
            u16x4 vhi = *(const u16x4 *)(row + 4 * ((g16 + 4) ^ dt));
            u16x8 av = {vlo[0], vlo[1], vlo[2], vlo[3], vhi[0], vhi[1], vhi[2], vhi[3]};
            o[dt] = MF::run(__builtin_bit_cast(V8, av), pb, o[dt]);
            if constexpr (TV == T_BF16) o[dt] = MF::run(__builtin_bit_cast(V8, av), pl, o[dt]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };

    // Blocks of this wave: kb0 + 128 n, n < n_blk.  Two register images
    // alternate; the loads of the next block are issued unconditionally
    // before the current block is computed, so the compiler's wait for the
    // current image leaves them in flight.  Under a dense mask the scan's
    // loads go out first (at the kernel's start), then Q's; then the first
    // block from the split start, and Q is converted (and the scan reduced)
    // while that block is in flight.  Without a mask the live range is the
    // split, so that block is always the first one; under a dense mask it is
    // the right block whenever the live range starts in the split's first 32
    // keys, as it does for every live split of a padding mask, and is loaded
    // again otherwise.  (A second speculative block measured slower: C5 28.2
    // against 27.0 us.)  Under a structured mask the block is loaded after
    // Q's conversion: loaded early, it made the compiler spill (C5's shape
    // under a structured mask: 35.1 against 27.4 us).
    constexpr bool kEarly = MM != kMaskStruct;
    {
        Blk x0, x1;
        const int kb_spec = k0 + 32 * t.wave;
        if constexpr (kEarly) {
            if (kb_spec < k1) load(kb_spec, x0);
        }
        if constexpr (kQ8) q_convert8(qraw, qq, dq);
        else q_convert16<TV>(a, qraw, qb);
        if constexpr (kDense) scan_finish(a, t, scan, k0, k1, range_lds, lo, hi);
        const int kb0 = k0 + ((lo - k0) & ~31) + 32 * t.wave;
        const int n_blk = (lo < hi && kb0 < hi) ? (hi - kb0 + 32 * kDecWaves - 1) / (32 * kDecWaves) : 0;
        if (n_blk > 0) {
            if (!kEarly || kb0 != kb_spec) load(kb0, x0);   // (early: kb0 differs under dense masks only)
            for (int n = 0;;) {
                const int kb = kb0 + 32 * kDecWaves * n;
                if (n + 1 == n_blk) {
                    compute(kb, x0);
                    break;
                }
                load(kb + 32 * kDecWaves, x1);
                compute(kb, x0);
                n++;
                if (n + 1 == n_blk) {
                    compute(kb + 32 * kDecWaves, x1);
                    break;
                }
                load(kb + 2 * 32 * kDecWaves, x0);
                compute(kb + 32 * kDecWaves, x1);
                n++;
            }
        }
    }
    finish_tile(a, t, sr.ns, o, m2, lsum, (float *)vt_lds, &last_lds);
}

// Zero-fill of the split tickets (run when the ticket buffer is created or
// grown; afterwards every merging workgroup leaves its ticket at zero).
__global__ void __launch_bounds__(256) fill_zero_kernel(int *p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0;
}

hipError_t launch_fill_zero(int *p, int64_t n, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, p, n);
    return hipGetLastError();
}

constexpr int kDecStages = 2;   // LDS ring depth of fa_decode_lds_kernel (2 workgroups per CU)

template <int KT, int MM>
static hipError_t launch_lds(const FaArgs &a, dim3 grid, hipStream_t stream) {
    constexpr int bytes = lds_bytes_lds_kernel<kDecStages>();
    // the dynamic LDS limit is a per-(function, device) attribute: set once
    // on each device that launches this instance
    static OncePerDevice attr;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    e = attr.run(dev, [] {
        return hipFuncSetAttribute((const void *)fa_decode_lds_kernel<KT, MM, kDecStages>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    });
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((fa_decode_lds_kernel<KT, MM, kDecStages>), grid, dim3(256), bytes, stream, a);
    return hipGetLastError();
}

template <int KT>
static hipError_t launch_typed(const FaArgs &a, dim3 grid, hipStream_t stream) {
    if constexpr (KT != T_Q8_0) {
        if (a.sm_flags) return launch_lds<KT, kMaskStruct>(a, grid, stream);
        if (!a.mask) return launch_lds<KT, kMaskNone>(a, grid, stream);
        if (a.mask_vec16) return launch_lds<KT, kMaskVec>(a, grid, stream);
        hipLaunchKernelGGL((fa_decode_reg_kernel<KT, kMaskScalar>), grid, dim3(256), 0, stream, a);
    } else {
        if (a.sm_flags) hipLaunchKernelGGL((fa_decode_reg_kernel<KT, kMaskStruct>), grid, dim3(256), 0, stream, a);
        else if (!a.mask) hipLaunchKernelGGL((fa_decode_reg_kernel<KT, kMaskNone>), grid, dim3(256), 0, stream, a);
        else if (a.mask_vec4) hipLaunchKernelGGL((fa_decode_reg_kernel<KT, kMaskVec>), grid, dim3(256), 0, stream, a);
        else hipLaunchKernelGGL((fa_decode_reg_kernel<KT, kMaskScalar>), grid, dim3(256), 0, stream, a);
    }
    return hipGetLastError();
}

hipError_t launch_fa_decode(const FaArgs &a, int ktype, hipStream_t stream) {
    const dim3 grid = a.dec_live > 0 ? dim3((uint32_t)a.dec_live) : dim3(a.n_splits, a.Nkv * a.row_tiles, a.B);
    return timed_launch("fa_decode", stream, [&] {
        switch (ktype) {
            case T_F16: return launch_typed<T_F16>(a, grid, stream);
            case T_BF16: return launch_typed<T_BF16>(a, grid, stream);
            case T_Q8_0: return launch_typed<T_Q8_0>(a, grid, stream);
            default: return hipErrorInvalidValue;
        }
    });
}

}  // namespace mxfa
