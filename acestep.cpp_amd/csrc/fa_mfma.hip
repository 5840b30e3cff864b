// fa_mfma.hip -- MFMA flash attention for prefill and DiT on gfx950.
//
// Serves the long-query call sites of the reference: LM causal prefill
// (src/qwen3-lm.h:465-469 with the causal mask of :597-610), DiT
// self-attention (src/dit-graph.h:227-231; sliding-window mask on even
// layers, none on odd ones, :575) and DiT cross-attention over the text
// encoder with its padding mask (src/dit-graph.h:348-352,
// src/dit-sampler.h:290-309), and the encoders (src/qwen3-enc.h:195-199).
//
// Work decomposition.  One workgroup = 4 waves = 128 consecutive queries of
// one (batch, q head); each wave owns 32 queries.  The workgroup walks the
// keys in 64-key tiles staged in LDS, double-buffered: while tile n is
// being multiplied, tile n+1 is already in flight from HBM into registers.
//
//   S^T[64 keys x 32 q] = K_tile . Q^T      v_mfma_f32_32x32x16_{f16,bf16}
//                                            (A = K rows from LDS, B = Q^T
//                                            held in registers all along)
//   online softmax on S^T in fp32 registers: each lane holds one query's
//   column, so the row max/sum need a single cross-lane step (lane ^ 32)
//   O^T[128 x 32 q] += V^T_tile . P^T       same MFMA; P^T comes straight
//                                            from the S^T accumulator layout,
//                                            V^T from the transposed LDS tile
//
// LDS tiles (16 KB each, XOR-swizzled so that the staging writes and the
// MFMA operand reads are bank-conflict free):
//   K   [64 keys][128 dims]  16-byte chunk c of key k at slot c ^ (k & 15)
//   V^T [128 dims][64 keys]  8-byte chunk c (4 keys) of dim d at slot
//                            c ^ ((d & 15) ^ ((d >> 4) & 7))
//
// Masks are data, not structure: a classifier pass (mask_classify_kernel)
// labels every (128-query x 64-key) tile of the mask as all -inf (skipped:
// no K/V traffic, no MFMA), all zero (no mask reads) or mixed (mask read per
// element).  The causal prefill mask thus costs half the work of the dense
// problem and no per-element mask traffic below the diagonal.

#include <type_traits>

#include "mxfa_common.h"
#include "mxfa_internal.h"


namespace mxfa {

constexpr int kTileBytes = 16384;            // one K or one V^T tile
constexpr int kStageBytes = 2 * kTileBytes;  // K + V^T
constexpr int kPfLds = 2 * kStageBytes;      // double buffered: 64 KB

__global__ void __launch_bounds__(256) mask_classify_kernel(const FaArgs a, uint8_t *cls) {
    // One workgroup per (key tile, query tile, mask plane).  Each row of the
    // tile (64 keys = 128 B) is read by 16 lanes with 8-byte loads; the
    // prefill path guarantees 8-byte aligned mask rows.
    const int kt = blockIdx.x, qt = blockIdx.y, plane = blockIdx.z;
    const int m2i = plane % a.m_ne2, m3i = plane / a.m_ne2;
    const char *base = a.mask + (int64_t)m2i * a.m_nb2 + (int64_t)m3i * a.m_nb3;
    const int q_lo = qt * kPfBM, k_lo = kt * kPfBN;
    const int c4 = threadIdx.x & 15;           // 4-key group within the row
    const int r0 = threadIdx.x >> 4;           // 16 rows per pass
    const int k = k_lo + 4 * c4;
    int all_ninf = 1, all_zero = 1;
#pragma unroll
    for (int pass = 0; pass < kPfBM / 16; pass++) {
        const int q = q_lo + r0 + 16 * pass;
        if (q >= a.Sq || k >= a.Skv) continue;
        const uint16_t *row = (const uint16_t *)(base + (int64_t)q * a.m_nb1);
        if (k + 3 < a.Skv) {
            const u16x4 v = *(const u16x4 *)(row + k);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                all_ninf &= (v[i] == 0xFC00u);
                all_zero &= ((v[i] & 0x7FFFu) == 0);
            }
        } else {
            for (int i = 0; i < 4 && k + i < a.Skv; i++) {
                const uint16_t v = row[k + i];
                all_ninf &= (v == 0xFC00u);
                all_zero &= ((v & 0x7FFFu) == 0);
            }
        }
    }
    all_ninf = __syncthreads_and(all_ninf);
    all_zero = __syncthreads_and(all_zero);
    if (threadIdx.x == 0) cls[((int64_t)plane * a.n_qt + qt) * a.n_kt_pad + kt] = all_ninf ? 0 : (all_zero ? 1 : 2);
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
    __device__ __forceinline__ int next_live(int kt, int n) const {
        if (!present) return kt;
        while (kt < n && at(kt) == 0) kt++;
        return kt;
    }
};

// Direct HBM -> LDS copy of 16 bytes per lane from a wave-uniform base plus
// a per-lane 32-bit byte offset (lane l's bytes land at lds_base + 16*l).
__device__ __forceinline__ void dma16_so(const char *sbase, uint32_t voff, void *lds_base) {
    const uint32_t lds_addr = (uint32_t)(uintptr_t)(lds_void *)lds_base;
    // the base is wave-uniform by contract; readfirstlane lets the compiler
    // see that too, so the "s" operand never lands in a VGPR pair
    const uint64_t b = (uint64_t)(uintptr_t)sbase;
    // (readfirstlane returns int: go through uint32_t so the low half is
    // zero-extended, never sign-extended into the high half)
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
    const uint64_t sb = ((uint64_t)hi << 32) | (uint64_t)lo;
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(voff), "s"(sb)
                 : "memory", "m0");
}

// Max of a lane's value and the same register of lane l ^ 32 (one
// v_permlane32_swap: lanes l and l ^ 32 hold the two key halves of a query).
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

template <int T>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
fa_prefill_kernel(const FaArgs a) {
    using MF = Mfma32<T>;
    using V8 = typename MF::v8;
    static_assert(kD == 128, "kernel is written for D = 128");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, h = lane >> 5;
    const int qt = gridDim.x - 1 - blockIdx.x;   // longest (causal) tiles first
    const int head = blockIdx.y, b = blockIdx.z;
    const int kvh = head / a.G, bk = b / a.rk3;
    const int qrow = qt * kPfBM + wave * 32 + l32;
    const bool row_ok = qrow < a.Sq;
    const int qrow_c = row_ok ? qrow : a.Sq - 1;

    // Q^T operand for the 8 dim-steps of 16: Q[qrow][16t + 8h + e].
    V8 qb[8];
    {
        const float *qp = (const float *)(a.q + (int64_t)qrow_c * a.q_nb1 + (int64_t)head * a.q_nb2 +
                                          (int64_t)b * a.q_nb3);
#pragma unroll
        for (int t = 0; t < 8; t++) {
            f32x4 x0 = {0.f, 0.f, 0.f, 0.f}, x1 = {0.f, 0.f, 0.f, 0.f};
            if (row_ok) {
                x0 = *(const f32x4 *)(qp + 16 * t + 8 * h);
                x1 = *(const f32x4 *)(qp + 16 * t + 8 * h + 4);
            }
            qb[t] = __builtin_bit_cast(V8, cvt8<T>(x0, x1));
        }
    }

    const int plane = a.mask ? (b % a.m_ne3) * a.m_ne2 + head % a.m_ne2 : 0;
    TileClasses tc{0u, 0u, a.tile_class != nullptr};
    if (tc.present) {
        const uint32_t *row = (const uint32_t *)(a.tile_class + ((int64_t)plane * a.n_qt + qt) * a.n_kt_pad);
        const int lane4 = 4 * lane;
        if (lane4 < a.n_kt) tc.w0 = row[lane4 >> 2];
        if (256 + lane4 < a.n_kt) tc.w1 = row[(256 + lane4) >> 2];
    }
    const uint16_t *mrow =
        a.mask ? (const uint16_t *)(a.mask + (int64_t)qrow_c * a.m_nb1 + (int64_t)(head % a.m_ne2) * a.m_nb2 +
                                    (int64_t)(b % a.m_ne3) * a.m_nb3)
               : nullptr;
    const float slope_l2 = alibi_slope(a, head) * kLog2e;
    const float sl2 = a.scale * kLog2e;
    const bool use_softcap = a.softcap != 0.0f;
    const float sc_in = use_softcap ? a.scale / a.softcap : 0.0f;
    // the lean path takes max over raw scores, valid for a positive scale
    const bool lean_ok = !use_softcap && sl2 > 0.0f;

    const char *kbase = a.k + (int64_t)kvh * a.k_nb2 + (int64_t)bk * a.k_nb3;
    const char *vbase = a.v + (int64_t)kvh * a.v_nb2 + (int64_t)bk * a.v_nb3;

    f32x16 o[4];
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[dt][r] = 0.0f;
    float m2 = -INFINITY, lsum = 0.0f;

    // Tile staging: each wave DMAs keys 16w..16w+15 of K and of V (4
    // instructions of 4 keys x 16 chunks); lane -> (key 4j + lane/16, slot
    // lane%16), the slot holding the swizzled logical chunk.  Row 4j + dk
    // (dk = lane/16) of the wave's 16 comes from the wave-uniform base
    // tile + (16w + 4j) rows plus a per-lane offset dk * nb1 + 16 * chunk.
    // With swz_k(k) = k & 15 the chunk is (slot ^ dk) ^ 4j, and with swz_v
    // it is (slot ^ swz_v(dk)) ^ 2(j & 1): when nb1 is a multiple of 256 the
    // offset is one register XOR a per-j constant.  The last, partial tile
    // clamps keys to Skv - 1.
    const int dma_key = lane >> 4, dma_slot = lane & 15;
    const bool nb_fast = (a.k_nb1 % 256 == 0) && (a.v_nb1 % 256 == 0);
    const uint32_t xk = (uint32_t)(dma_key * a.k_nb1) | (16u * (uint32_t)(dma_slot ^ dma_key));
    const uint32_t xv = (uint32_t)(dma_key * a.v_nb1) | (16u * (uint32_t)(dma_slot ^ swz_v(dma_key)));
    auto issue = [&](int kt, int stage) {
        uint8_t *ks = smem + stage * kStageBytes;
        uint8_t *vs = ks + kTileBytes;
        const int key0 = kt * kPfBN;
        if (key0 + kPfBN <= a.Skv && nb_fast) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int r0 = key0 + 16 * wave + 4 * j;
                dma16_so(kbase + (int64_t)r0 * a.k_nb1, xk ^ (64u * j), ks + (16 * wave + 4 * j) * 256);
                dma16_so(vbase + (int64_t)r0 * a.v_nb1, xv ^ (32u * (j & 1)), vs + (16 * wave + 4 * j) * 256);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int krow = 16 * wave + 4 * j + dma_key;
                const int kr = min(key0 + krow, a.Skv - 1);
                dma16(kbase + (int64_t)kr * a.k_nb1 + 16 * (dma_slot ^ swz_k(krow)), ks + (16 * wave + 4 * j) * 256);
                dma16(vbase + (int64_t)kr * a.v_nb1 + 16 * (dma_slot ^ swz_v(krow)), vs + (16 * wave + 4 * j) * 256);
            }
        }
    };

    // LDS read geometry.  K operand of dim-step t for keys 32kb + l32:
    // chunk (2t + h) ^ (l32 & 15) of row l32 (+ kb * 32 rows).  V^T operand
    // (transpose reads) of dim tile dt for keys 16ks + 8u + tr_key:
    // chunk (4dt + c0) ^ swz_v(tr_key) of that row.
    uint32_t kaddr[8], vaddr[4];
#pragma unroll
    for (int t = 0; t < 8; t++) kaddr[t] = l32 * 256 + 16 * ((2 * t + h) ^ (l32 & 15));
    {
        const int trg = lane >> 4, tri = lane & 15;
        const int tr_key = 4 * (trg >> 1) + (tri >> 2);
        const int c0 = 2 * (trg & 1) + ((tri & 3) >> 1);
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
            vaddr[dt] = tr_key * 256 + 16 * ((4 * dt + c0) ^ swz_v(tr_key)) + 8 * (tri & 1);
    }

    // One key tile.  STAGE is compile time so every LDS address is a
    // register plus an immediate.
    auto tile = [&](auto stage_c, int kt) {
        constexpr int ST = decltype(stage_c)::value;
        const uint8_t *ks = smem + ST * kStageBytes;
        const uint8_t *vs = ks + kTileBytes;
        const int cl = tc.at(kt);
        const int key0 = kt * kPfBN;
        const bool tail = key0 + kPfBN > a.Skv;
        const bool general = cl == 2 || tail || !lean_ok;

        // S^T = K . Q^T for the two 32-key halves (independent MFMA chains),
        // K operands read two steps ahead of their MFMA.
        f32x16 s[2];
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
            for (int r = 0; r < 16; r++) s[kb][r] = 0.0f;
        u16x8 ka[2][3];   // rolling window: dim-steps t, t+1, t+2
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int kb = 0; kb < 2; kb++) ka[kb][t] = *(const u16x8 *)(ks + kaddr[t] + kb * 32 * 256);
#pragma unroll
        for (int t = 0; t < 8; t++) {
            if (t + 2 < 8) {
#pragma unroll
                for (int kb = 0; kb < 2; kb++)
                    ka[kb][(t + 2) % 3] = *(const u16x8 *)(ks + kaddr[t + 2] + kb * 32 * 256);
            }
#pragma unroll
            for (int kb = 0; kb < 2; kb++) s[kb] = MF::run(__builtin_bit_cast(V8, ka[kb][t % 3]), qb[t], s[kb]);
            __builtin_amdgcn_sched_barrier(0);
        }

        // scores -> probabilities (exp2 domain).  lane: query l32, keys
        // 32kb + 8(r/4) + 4h + r%4.
        // Row max of the tile.  Lean tiles (all-zero mask, full, no softcap,
        // positive scale) take it on the raw scores; general tiles first
        // form x = scale*s (+ softcap) + slope*mask in the exp2 domain, with
        // -inf for masked and out-of-range keys.
        float bmax;
        if (!general) {
            float mx = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < 2; kb++)
#pragma unroll
                for (int r = 0; r < 16; r += 2) mx = __builtin_fmaxf(mx, __builtin_fmaxf(s[kb][r], s[kb][r + 1]));
            bmax = max_pair32(mx) * sl2;
        } else {
#pragma unroll
            for (int kb = 0; kb < 2; kb++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int kbase4 = key0 + 32 * kb + 8 * j + 4 * h;
                    float mv[4] = {0.f, 0.f, 0.f, 0.f};
                    if (cl == 2) {
                        if (kbase4 + 3 < a.Skv) {
                            const u16x4 mw = *(const u16x4 *)(mrow + kbase4);
#pragma unroll
                            for (int i = 0; i < 4; i++) mv[i] = h2f_bits(mw[i]) * slope_l2;
                        } else {
#pragma unroll
                            for (int i = 0; i < 4; i++)
                                mv[i] = (kbase4 + i < a.Skv) ? h2f_bits(mrow[kbase4 + i]) * slope_l2 : -INFINITY;
                        }
                    }
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int r = 4 * j + i;
                        float xv;
                        if (use_softcap) xv = (a.softcap * tanhf(s[kb][r] * sc_in)) * kLog2e + mv[i];
                        else xv = fmaf(s[kb][r], sl2, mv[i]);
                        if (mv[i] == -INFINITY || kbase4 + i >= a.Skv) xv = -INFINITY;
                        s[kb][r] = xv;
                    }
                }
            float mx = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < 2; kb++)
#pragma unroll
                for (int r = 0; r < 16; r++) mx = fmaxf(mx, s[kb][r]);
            bmax = max_pair32(mx);
        }
        // Lazy rescale (one place for both paths, so O is rescaled in
        // place): the reference max m2 is raised only when some row's new
        // max exceeds it by more than 8 (exp2 domain), so p <= 2^8.  O and l
        // always share the reference, so the softmax is unchanged.
        if (__any(bmax > m2 + 8.0f)) {
            const float mnew = fmaxf(m2, bmax);
            const float alpha = (mnew == -INFINITY || m2 == -INFINITY) ? 1.0f : fast_exp2(m2 - mnew);
            m2 = mnew;
            lsum *= alpha;
#pragma unroll
            for (int dt = 0; dt < 4; dt++) o[dt] *= alpha;
        }
        const float mneg = (m2 == -INFINITY) ? 0.0f : -m2;
        if (!general) {
#pragma unroll
            for (int kb = 0; kb < 2; kb++)
#pragma unroll
                for (int r = 0; r < 16; r++) s[kb][r] = fast_exp2(fmaf(s[kb][r], sl2, mneg));
        } else {
#pragma unroll
            for (int kb = 0; kb < 2; kb++)
#pragma unroll
                for (int r = 0; r < 16; r++) s[kb][r] = fast_exp2(s[kb][r] + mneg);   // exp2(-inf) = 0
        }
        // P^T operands of the four 16-key steps ks:
        // k-slot 4u+i <-> key 16ks + 8u + 4h + i = register 8(ks&1) + 4u + i of s[ks>>1].
        // The row sum adds exactly the rounded values the MFMA consumes.
        V8 pb[4];
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const int kb = ks >> 1, rb = 8 * (ks & 1);
            const u16x8 bits = cvt8<T>(f32x4{s[kb][rb], s[kb][rb + 1], s[kb][rb + 2], s[kb][rb + 3]},
                                       f32x4{s[kb][rb + 4], s[kb][rb + 5], s[kb][rb + 6], s[kb][rb + 7]});
            lsum = sum8<T>(bits, lsum);
            pb[ks] = __builtin_bit_cast(V8, bits);
        }
        // O^T += V^T . P^T; the V^T operand comes from two transpose reads of
        // the row-major V tile (keys 16ks + 8u + tr_key, dims 32dt + l32).
        // operands read three MFMAs ahead (rolling window of 4)
        u16x8 va[4];
        // MFMA i = 4ks + dt: consecutive MFMAs go to different accumulators
        auto vread = [&](int i) {
            const int dt = i & 3, ks = i >> 2;
            const u16x4 p0 = lds_read_tr16(vs + vaddr[dt] + (16 * ks) * 256);
            const u16x4 p1 = lds_read_tr16(vs + vaddr[dt] + (16 * ks + 8) * 256);
            return u16x8{p0[0], p0[1], p0[2], p0[3], p1[0], p1[1], p1[2], p1[3]};
        };
#pragma unroll
        for (int i = 0; i < 3; i++) va[i] = vread(i);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            if (i + 3 < 16) va[(i + 3) & 3] = vread(i + 3);
            o[i & 3] = MF::run(__builtin_bit_cast(V8, va[i & 3]), pb[i >> 2], o[i & 3]);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Double-buffered loop over the live tiles.  Per tile: wait for this
    // wave's copies of the tile, one barrier (every wave's copies have
    // landed and every wave is done with the other stage), issue the next
    // tile into the other stage, compute.
    const int n_kt = a.n_kt;
    int kt = tc.next_live(0, n_kt);
    if (kt < n_kt) issue(kt, 0);
    std::integral_constant<int, 0> st0;
    std::integral_constant<int, 1> st1;
    while (kt < n_kt) {
        int kn = tc.next_live(kt + 1, n_kt);
        MXFA_WAIT_VMCNT(0);
        __builtin_amdgcn_s_barrier();
        if (kn < n_kt) issue(kn, 1);
        tile(st0, kt);
        kt = kn;
        if (kt >= n_kt) break;
        kn = tc.next_live(kt + 1, n_kt);
        MXFA_WAIT_VMCNT(0);
        __builtin_amdgcn_s_barrier();
        if (kn < n_kt) issue(kn, 0);
        tile(st1, kt);
        kt = kn;
    }

    lsum = sum_pair32(lsum);
    if (!row_ok) return;
    const float inv = (lsum == 0.0f) ? 0.0f : 1.0f / lsum;
    float *dp = a.dst + (((int64_t)b * a.Sq + qrow) * a.Nh + head) * kD;
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int d0 = 32 * dt + 8 * j + 4 * h;
            *(f32x4 *)(dp + d0) = f32x4{o[dt][4 * j] * inv, o[dt][4 * j + 1] * inv, o[dt][4 * j + 2] * inv,
                                        o[dt][4 * j + 3] * inv};
        }
}

hipError_t launch_mask_classify(const FaArgs &a, int n_planes, uint8_t *classes, hipStream_t stream) {
    dim3 grid(a.n_kt, a.n_qt, n_planes);
    hipLaunchKernelGGL(mask_classify_kernel, grid, dim3(256), 0, stream, a, classes);
    return hipGetLastError();
}

hipError_t launch_fa_prefill(const FaArgs &a, int ktype, hipStream_t stream) {
    dim3 grid(a.n_qt, a.Nh, a.B);
    if (ktype == T_F16) {
        hipLaunchKernelGGL(fa_prefill_kernel<T_F16>, grid, dim3(256), kPfLds, stream, a);
    } else if (ktype == T_BF16) {
        hipLaunchKernelGGL(fa_prefill_kernel<T_BF16>, grid, dim3(256), kPfLds, stream, a);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace mxfa
