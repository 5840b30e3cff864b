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
// keys in 64-key tiles that buffer_load ... lds DMA copies straight from HBM
// into LDS, double-buffered: while tile n is being multiplied, tile n+1 is in
// flight (the first one is issued before Q is loaded).  Workgroups go
// round-robin to the 8 XCDs; the job index is remapped so that each XCD runs
// one contiguous block of jobs ordered (batch, KV head), then q tile (longest
// causal rows first), then the q heads of the GQA group, and the K/V stream
// of a KV head stays in one XCD's L2.
//
//   S^T[64 keys x 32 q] = K_tile . Q^T      v_mfma_f32_32x32x16_{f16,bf16}
//                                            (A = K rows from LDS, B = Q^T
//                                            held in registers all along)
//   online softmax on S^T in fp32 registers: each lane holds one query's
//   column, so the row max/sum need a single cross-lane step (lane ^ 32)
//   O^T[128 x 32 q] += V^T_tile . P^T       same MFMA; P^T comes straight
//                                            from the S^T accumulator layout,
//                                            V^T from the row-major V tile
//                                            through ds_read_b64_tr_b16
//
// Within a tile the two 32-key halves are software-pipelined: the QK MFMAs
// of the second half overlap the softmax of the first, and the PV MFMAs of
// the first overlap the softmax of the second.
//
// LDS tiles (16 KB each, rows of 256 B, 16-byte chunks XOR-swizzled so that
// the DMA writes, the K operand reads and the V transpose reads are
// bank-conflict free):
//   K [64 keys][128 dims]  chunk c of key k at slot c ^ swz_k(k)
//   V [64 keys][128 dims]  chunk c of key k at slot c ^ swz_v(k)
//
// Masks are data, not structure: a classifier pass (mask_classify_kernel)
// labels every (128-query x 64-key) tile of the mask as all -inf (skipped:
// no K/V traffic, no MFMA), all zero (no mask reads), mixed of 0 and -inf
// only (a 64-bit liveness word per row, loaded one tile ahead) or mixed
// (mask read per element).  The causal prefill mask thus costs half the
// work of the dense problem and no per-element mask traffic.

#include <type_traits>

#include "fa_prefill.h"


namespace mxfa {

#ifndef MXFA_PF_LOOK
#define MXFA_PF_LOOK 2
#endif
constexpr int kPfLook = MXFA_PF_LOOK;        // LDS operand reads ahead of their MFMA (1..7)
constexpr int kPfEarlyMaxKt = 4;             // key tiles up to which a tile's copies go out before it
constexpr int kPfWindowEarlyMaxKt = 8;       // the same for the key tiles a structured window spans
static_assert(kPfLook >= 1 && kPfLook <= 7, "operand ring holds 8");

__global__ void __launch_bounds__(256) mask_classify_kernel(const FaArgs a, uint8_t *cls) {
    // One workgroup per (key tile, query tile, mask plane).  Each row of the
    // tile (64 keys = 128 B) is read by 16 lanes with 8-byte loads (the
    // prefill path guarantees 8-byte aligned mask rows).  All 8 loads of a
    // lane are issued before any is looked at: addresses are clamped into
    // the live rows and keys, so no load needs a branch, and rows / keys
    // outside [0, Sq) x [0, Skv) are excluded afterwards by predicates.  The
    // loads go through a buffer resource over the mask plane.
    // Tiles in (plane, query tile, key tile) order, key tile fastest; the
    // 1D grid's workgroups go round-robin to the 8 XCDs, and XCD x takes the
    // x-th contiguous eighth of the tiles: neighbouring key tiles of a row
    // share the 128-byte lines their row pieces straddle (rows whose length
    // is not a multiple of 128 bytes), and fetch them into one L2.
    const uint32_t n_tiles = (uint32_t)a.n_kt * (uint32_t)a.n_qt * (uint32_t)(a.m_ne2 * a.m_ne3);
    const uint32_t L = blockIdx.x, x = L % kXcds, per = n_tiles / kXcds, rem = n_tiles % kXcds;
    const uint32_t T = x * per + min(x, rem) + L / kXcds;
    const int kt = (int)(T % (uint32_t)a.n_kt), qt = (int)((T / (uint32_t)a.n_kt) % (uint32_t)a.n_qt);
    const int plane = (int)(T / ((uint32_t)a.n_kt * (uint32_t)a.n_qt));
    const int m2i = plane % a.m_ne2, m3i = plane / a.m_ne2;
    // (the plane base is uniform; readfirstlane lets the compiler know, so
    // the buffer loads need no waterfall loop.  readfirstlane returns a
    // signed int: each half is taken as uint32_t before it is widened, or a
    // low word >= 2^31 would sign-extend over the high word)
    const uint64_t boff = (uint64_t)((int64_t)m2i * a.m_nb2 + (int64_t)m3i * a.m_nb3);
    const uint64_t bu = (uint64_t)(uintptr_t)a.mask + boff;
    const uint32_t b_lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)bu);
    const uint32_t b_hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(bu >> 32));
    const char *base = (const char *)(uintptr_t)(((uint64_t)b_hi << 32) | (uint64_t)b_lo);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)a.m_plane_bytes, 0x00020000);
    const int q_lo = qt * kPfBM, k_lo = kt * kPfBN;
    const int c4 = threadIdx.x & 15;           // 4-key group within the row
    const int r0 = threadIdx.x >> 4;           // 16 rows per pass
    const int k = k_lo + 4 * c4;
    // a group starting at or past Skv is read at the last live group
    // instead (its values are excluded below); with the mask's ne0 % 4 == 0
    // (host-checked) every group read lies inside its row
    const uint32_t kc = (uint32_t)min(k, (a.Skv - 1) & ~3);
    u16x4 v[kPfBM / 16];
#pragma unroll
    for (int pass = 0; pass < kPfBM / 16; pass++) {
        const uint32_t q = (uint32_t)min(q_lo + r0 + 16 * pass, a.Sq - 1);
        v[pass] = __builtin_bit_cast(u16x4, __builtin_amdgcn_raw_buffer_load_b64(
                                                rs, q * (uint32_t)a.m_nb1 + 2u * kc, 0, 0));
    }
    bool all_ninf = true, all_zero = true, all_bin = true;
    uint32_t live = 0;   // bit 4 pass + i: key k + i of row q_lo + r0 + 16 pass is live (0 past Skv)
#pragma unroll
    for (int pass = 0; pass < kPfBM / 16; pass++) {
        const bool row_ok = q_lo + r0 + 16 * pass < a.Sq;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const bool ok = row_ok & (k + i < a.Skv);
            const bool ninf = v[pass][i] == 0xFC00u, zero = (v[pass][i] & 0x7FFFu) == 0;
            all_ninf &= !ok | ninf;
            all_zero &= !ok | zero;
            all_bin &= !ok | ninf | zero;
            live |= (uint32_t)(k + i < a.Skv && !ninf) << (4 * pass + i);
        }
    }
    // wave votes, then one barrier across the 4 waves
    __shared__ uint32_t votes[4];
    const uint64_t bad_ninf = __ballot(!all_ninf), bad_zero = __ballot(!all_zero), bad_bin = __ballot(!all_bin);
    if ((threadIdx.x & 63) == 0)
        votes[threadIdx.x >> 6] = (bad_ninf ? 1u : 0u) | (bad_zero ? 2u : 0u) | (bad_bin ? 4u : 0u);
    __syncthreads();
    const uint32_t any = votes[0] | votes[1] | votes[2] | votes[3];
    const int c = !(any & 1u) ? 0 : (!(any & 2u) ? 1 : (!(any & 4u) && a.tile_bits ? 3 : 2));
    if (threadIdx.x == 0) cls[((int64_t)plane * a.n_qt + qt) * a.n_kt_pad + kt] = (uint8_t)c;
    if (c == 3) {   // (uniform) the liveness words of the tile's rows
        uint64_t *bits = a.tile_bits + (((int64_t)plane * a.n_qt + qt) * a.n_kt + kt) * kPfBM;
#pragma unroll
        for (int pass = 0; pass < kPfBM / 16; pass++) {
            // the 16 lanes of a row (one DPP row) OR their 4-key nibbles
            // into one word
            const uint32_t nib = (live >> (4 * pass)) & 0xFu;
            const uint32_t lo = or_rows16(c4 < 8 ? nib << (4 * c4) : 0u);
            const uint32_t hi = or_rows16(c4 >= 8 ? nib << (4 * (c4 - 8)) : 0u);
            if (c4 == 0) bits[r0 + 16 * pass] = ((uint64_t)hi << 32) | lo;
        }
    }
}

// CAP: logit softcap on (a per-call constant; its tanh path is compiled only
// into the instances that need it, so it costs the common path no registers).
// SM: structured mask (a.sm_*): tile classes and per-element liveness are
// arithmetic on (query row, key) -- no classifier pass, no mask reads.
// QQ8: Q quantised to Q8_0 on load, as ggml quantises Q for a Q8_0 K (the
// K/V rows of a Q8_0 cache are staged in F16 by q8_stage.hip first).
// SPREAD: the next tile's copies go out one per QK MFMA of the current
// tile (true), or all before the tile, with Q loaded as whole rows (false:
// jobs of few key tiles, chosen in launch_fa_prefill).
template <int T, bool CAP, bool SM, bool QQ8, bool SPREAD = true>
__device__ __forceinline__ void fa_prefill_body(const FaArgs a) {
    using MF = Mfma32<T>;
    using V8 = typename MF::v8;
    static_assert(kD == 128, "kernel is written for D = 128");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    // dense masks' liveness words (class-3 tiles); the Q8_0 instance keeps
    // the mask reads (the host gives Q8_0 calls no words)
    constexpr bool kBits = !SM && !QQ8;

    // (work-item / group ids through the intrinsics: always inline, scalar)
    const int tid = (int)__builtin_amdgcn_workitem_id_x();
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, h = lane >> 5;
    // Job of this workgroup.  Workgroup ids go round-robin to the XCDs; each
    // XCD gets a contiguous block of the job list, which is ordered by
    // (batch, kv head), then by query tile from the last (longest under a
    // causal mask) down, then by q head within the GQA group: the q tiles
    // that share K/V rows run on one XCD and share its L2.
    int qt, head, b;
    bool second = false;   // the CU's second workgroup of the first pair
    pf_job(a, a.n_qt, qt, head, b, second);
    // The two workgroups of a CU's first pair start together, and both would
    // first fetch Q (64 KB in F32) and their first tile.  The second one
    // waits ~2 us (s_sleep 64: 64 x 64 clocks) so that the first pair's
    // fetches do not share one burst: the first workgroup (the long causal
    // row under a causal mask) starts computing sooner, and in later rounds
    // each CU's two workgroups stay out of phase between loading and
    // computing.  Measured: C2 55.0 -> 53.9 us, C4 cross 37.3 -> 34.9 us.
    if (second) __builtin_amdgcn_s_sleep(64);
    const int kvh = head / a.G, bk = b / a.rk3;
    const int qrow = qt * kPfBM + wave * 32 + l32;
    const bool row_ok = qrow < a.Sq;
    const int qrow_c = row_ok ? qrow : a.Sq - 1;
    // Structured mask: the tile's rows together cover keys [lo(first row),
    // hi(last row)) -- key tiles outside are skipped -- and every row sees
    // [lo(last row), hi(first row)) = [sm_in_lo, sm_in_hi): a key tile in
    // there needs no per-element test (class 1); the others test each key
    // against the lane's own row range [row_lo, row_hi).
    int sm_kt_first = 0, sm_kt_end = 0, sm_in_lo = 0, sm_in_hi = 0, row_lo = 0, row_hi = 0;
    if constexpr (SM) {
        const int q_first = qt * kPfBM, q_last = min(q_first + kPfBM, a.Sq) - 1;
        int lo_f, hi_f, lo_l, hi_l;
        sm_row_range(a, b, q_first, lo_f, hi_f);
        sm_row_range(a, b, q_last, lo_l, hi_l);
        sm_kt_first = __builtin_amdgcn_readfirstlane(max(lo_f, 0) / kPfBN);
        sm_kt_end = __builtin_amdgcn_readfirstlane(lo_f < hi_l ? (hi_l + kPfBN - 1) / kPfBN : 0);
        sm_in_lo = __builtin_amdgcn_readfirstlane(lo_l);
        sm_in_hi = __builtin_amdgcn_readfirstlane(hi_f);
        sm_row_range(a, b, qrow_c, row_lo, row_hi);
    }
    const int plane = a.mask ? (b % a.m_ne3) * a.m_ne2 + head % a.m_ne2 : 0;
    TileClasses tc{0u, 0u, !SM && a.tile_class != nullptr};
    if (tc.present) {
        const uint32_t *row = (const uint32_t *)(a.tile_class + ((int64_t)plane * a.n_qt + qt) * a.n_kt_pad);
        const int lane4 = 4 * lane;
        if (lane4 < a.n_kt) tc.w0 = row[lane4 >> 2];
        if (256 + lane4 < a.n_kt) tc.w1 = row[(256 + lane4) >> 2];
    }
    // first live key tile at or after kt (n_kt: none), and a tile's class
    auto next_live = [&](int kt) __attribute__((always_inline)) -> int {
        if constexpr (SM) {
            const int k = max(kt, sm_kt_first);
            return k < sm_kt_end ? k : a.n_kt;
        } else {
            return tc.next_live(kt, a.n_kt);
        }
    };
    auto class_of = [&](int kt) __attribute__((always_inline)) -> int {
        if constexpr (SM) return (kt * kPfBN >= sm_in_lo && kt * kPfBN + kPfBN <= sm_in_hi) ? 1 : 2;
        else return tc.at(kt);
    };
    // Mask rows of this (batch, head) plane through a buffer resource: lane
    // offset qrow * nb1 + 2 * key (32-bit, the host checks the plane size);
    // reads past the plane return zeros, so 4-key groups at the row end need
    // no clamp (keys past Skv are masked anyway).
    const char *mplane = a.mask ? a.mask + (int64_t)(head % a.m_ne2) * a.m_nb2 + (int64_t)(b % a.m_ne3) * a.m_nb3
                                : a.q;
    const __amdgpu_buffer_rsrc_t mrs =
        __builtin_amdgcn_make_buffer_rsrc((void *)mplane, (short)0, a.mask ? (int)a.m_plane_bytes : 0, 0x00020000);
    const uint32_t mrow_off = (uint32_t)qrow_c * (uint32_t)a.m_nb1 + 8u * (uint32_t)h;
    const float slope_l2 = alibi_slope(a, head) * kLog2e;
    const float sl2 = a.scale * kLog2e;
    const float sc_in = a.softcap_in;
    // the lean path takes max over raw scores, valid for a positive scale
    const bool lean_ok = !CAP && sl2 > 0.0f;
    const int n_kt = a.n_kt;

    // K and V rows of this (batch, kv head).
    const char *kbase = a.k + (int64_t)kvh * a.k_nb2 + (int64_t)bk * a.k_nb3;
    const char *vbase = a.v + (int64_t)kvh * a.v_nb2 + (int64_t)bk * a.v_nb3;
    const uint64_t k_avail = (uint64_t)(a.Skv - 1) * (uint64_t)a.k_nb1 + 2 * kD;
    const uint64_t v_avail = (uint64_t)(a.Skv - 1) * (uint64_t)a.v_nb1 + 2 * kD;
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void *)smem);
    const uint32_t k_row = (uint32_t)a.k_nb1, v_row = (uint32_t)a.v_nb1;

    // Tile staging (double buffered, one 64-key tile per stage: K rows at
    // +0, V rows at +16 KB, 256 B per key, 16-byte chunks XOR-swizzled).
    // Wave w copies keys 16w..16w+15 of the tile (four copies of 4 keys x
    // 16 chunks for K and for V): lane -> (key 16w + 4c + lane/16, slot
    // lane%16), the slot holding the swizzled logical chunk.  Each copy goes
    // through a buffer resource based at the wave's first row and sized to
    // the rows that exist, so keys past Skv (the last partial tile, and the
    // look-ahead past the last tile) read as zeros and touch no memory.
    const int dkey = lane >> 4, dslot = lane & 15;
    uint32_t vk[4], vv[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        vk[c] = (uint32_t)(4 * c + dkey) * k_row + 16u * (uint32_t)(dslot ^ swz_k(4 * c + dkey));
        vv[c] = (uint32_t)(4 * c + dkey) * v_row + 16u * (uint32_t)(dslot ^ swz_v(4 * c + dkey));
    }
    // (32-bit row offsets: the host routes here only (batch, kv head)
    // slices whose key tiles lie within 4 GiB of their base; a look-ahead
    // tile at or past n_kt gets an empty resource and reads nothing)
    auto tile_rsrc = [&](const char *base, uint64_t avail, uint32_t row, int kt) __attribute__((always_inline)) {
        const uint32_t off = (uint32_t)(kt * kPfBN + 16 * wave) * row;
        const uint64_t n = kt < a.n_kt && avail > off ? min(avail - off, (uint64_t)0xFFFFFFFFu) : 0;
        return buf_rsrc(base + off, (uint32_t)n);
    };
    auto issue = [&](int kt, auto st_c) __attribute__((always_inline)) {
        constexpr int ST = decltype(st_c)::value;
        const uint32_t l0 = lds0 + ST * kStageBytes + (uint32_t)(16 * wave) * 256u;
        const i32x4 rk = tile_rsrc(kbase, k_avail, k_row, kt);
        const i32x4 rv = tile_rsrc(vbase, v_avail, v_row, kt);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            dma16_buf(rk, vk[c], l0 + 4 * c * 256);
            dma16_buf(rv, vv[c], l0 + kTileBytes + 4 * c * 256);
        }
    };

    // The first live tile's copies go out before Q is loaded: the two
    // fetches share one memory latency.
    int kt = next_live(0);
    if (kt < n_kt) issue(kt, std::integral_constant<int, 0>{});

    // Q^T operand for the 8 dim-steps of 16: Q[qrow][16t + 8h + e], F32
    // rounded to T (round to nearest even, as ggml converts Q to K's
    // vec-dot type), or already stored in T (a.q16).
    V8 qb[8];
    if constexpr (!SPREAD && !QQ8) {
        // Calls of few key tiles are bound by their Q and O bytes: Q comes
        // in as whole rows (2 F32 rows or 4 16-bit rows per 16-byte load,
        // whole 128-byte lines), goes through the wave's 8 KB of the free
        // stage (16-byte chunk k of a row at slot k ^ (row & 15)) and is
        // read back in the operand layout.  Rows past Sq load the last row;
        // their outputs are not stored.
        const char *qhead = a.q + (int64_t)head * a.q_nb2 + (int64_t)b * a.q_nb3;
        const int q0w = qt * kPfBM + wave * 32;
        uint8_t *qst = smem + kStageBytes + wave * 8192;
        if (a.q16) {
            u16x8 xr[8];   // load i: rows 4i + lane/16, chunk lane%16
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int row = min(q0w + 4 * i + (lane >> 4), a.Sq - 1);
                xr[i] = *(const u16x8 *)(qhead + (int64_t)row * a.q_nb1 + 16 * (lane & 15));
            }
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int rl = 4 * i + (lane >> 4);
                *(u16x8 *)(qst + rl * 256 + 16 * ((lane & 15) ^ (rl & 15))) = xr[i];
            }
        } else {
            f32x4 xq[16];  // load i: rows 2i + lane/32, dims 4(lane%32) .. +3
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int row = min(q0w + 2 * i + (lane >> 5), a.Sq - 1);
                xq[i] = *(const f32x4 *)(qhead + (int64_t)row * a.q_nb1 + 16 * (lane & 31));
            }
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int rl = 2 * i + (lane >> 5), c4 = lane & 31;
                const u16x8 hv = cvt8<T>(xq[i], xq[i]);
                *(u16x4 *)(qst + rl * 256 + 16 * ((c4 >> 1) ^ (rl & 15)) + 8 * (c4 & 1)) =
                    u16x4{hv[0], hv[1], hv[2], hv[3]};
            }
        }
#pragma unroll
        for (int t = 0; t < 8; t++)
            qb[t] = __builtin_bit_cast(V8, *(const u16x8 *)(qst + l32 * 256 + 16 * ((2 * t + h) ^ (l32 & 15))));
        // (every wave's staging reads are done before the first tile's
        // barrier, after which the stage takes the next tile's copies)
        MXFA_WAIT_LGKMCNT0();
    } else {
        const char *qrow_p = a.q + (int64_t)qrow_c * a.q_nb1 + (int64_t)head * a.q_nb2 + (int64_t)b * a.q_nb3;
        if (a.q16) {
            const uint16_t *qh = (const uint16_t *)qrow_p;
#pragma unroll
            for (int t = 0; t < 8; t++) {
                u16x8 x = {0, 0, 0, 0, 0, 0, 0, 0};
                if (row_ok) x = *(const u16x8 *)(qh + 16 * t + 8 * h);
                qb[t] = __builtin_bit_cast(V8, x);
            }
        } else if constexpr (QQ8) {
            // Q8_0 block bb = dims 32bb .. 32bb+31 = dim-steps 2bb, 2bb+1 of
            // both halves (this lane and lane ^ 32, the same query row):
            // d = fp16(amax / 127), q = rint(x * 127 / amax), operand
            // T(q * d), the product exact in F32
            const float *qp = (const float *)qrow_p;
#pragma unroll
            for (int bb = 0; bb < 4; bb++) {
                f32x4 x[4];
#pragma unroll
                for (int i = 0; i < 4; i++) x[i] = f32x4{0.f, 0.f, 0.f, 0.f};
                if (row_ok) {
#pragma unroll
                    for (int i = 0; i < 4; i++) x[i] = *(const f32x4 *)(qp + 32 * bb + 16 * (i >> 1) + 8 * h + 4 * (i & 1));
                }
                float amax = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int e = 0; e < 4; e++) amax = fmaxf(amax, fabsf(x[i][e]));
                amax = fmaxf(amax, __shfl_xor(amax, 32));
                const float d = (float)(_Float16)(amax / 127.0f);
                const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int e = 0; e < 4; e++) x[i][e] = (float)(int)__builtin_rintf(x[i][e] * id) * d;
                qb[2 * bb] = __builtin_bit_cast(V8, cvt8<T>(x[0], x[1]));
                qb[2 * bb + 1] = __builtin_bit_cast(V8, cvt8<T>(x[2], x[3]));
            }
        } else {
            const float *qp = (const float *)qrow_p;
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
    }

    // LDS operand addresses.  QK: K operand of dim-step t for key l32 of a
    // half: chunk (2t + h) ^ swz_k(l32) of row l32.  PV: V^T operand of dim
    // tile dt for the 16-key step kk (keys 16kk + 8u + tr_key of a half):
    // chunk (4dt + c0) ^ swz_v(tr_key) of that row, two transpose reads.
    uint32_t kaddr[8], vaddr[4];
#pragma unroll
    for (int t = 0; t < 8; t++) kaddr[t] = l32 * 256 + 16 * ((2 * t + h) ^ swz_k(l32));
    {
        const int trg = lane >> 4, tri = lane & 15;
        const int tr_key = 4 * (trg >> 1) + (tri >> 2);
        const int c0 = 2 * (trg & 1) + ((tri >> 1) & 1);
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
            vaddr[dt] = tr_key * 256 + 16 * ((4 * dt + c0) ^ swz_v(tr_key)) + 8 * (tri & 1);
    }
    // K operand t of half p; V operand i = 4kk + dt of half p
    auto kread = [&](auto st_c, int p, int t) __attribute__((always_inline)) -> u16x8 {
        constexpr int ST = decltype(st_c)::value;
        return *(const u16x8 *)(smem + ST * kStageBytes + p * 32 * 256 + kaddr[t]);
    };
    auto vread = [&](auto st_c, int p, int i) __attribute__((always_inline)) -> u16x8 {
        constexpr int ST = decltype(st_c)::value;
        const int dt = i & 3, kk = i >> 2;
        const uint8_t *q = smem + ST * kStageBytes + kTileBytes + (32 * p + 16 * kk) * 256 + vaddr[dt];
        const u16x4 p0 = lds_read_tr16(q);
        const u16x4 p1 = lds_read_tr16(q + 8 * 256);
        return u16x8{p0[0], p0[1], p0[2], p0[3], p1[0], p1[1], p1[2], p1[3]};
    };

    f32x16 o[4];
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[dt][r] = 0.0f;
    float m2 = -INFINITY, lsum = 0.0f;

    // General tiles (mixed mask, tail, softcap, non-positive scale): the
    // raw scores of a half become x = scale*s (+softcap) + slope*mask in the
    // exp2 domain, -inf for masked keys and keys past Skv (lane: query l32,
    // keys 8(r/4) + 4h + r%4 of the half).  The mask is read for every
    // general tile: on a tile of class 1 it is all zero, and without a mask
    // the resource is empty (reads return zero), so no branch is needed.
    auto general_x = [&](f32x16 &sc, int key0, int cl, uint32_t bits) __attribute__((always_inline)) {
        if constexpr (SM) {
            // live keys 8j + i of [lo_rel, hi_rel) (row_hi <= Skv); the
            // zero mask value keeps the arithmetic of the dense path
            const int lo_rel = row_lo - key0 - 4 * h, hi_rel = row_hi - key0 - 4 * h;
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = 4 * j + i, off = 8 * j + i;
                    float x;
                    if constexpr (CAP) x = (a.softcap * fast_tanh(sc[r] * sc_in)) * kLog2e + 0.0f;
                    else x = fmaf(sc[r], sl2, 0.0f);
                    sc[r] = (off >= lo_rel && off < hi_rel) ? x : -INFINITY;
                }
            return;
        }
        if (kBits && cl == 3) {
            // a mask of 0 and -inf only: liveness from the tile's word for
            // this row (bits of this half's keys 8j + 4h + i; 0 past Skv)
            // and the arithmetic of a zero mask value
            const uint32_t w = bits >> (4 * h);
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = 4 * j + i;
                    float x;
                    if constexpr (CAP) x = (a.softcap * fast_tanh(sc[r] * sc_in)) * kLog2e + 0.0f;
                    else x = fmaf(sc[r], sl2, 0.0f);
                    sc[r] = ((w >> (8 * j + i)) & 1u) ? x : -INFINITY;
                }
            return;
        }
        const int kmax = a.Skv - key0 - 4 * h;   // keys 8j + i >= kmax lie past Skv
        // (the four mask words go out together: one memory round trip)
        u16x4 mw4[4];
#pragma unroll
        for (int j = 0; j < 4; j++)
            mw4[j] = __builtin_bit_cast(
                u16x4, __builtin_amdgcn_raw_buffer_load_b64(mrs, mrow_off + 2u * (uint32_t)key0 + 16u * j, 0, 0));
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const u16x4 mw = mw4[j];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = 4 * j + i;
                const float mv = h2f_bits(mw[i]) * slope_l2;
                float x;
                if constexpr (CAP) x = (a.softcap * fast_tanh(sc[r] * sc_in)) * kLog2e + mv;
                else x = fmaf(sc[r], sl2, mv);
                sc[r] = (mv == -INFINITY || 8 * j + i >= kmax) ? -INFINITY : x;
            }
        }
    };
    // probabilities of pair u (registers 2u, 2u+1) of a half, packed into
    // the P^T operand: k-slot 4u' + i <-> key 16kk + 8u' + 4h + i =
    // register 8kk + 4u' + i, i.e. operand kk holds registers 8kk..8kk+7.
    // bf16: pl receives the lo parts (bf16_lo), which a second PV MFMA adds.
    constexpr bool kLo = T == T_BF16;
    auto pair = [&](const f32x16 &sc, int u, float g, float mneg, u16x8 (&pw)[2], u16x8 (&pl)[2])
                    __attribute__((always_inline)) {
        const float p0 = fast_exp2(fmaf(sc[2 * u], g, mneg));
        const float p1 = fast_exp2(fmaf(sc[2 * u + 1], g, mneg));
        const uint16_t h0 = Mfma16<T>::from_f32(p0), h1 = Mfma16<T>::from_f32(p1);
        pw[u >> 2][2 * (u & 3)] = h0;
        pw[u >> 2][2 * (u & 3) + 1] = h1;
        if constexpr (kLo) {
            pl[u >> 2][2 * (u & 3)] = bf16_lo(p0, h0);
            pl[u >> 2][2 * (u & 3) + 1] = bf16_lo(p1, h1);
        }
    };
    // the denominator sums exactly the weights the PV product uses
    auto psum = [&](const u16x8 (&pw)[2], const u16x8 (&pl)[2]) __attribute__((always_inline)) -> float {
        float l = sum8<T>(pw[1], sum8<T>(pw[0], 0.0f));
        if constexpr (kLo) l = sum8<T>(pl[1], sum8<T>(pl[0], l));
        return l;
    };
    auto half_max = [&](const f32x16 &sc) __attribute__((always_inline)) {
        return fmaxf(fmaxf(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])),
                           fmaxf(fmaxf(sc[4], sc[5]), fmaxf(sc[6], sc[7]))),
                     fmaxf(fmaxf(fmaxf(sc[8], sc[9]), fmaxf(sc[10], sc[11])),
                           fmaxf(fmaxf(sc[12], sc[13]), fmaxf(sc[14], sc[15]))));
    };

    // One 64-key tile, as two 32-key halves a (keys 0..31) and b:
    //   R1  QK a                         (matrix cores)
    //   R2  QK b       | softmax of a, speculative with the current
    //                    reference max m2 (vector ALUs, interleaved)
    //   R3  max of b; if some row's tile max exceeds m2 by more than 8
    //       (exp2 domain), raise m2, rescale O and l, redo a  (rare)
    //   R4  PV a       | softmax of b
    //   R5  PV b
    // The code is laid out in issue order; sched_barrier fences keep it.
    // The tile's 32 MFMA operands (K of half a and b, then V^T of half a and
    // b) are read from LDS in one sequence kPfLook items ahead of the MFMA
    // that consumes them (a ring of 8 operand registers).
    //
    // kn is the next live tile (n_kt: none), whose copies into the other
    // stage NST go out one per QK MFMA of half a (SPREAD): spread so, their
    // issue (~40 cycles each, with the LDS address set per copy) hides under
    // the matrix cores instead of holding up the tile's first MFMAs.
    auto tile = [&](auto st_c, int kt, auto nst_c, int kn, uint64_t tbits) __attribute__((always_inline)) {
        constexpr int NST = decltype(nst_c)::value;
        const bool do_issue = SPREAD && kn < n_kt;   // uniform
        const uint32_t nl0 = lds0 + NST * kStageBytes + (uint32_t)(16 * wave) * 256u;
        i32x4 nrk = {0, 0, 0, 0}, nrv = {0, 0, 0, 0};
        if (do_issue) {
            nrk = tile_rsrc(kbase, k_avail, k_row, kn);
            nrv = tile_rsrc(vbase, v_avail, v_row, kn);
        }
        const int cl = __builtin_amdgcn_readfirstlane(class_of(kt));
        const int key0 = kt * kPfBN;
        const bool general =
            __builtin_amdgcn_readfirstlane((int)(cl >= 2 || key0 + kPfBN > a.Skv || !lean_ok)) != 0;
        const float g = general ? 1.0f : sl2;   // wave-uniform
        f32x16 sa, sb;
        u16x8 op[8];
        // operand n of the tile: K(a) 0..7, K(b) 8..15, V^T(a) 16..23, V^T(b) 24..31
        auto fetch = [&](int n) __attribute__((always_inline)) {
            if (n < 8) op[n & 7] = kread(st_c, 0, n);
            else if (n < 16) op[n & 7] = kread(st_c, 1, n - 8);
            else if (n < 24) op[n & 7] = vread(st_c, 0, n - 16);
            else if (n < 32) op[n & 7] = vread(st_c, 1, n - 24);
        };

        // ---- R1: QK a ----
#pragma unroll
        for (int n = 0; n < kPfLook; n++) fetch(n);
#pragma unroll
        for (int t = 0; t < 8; t++) {
            fetch(t + kPfLook);
            sa = MF::run(__builtin_bit_cast(V8, op[t & 7]), qb[t], t == 0 ? f32x16{} : sa);
            if (do_issue) {   // the next tile's copy c = t/2 of its K rows (t even) or V rows
                if (t & 1) dma16_buf(nrv, vv[t >> 1], nl0 + kTileBytes + 4 * (t >> 1) * 256);
                else dma16_buf(nrk, vk[t >> 1], nl0 + 4 * (t >> 1) * 256);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (general) general_x(sa, key0, cl, (uint32_t)tbits);
        __builtin_amdgcn_sched_barrier(0);

        // ---- R2: QK b | softmax a (speculative) ----
        const float mneg0 = (m2 == -INFINITY) ? 0.0f : -m2;
        float mxa = 0.0f;
        u16x8 pa[2], pb[2], pal[2], pbl[2];
#pragma unroll
        for (int t = 0; t < 8; t++) {
            fetch(8 + t + kPfLook);
            sb = MF::run(__builtin_bit_cast(V8, op[(8 + t) & 7]), qb[t], t == 0 ? f32x16{} : sb);
            if (t == 0) mxa = half_max(sa);
            else pair(sa, t - 1, g, mneg0, pa, pal);
            if (t == 7) pair(sa, 7, g, mneg0, pa, pal);
            __builtin_amdgcn_sched_barrier(0);
        }
        float la = psum(pa, pal);
        // keep the speculative softmax here, overlapped with QK b (it is
        // redone on the rare path, so it would otherwise sink past R3)
        asm volatile("" ::"v"(pa[0]), "v"(pa[1]), "v"(la), "v"(mxa));
        if constexpr (kLo) asm volatile("" ::"v"(pal[0]), "v"(pal[1]));
        if (general) general_x(sb, key0 + 32, cl, (uint32_t)(tbits >> 32));
        __builtin_amdgcn_sched_barrier(0);

        // ---- R3: tile max, reference update (rare rescale) ----
        const float bmax = max_pair32(fmaxf(mxa, half_max(sb))) * g;
        const bool any_need = __builtin_amdgcn_ballot_w64(bmax > m2 + 8.0f) != 0;   // wave-uniform
        if (any_need) {
            const float mnew = fmaxf(m2, bmax);
            const float alpha = (m2 == -INFINITY) ? 1.0f : fast_exp2(m2 - mnew);
            m2 = mnew;
            lsum *= alpha;
#pragma unroll
            for (int dt = 0; dt < 4; dt++) o[dt] *= alpha;
            const float mn = (m2 == -INFINITY) ? 0.0f : -m2;
#pragma unroll
            for (int u = 0; u < 8; u++) pair(sa, u, g, mn, pa, pal);
            la = psum(pa, pal);
        }
        const float mneg = (m2 == -INFINITY) ? 0.0f : -m2;
        __builtin_amdgcn_sched_barrier(0);

        // ---- R4: PV a | softmax b ----
#pragma unroll
        for (int i = 0; i < 8; i++) {
            fetch(16 + i + kPfLook);
            o[i & 3] = MF::run(__builtin_bit_cast(V8, op[(16 + i) & 7]), __builtin_bit_cast(V8, pa[i >> 2]), o[i & 3]);
            if constexpr (kLo)
                o[i & 3] = MF::run(__builtin_bit_cast(V8, op[(16 + i) & 7]), __builtin_bit_cast(V8, pal[i >> 2]),
                                   o[i & 3]);
            pair(sb, i, g, mneg, pb, pbl);
            __builtin_amdgcn_sched_barrier(0);
        }
        const float lb = psum(pb, pbl);
        __builtin_amdgcn_sched_barrier(0);

        // ---- R5: PV b ----
#pragma unroll
        for (int i = 0; i < 8; i++) {
            fetch(24 + i + kPfLook);
            o[i & 3] = MF::run(__builtin_bit_cast(V8, op[(24 + i) & 7]), __builtin_bit_cast(V8, pb[i >> 2]), o[i & 3]);
            if constexpr (kLo)
                o[i & 3] = MF::run(__builtin_bit_cast(V8, op[(24 + i) & 7]), __builtin_bit_cast(V8, pbl[i >> 2]),
                                   o[i & 3]);
            __builtin_amdgcn_sched_barrier(0);
        }
        lsum += la + lb;
    };

    // Double-buffered loop over the live tiles.  Per tile: wait for this
    // wave's copies of the tile, one barrier (every wave's copies have
    // landed and every wave is done with the other stage), compute, with the
    // next live tile's copies into the other stage spread over the first
    // MFMAs (SPREAD) or issued before them.  Measured, spread against
    // before: C2 52.5 against 53.8 us, C4 self 157 against 160, and C4
    // cross (4 tiles per job, bound by memory latency) 35.3 against 34.6,
    // so calls of few key tiles take the other instance.  (No divergent
    // early exits anywhere: they would put the tile loop under divergent
    // control flow.)
    // A class-3 tile's liveness word of this lane's row: loaded one tile
    // ahead, right after the tile's barrier, so that it lands with the next
    // tile's copies (the wait at that tile's top covers both).
    const uint64_t *brow = (kBits && tc.present && a.tile_bits)
                               ? a.tile_bits + ((int64_t)plane * a.n_qt + qt) * a.n_kt * kPfBM + wave * 32 + l32
                               : nullptr;
    auto load_bits = [&](int k) __attribute__((always_inline)) -> uint64_t {
        if (!kBits || brow == nullptr || k >= n_kt || __builtin_amdgcn_readfirstlane(class_of(k)) != 3) return 0;
        return brow[(int64_t)k * kPfBM];
    };
    std::integral_constant<int, 0> st0;
    std::integral_constant<int, 1> st1;
    int ofree = 1;   // the stage no tile still reads at the end
    uint64_t cbits = load_bits(kt);
    while (kt < n_kt) {
        int kn = next_live(kt + 1);
        MXFA_WAIT_VMCNT(0);
        __builtin_amdgcn_s_barrier();
        if (!SPREAD && kn < n_kt) issue(kn, st1);
        uint64_t nbits = load_bits(kn);
        tile(st0, kt, st1, kn, cbits);
        cbits = nbits;
        ofree = 1;
        kt = kn;
        if (kt >= n_kt) break;
        kn = next_live(kt + 1);
        MXFA_WAIT_VMCNT(0);
        __builtin_amdgcn_s_barrier();
        if (!SPREAD && kn < n_kt) issue(kn, st0);
        nbits = load_bits(kn);
        tile(st1, kt, st0, kn, cbits);
        cbits = nbits;
        ofree = 0;
        kt = kn;
    }

    lsum = sum_pair32(lsum);
    const float inv = (lsum == 0.0f) ? 0.0f : 1.0f / lsum;
    // O leaves as whole rows through the stage the last tile did not read
    // (every wave was past its last read at that tile's barrier, and no
    // copy has gone into it since; with no live tile, each wave's 8 KB is
    // the Q staging it has already read back): each wave stages its 32
    // rows in its own 8 KB, dims 0..63 then 64..127, 16-byte chunk k of a
    // row at slot k ^ (row & 15), and stores 4 half rows per 16-byte store
    // (whole 128-byte lines, where the MFMA layout's direct stores touched
    // 32 rows per store).  No barrier: a wave that ends early does not wait
    // for the others.  Measured against the direct stores: C4 cross 32.9
    // against 35.3 us, C4 self 157.5 against 159.6, C2 53.0 against 53.3.
    {
        uint8_t *ost = smem + ofree * kStageBytes + wave * 8192;
        const int q0w = qt * kPfBM + wave * 32;
        float *drow = a.dst + ((int64_t)b * a.Sq * a.Nh + head) * kD;   // + q * Nh * kD per row
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
#pragma unroll
            for (int dt = 0; dt < 2; dt++)
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    const int k = 8 * dt + 2 * jj + h;   // dims 64hh + 4k .. +3
                    const f32x16 &od = o[2 * hh + dt];
                    *(f32x4 *)(ost + l32 * 256 + 16 * (k ^ (l32 & 15))) =
                        f32x4{od[4 * jj] * inv, od[4 * jj + 1] * inv, od[4 * jj + 2] * inv, od[4 * jj + 3] * inv};
                }
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int rl = 4 * i + (lane >> 4), c = lane & 15;
                const f32x4 v = *(const f32x4 *)(ost + rl * 256 + 16 * (c ^ (rl & 15)));
                if (q0w + rl < a.Sq) *(f32x4 *)(drow + (int64_t)(q0w + rl) * a.Nh * kD + 64 * hh + 4 * c) = v;
            }
        }
    }
}

template <int T, bool CAP, bool SM, bool SPREAD>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
fa_prefill_kernel(const FaArgs a) {
    fa_prefill_body<T, CAP, SM, false, SPREAD>(a);
}

// Prefill over a Q8_0 cache: K/V rows staged in F16, Q quantised on load.
template <bool CAP, bool SM>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
fa_prefill_q8q_kernel(const FaArgs a) {
    fa_prefill_body<T_F16, CAP, SM, true>(a);
}

hipError_t launch_mask_classify(const FaArgs &a, int n_planes, uint8_t *classes, hipStream_t stream) {
    // (1D over every tile of the n_planes = m_ne2 * m_ne3 mask planes)
    if (n_planes != a.m_ne2 * a.m_ne3) return hipErrorInvalidValue;
    dim3 grid((uint32_t)a.n_kt * (uint32_t)a.n_qt * (uint32_t)n_planes);
    hipLaunchKernelGGL(mask_classify_kernel, grid, dim3(256), 0, stream, a, classes);
    return hipGetLastError();
}

hipError_t launch_fa_prefill(const FaArgs &a, int ktype, hipStream_t stream) {
    dim3 grid((uint32_t)a.n_qt * (uint32_t)a.Nh * (uint32_t)a.B);
    const bool cap = a.softcap != 0.0f, sm = a.sm_flags != 0;
    // Jobs of few key tiles take the instance that issues a tile's copies
    // before it and loads Q as whole rows: calls of at most 4 key tiles,
    // and structured windows whose 128 rows see at most 8 tiles (2 window
    // + 128 keys, causal: window + 128, +1 tile for the alignment).
    // Measured on the DiT window layer (window 128, 7 tiles): c4swm 50.5
    // against 52.3 us, c4swm8 45.8 against 47.9.
    bool spread = a.n_kt > kPfEarlyMaxKt;
    if (a.sm_flags & kSmWindow) {
        const int64_t span = (a.sm_flags & kSmCausal) ? (int64_t)a.sm_window + kPfBM
                                                      : 2 * (int64_t)a.sm_window + kPfBM;
        if ((span + kPfBN - 1) / kPfBN + 1 <= kPfWindowEarlyMaxKt) spread = false;
    }
#define MXFA_PF(TT, C, S)                                                                                    \
    do {                                                                                                     \
        if (spread) hipLaunchKernelGGL((fa_prefill_kernel<TT, C, S, true>), grid, dim3(256), kPfLds, stream, a); \
        else hipLaunchKernelGGL((fa_prefill_kernel<TT, C, S, false>), grid, dim3(256), kPfLds, stream, a);       \
    } while (0)
    if (ktype == T_F16) {
        if (sm) { if (cap) MXFA_PF(T_F16, true, true); else MXFA_PF(T_F16, false, true); }
        else { if (cap) MXFA_PF(T_F16, true, false); else MXFA_PF(T_F16, false, false); }
    } else if (ktype == T_BF16) {
        if (sm) { if (cap) MXFA_PF(T_BF16, true, true); else MXFA_PF(T_BF16, false, true); }
        else { if (cap) MXFA_PF(T_BF16, true, false); else MXFA_PF(T_BF16, false, false); }
    } else if (ktype == T_Q8_0) {
#define MXFA_PFQ(C, S) hipLaunchKernelGGL((fa_prefill_q8q_kernel<C, S>), grid, dim3(256), kPfLds, stream, a)
        if (sm) { if (cap) MXFA_PFQ(true, true); else MXFA_PFQ(false, true); }
        else { if (cap) MXFA_PFQ(true, false); else MXFA_PFQ(false, false); }
#undef MXFA_PFQ
    } else {
        return hipErrorInvalidValue;
    }
#undef MXFA_PF
    return hipGetLastError();
}

}  // namespace mxfa
