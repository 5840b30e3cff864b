// fa_wide.hip -- MFMA flash attention with 48 queries per wave (gfx950).
//
// Serves the DiT's calls with F16 K/V: the self-attention of the odd layers
// (src/dit-graph.h:227-231, no mask; the CFG pair as batch 2) and the
// cross-attention over the text encoder's keys (src/dit-graph.h:348-352,
// a dense padding mask over at most 4 key tiles); the host routes them here
// (mxfa_api.cpp, make_plan).  One workgroup = 4 waves = 192 consecutive queries
// of one (batch, q head); each wave owns 48 queries as three 16-query
// blocks.  Keys come in the same 64-key K/V tiles as fa_mfma.hip (DMA into
// LDS, double-buffered, XOR-swizzled rows), but every LDS operand now feeds
// three MFMAs instead of one:
//
//   S^T[16 keys x 16 q] = K . Q^T     v_mfma_f32_16x16x32_f16
//                                      (A = 16 K rows x 32 dims from LDS,
//                                      one read for the 3 query blocks;
//                                      B = Q^T in registers all along)
//   O^T[16 dims x 16 q] += V^T . P^T  same MFMA, 32 keys per step (A = V^T
//                                      by two ds_read_b64_tr_b16, one read
//                                      for the 3 query blocks; B = P^T
//                                      straight from the S^T accumulators)
//
// Per 64-key tile a wave reads the same 32 KB of LDS operands as the
// 32-query kernel for 1.5x the matrix work, and a 3000-token DiT call is
// 16 query tiles (512 workgroups: one round on 256 CUs at two workgroups
// per CU) instead of 24 (768: a second round with one workgroup per CU).
//
// Lane l = 16 g + n holds, per query block, query n and keys 4g..4g+3 of
// each 16-key block, so a query's scores are spread over lanes n, n+16,
// n+32, n+48.  The online softmax keeps one reference max per (lane, query
// block), equal across those four lanes; the lazy rescale needs no
// cross-lane step in the common case (a wave-wide ballot of "some lane's own
// maximum exceeds the reference by more than 8"), and takes the row maximum
// over the four lanes only when it raises the reference.

#include "fa_prefill.h"

namespace mxfa {

// Mask modes: none (the general path only bounds keys by Skv), a dense
// mask (tile classes from the classifier, per-element mask reads in mixed
// tiles) or a structured one (a.sm_*: classes and liveness by arithmetic).
enum : int { kWideNone = 0, kWideDense = 1, kWideSm = 2 };

template <int T, int MODE>
__device__ __forceinline__ void fa_wide_body(const FaArgs a) {
    constexpr bool MASKED = MODE == kWideDense, SM = MODE == kWideSm;
    using MF = Mfma16<T>;
    using V8 = typename MF::v8;
    static_assert(kD == 128, "kernel is written for D = 128");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    // (F16 only: BF16 calls stay on fa_mfma.hip, whose P hi/lo pair would
    // not fit this kernel's registers)
    static_assert(T == T_F16, "F16 K/V only");

    const int tid = (int)__builtin_amdgcn_workitem_id_x();
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n16 = lane & 15, g = lane >> 4;
    int qt, head, b;
    bool second = false;
    pf_job(a, a.n_qt_w, qt, head, b, second);
    // (the staggered start of fa_mfma.hip: the CU's second workgroup of the
    // first pair waits ~2 us so that the two do not fetch in one burst)
    if (second) __builtin_amdgcn_s_sleep(64);
    const int kvh = head / a.G, bk = b / a.rk3;
    const int q0w = qt * kPfWideBM + wave * 48;   // first query of this wave
    int qrow_c[3];                                // lane's query of block qb (rows past Sq: the last row)
#pragma unroll
    for (int qb = 0; qb < 3; qb++) qrow_c[qb] = min(q0w + 16 * qb + n16, a.Sq - 1);

    // Tile classes: the classifier labels 128-query tiles; this job's 192
    // rows lie within two of them (rows r0 .. r1), whose union class is
    // exact or conservative (mixed).
    const int plane = a.mask ? (b % a.m_ne3) * a.m_ne2 + head % a.m_ne2 : 0;
    const int r0 = qt * kPfWideBM / kPfBM;
    const int r1 = min((qt * kPfWideBM + kPfWideBM - 1) / kPfBM, (a.Sq - 1) / kPfBM);
    TileClasses tc{0u, 0u, MASKED && a.tile_class != nullptr};
    if (tc.present) {
        const uint32_t *row0 = (const uint32_t *)(a.tile_class + ((int64_t)plane * a.n_qt + r0) * a.n_kt_pad);
        const uint32_t *row1 = (const uint32_t *)(a.tile_class + ((int64_t)plane * a.n_qt + r1) * a.n_kt_pad);
        const int lane4 = 4 * lane;
        if (lane4 < a.n_kt) tc.w0 = class_union4(row0[lane], row1[lane]);
        if (256 + lane4 < a.n_kt) tc.w1 = class_union4(row0[64 + lane], row1[64 + lane]);
    }
    // Mask rows of this (batch, head) plane through a buffer resource (as
    // in fa_mfma.hip): lane offset qrow * nb1 + 2 * (4g + key), reads past
    // the plane return zeros.
    const char *mplane = a.mask ? a.mask + (int64_t)(head % a.m_ne2) * a.m_nb2 + (int64_t)(b % a.m_ne3) * a.m_nb3
                                : a.q;
    const __amdgpu_buffer_rsrc_t mrs =
        __builtin_amdgcn_make_buffer_rsrc((void *)mplane, (short)0, a.mask ? (int)a.m_plane_bytes : 0, 0x00020000);
    uint32_t mrow_off[3] = {0u, 0u, 0u};
    float slope_l2 = 0.0f;
    if constexpr (MASKED) {
#pragma unroll
        for (int qb = 0; qb < 3; qb++) mrow_off[qb] = (uint32_t)qrow_c[qb] * (uint32_t)a.m_nb1 + 8u * (uint32_t)g;
        slope_l2 = alibi_slope(a, head) * kLog2e;
    }
    // Structured mask: live keys of row q are [lo(q), hi(q)), both
    // non-decreasing in q (sm_row_range, from the job's uniform pos0 and
    // length).  The job's tile range and classes are taken over the rows of
    // the two 128-query tiles r0, r1 that a dense mask's classes unite, so
    // that a structured call and the same call with the dense mask take the
    // same tiles down the same paths (bit-identical outputs): tiles outside
    // [lo(first), hi(last)) are skipped, tiles inside [lo(last), hi(first))
    // need no per-element test.
    int sm_p0 = 0, sm_hi = a.Skv, sm_kt_first = 0, sm_kt_end = 0, sm_in_lo = 0, sm_in_hi = 0;
    auto row_range = [&](int q, int &lo, int &hi) __attribute__((always_inline)) {
        const int p = sm_p0 + q;
        lo = 0;
        hi = sm_hi;
        if (a.sm_flags & kSmCausal) hi = min(hi, p + 1);
        if (a.sm_flags & kSmWindow) {
            lo = max(lo, p - a.sm_window);
            hi = min(hi, p + a.sm_window + 1);
        }
    };
    if constexpr (SM) {
        // (pos0 and the batch's length, read and clamped as sm_row_range does)
        sm_p0 = a.sm_pos0;
        if (a.sm_pos0_dev) {
            const int d = sm_dev_load(a.sm_pos0_dev);
            sm_p0 = d < 0 ? 0 : (d > (1 << 30) - 1 ? (1 << 30) - 1 : d);
        }
        sm_p0 = __builtin_amdgcn_readfirstlane(sm_p0);
        int len = a.Skv;
        if (a.sm_flags & kSmLengths) {
            len = a.sm_len[b % a.sm_nlen];
            if (a.sm_len_dev) len = sm_dev_load(a.sm_len_dev + b % a.sm_nlen);
            len = len < 0 ? 0 : len;
        }
        sm_hi = __builtin_amdgcn_readfirstlane(min(a.Skv, len));
        const int q_first = r0 * kPfBM, q_last = min((r1 + 1) * kPfBM, a.Sq) - 1;
        int lo_f, hi_f, lo_l, hi_l;
        row_range(q_first, lo_f, hi_f);
        row_range(q_last, lo_l, hi_l);
        sm_kt_first = __builtin_amdgcn_readfirstlane(max(lo_f, 0) / kPfBN);
        sm_kt_end = __builtin_amdgcn_readfirstlane(lo_f < hi_l ? (hi_l + kPfBN - 1) / kPfBN : 0);
        sm_in_lo = __builtin_amdgcn_readfirstlane(lo_l);
        sm_in_hi = __builtin_amdgcn_readfirstlane(hi_f);
    }
    const float sl2 = a.scale * kLog2e;
    const bool lean_ok = sl2 > 0.0f;   // the lean path takes max over raw scores
    const int n_kt = a.n_kt;

    // K and V rows of this (batch, kv head); tile copies exactly as in
    // fa_mfma.hip (wave w copies keys 16w..16w+15 of a tile, four 16-byte
    // copies of K rows and four of V rows, through a buffer resource sized
    // to the rows that exist).
    const char *kbase = a.k + (int64_t)kvh * a.k_nb2 + (int64_t)bk * a.k_nb3;
    const char *vbase = a.v + (int64_t)kvh * a.v_nb2 + (int64_t)bk * a.v_nb3;
    const uint64_t k_avail = (uint64_t)(a.Skv - 1) * (uint64_t)a.k_nb1 + 2 * kD;
    const uint64_t v_avail = (uint64_t)(a.Skv - 1) * (uint64_t)a.v_nb1 + 2 * kD;
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void *)smem);
    const uint32_t k_row = (uint32_t)a.k_nb1, v_row = (uint32_t)a.v_nb1;
    // Copy c of a wave moves keys 4c + dkey, 16-byte slot dslot: K chunk
    // dslot ^ swz_k(key) = (dslot ^ dkey) ^ 4c, V chunk dslot ^ swz_v(key)
    // (swz_v depends on key & 7 = 4(c & 1) + dkey).  The lane offsets are
    // rebuilt per copy from four registers (kd, kx, vd[2]) and the scalar
    // 4c * row, which keeps eight registers free in the tile loop.
    const int dkey = lane >> 4, dslot = lane & 15;
    const uint32_t kd = (uint32_t)dkey * k_row, kx = 16u * (uint32_t)(dslot ^ dkey);
    const uint32_t vd[2] = {(uint32_t)dkey * v_row + 16u * (uint32_t)(dslot ^ swz_v(dkey)),
                            (uint32_t)dkey * v_row + 16u * (uint32_t)(dslot ^ swz_v(4 + dkey))};
    auto koff = [&](uint32_t kd_, uint32_t kx_, int c) __attribute__((always_inline)) {
        return kd_ + (kx_ ^ (64u * (uint32_t)c)) + 4u * (uint32_t)c * k_row;
    };
    auto voff = [&](const uint32_t (&vd_)[2], int c) __attribute__((always_inline)) {
        return vd_[c & 1] + 4u * (uint32_t)c * v_row;
    };
    auto tile_rsrc = [&](const char *base, uint64_t avail, uint32_t row, int kt) __attribute__((always_inline)) {
        const uint32_t off = (uint32_t)(kt * kPfBN + 16 * wave) * row;
        const uint64_t n = kt < a.n_kt && avail > off ? min(avail - off, (uint64_t)0xFFFFFFFFu) : 0;
        return buf_rsrc(base + off, (uint32_t)n);
    };
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

    int kt = next_live(0);
    if (kt < n_kt) {   // the first live tile's copies go out before Q is loaded
        const uint32_t l0 = lds0 + (uint32_t)(16 * wave) * 256u;
        const i32x4 rk = tile_rsrc(kbase, k_avail, k_row, kt);
        const i32x4 rv = tile_rsrc(vbase, v_avail, v_row, kt);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            dma16_buf(rk, koff(kd, kx, c), l0 + 4 * c * 256);
            dma16_buf(rv, voff(vd, c), l0 + kTileBytes + 4 * c * 256);
        }
    }

    // Q^T operands: qv[qb][t] = Q[query 16qb + n][32t + 8g .. +7], F32
    // rounded to T (round to nearest even), or already in T (a.q16).
    // (one branch around all the loads, so that they go out back to back
    // and share one memory latency)
    V8 qv[3][4];
    const char *qh = a.q + (int64_t)head * a.q_nb2 + (int64_t)b * a.q_nb3;
    if (a.q16) {
        u16x8 x[3][4];
#pragma unroll
        for (int qb = 0; qb < 3; qb++)
#pragma unroll
            for (int t = 0; t < 4; t++)
                x[qb][t] = *(const u16x8 *)(qh + (int64_t)qrow_c[qb] * a.q_nb1 + 2 * (32 * t + 8 * g));
#pragma unroll
        for (int qb = 0; qb < 3; qb++)
#pragma unroll
            for (int t = 0; t < 4; t++) qv[qb][t] = __builtin_bit_cast(V8, x[qb][t]);
    } else {
        f32x4 x[3][4][2];
#pragma unroll
        for (int qb = 0; qb < 3; qb++)
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const float *qf = (const float *)(qh + (int64_t)qrow_c[qb] * a.q_nb1) + 32 * t + 8 * g;
                x[qb][t][0] = *(const f32x4 *)qf;
                x[qb][t][1] = *(const f32x4 *)(qf + 4);
            }
#pragma unroll
        for (int qb = 0; qb < 3; qb++)
#pragma unroll
            for (int t = 0; t < 4; t++) qv[qb][t] = __builtin_bit_cast(V8, cvt8<T>(x[qb][t][0], x[qb][t][1]));
    }

    // LDS operand addresses.  K operand (key block kb, dim step t): row
    // 16kb + n, 16-byte chunk 4t + g at slot (4t + g) ^ n (swz_k).  V^T
    // operand (dim block db, half p): two transpose reads of rows 32p + 4g
    // + j/4 and 32p + 16 + 4g + j/4 (j = n), dims 16db + 4(j%4) .. +3, so
    // that lane j receives dim 16db + j of keys 4g..4g+3 and 16+4g..16+4g+3:
    // the k-slots of the P^T operand the S^T accumulators give this lane.
    //   K:   n*256 + 16((4t + g) ^ n)            = kb0 ^ 64t
    //   V^T: vrow*256 + 8(n & 1) + 16((2db + vc) ^ swz_v(vrow))
    //                                             = vb0 ^ 32db
    // (the XOR terms occupy bits 4-7 apart from the row and 8-byte terms;
    // swz_v is even), rebuilt from the two bases where they are read.
    const int vrow = 4 * g + (n16 >> 2);
    const uint32_t kb0 = n16 * 256 + 16 * (g ^ n16);
    const uint32_t vb0 = vrow * 256 + 8 * (n16 & 1) + 16 * ((n16 & 3) >> 1) + 16 * swz_v(vrow);
    auto kread = [&](auto st_c, uint32_t kb0_, int kb, int t) __attribute__((always_inline)) -> u16x8 {
        constexpr int ST = decltype(st_c)::value;
        return *(const u16x8 *)(smem + ST * kStageBytes + kb * 16 * 256 + (kb0_ ^ (64u * (uint32_t)t)));
    };
    auto vread = [&](auto st_c, uint32_t vb0_, int p, int db) __attribute__((always_inline)) -> u16x8 {
        constexpr int ST = decltype(st_c)::value;
        const uint8_t *q = smem + ST * kStageBytes + kTileBytes + p * 32 * 256 + (vb0_ ^ (32u * (uint32_t)db));
        const u16x4 p0 = lds_read_tr16(q);
        const u16x4 p1 = lds_read_tr16(q + 16 * 256);
        return u16x8{p0[0], p0[1], p0[2], p0[3], p1[0], p1[1], p1[2], p1[3]};
    };

    // O^T accumulators: o[db][qb] holds dims 16db + 4g + i of query 16qb + n
    f32x4 o[8][3];
#pragma unroll
    for (int db = 0; db < 8; db++)
#pragma unroll
        for (int qb = 0; qb < 3; qb++) o[db][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m2[3] = {-INFINITY, -INFINITY, -INFINITY}, lsum[3] = {0.f, 0.f, 0.f};

    // A half's scores s[kb][qb] (kb: its two 16-key blocks) for general
    // tiles (mask, tail, non-positive scale) become x = scale*s +
    // slope*mask in the exp2 domain, -inf for masked keys and keys past Skv
    // (lane: key 16kb + 4g + i of the half).
    auto general_x = [&](f32x4 (&s)[2][3], int key0) __attribute__((always_inline)) {
        const int kmax = a.Skv - key0 - 4 * g;
        if constexpr (SM) {
            // the zero mask value keeps the arithmetic of the dense path
#pragma unroll
            for (int qb = 0; qb < 3; qb++) {
                int lo, hi;
                row_range(qrow_c[qb], lo, hi);
                const int lo_rel = lo - key0 - 4 * g, hi_rel = hi - key0 - 4 * g;
#pragma unroll
                for (int kb = 0; kb < 2; kb++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int off = 16 * kb + i;
                        const float x = fmaf(s[kb][qb][i], sl2, 0.0f);
                        s[kb][qb][i] = (off >= lo_rel && off < hi_rel) ? x : -INFINITY;
                    }
            }
            return;
        }
        if constexpr (!MASKED) {
#pragma unroll
            for (int kb = 0; kb < 2; kb++)
#pragma unroll
                for (int qb = 0; qb < 3; qb++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        s[kb][qb][i] = 16 * kb + i >= kmax ? -INFINITY : s[kb][qb][i] * sl2;
            return;
        }
        u16x4 mw[2][3];
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
            for (int qb = 0; qb < 3; qb++)
                mw[kb][qb] = __builtin_bit_cast(
                    u16x4, __builtin_amdgcn_raw_buffer_load_b64(mrs, mrow_off[qb] + 2u * (uint32_t)(key0 + 16 * kb),
                                                                0, 0));
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
            for (int qb = 0; qb < 3; qb++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float mv = h2f_bits(mw[kb][qb][i]) * slope_l2;
                    const float x = fmaf(s[kb][qb][i], sl2, mv);
                    s[kb][qb][i] = (mv == -INFINITY || 16 * kb + i >= kmax) ? -INFINITY : x;
                }
    };
    // Probabilities of query block qb, key block kb of a half into the P^T
    // operand (k-slots 4kb + i).
    auto probs = [&](const f32x4 (&s)[2][3], int qb, int kb, float gs, float mneg, u16x8 (&pw)[3])
                     __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float p = fast_exp2(fmaf(s[kb][qb][i], gs, mneg));
            const uint16_t hbits = MF::from_f32(p);
            pw[qb][4 * kb + i] = hbits;
        }
    };
    auto max8 = [&](const f32x4 (&s)[2][3], int qb) __attribute__((always_inline)) {
        const f32x4 &x = s[0][qb], &y = s[1][qb];
        return fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])), fmaxf(fmaxf(y[0], y[1]), fmaxf(y[2], y[3])));
    };

    // One 64-key tile as two 32-key halves a, b (as fa_mfma.hip):
    //   R1  QK a                          (matrix cores; the next tile's
    //                                      copies, one per K operand)
    //   R2  QK b       | softmax of a, speculative with the reference m2
    //   R3  some lane's own max of the tile above m2 + 8 (ballot)?  then
    //       raise m2 to the row maxima, rescale O and l, and recompute S and
    //       P of half a (rare: a job's first tile, or a row that grows)
    //   R4  PV a       | softmax of b
    //   R5  PV b
    // The 32 LDS operands of a tile (K of a, K of b, V^T of a, V^T of b;
    // K operand n of a half is (dim step n/2, key block n%2)) are read kLook
    // operands ahead of the three MFMAs that consume each (a ring of kRing).
    // (a look-ahead of 3 measured the same: C4 self 148.8-149.8 us against
    // 149.0)
    constexpr int kLook = 2, kRing = kLook + 1;
    auto tile = [&](auto st_c, int kt, auto nst_c, int kn) __attribute__((always_inline)) {
        constexpr int NST = decltype(nst_c)::value;
        const bool do_issue = kn < n_kt;   // uniform
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
        const float gs = general ? 1.0f : sl2;   // wave-uniform
        // (address bases made opaque per tile, so that the addresses derived
        // from them are formed where they are used, not kept live across the
        // loop)
        uint32_t tkb0 = kb0, tvb0 = vb0, tkd = kd, tkx = kx, tvd[2] = {vd[0], vd[1]};
        asm volatile("" : "+v"(tkb0), "+v"(tvb0), "+v"(tkd), "+v"(tkx), "+v"(tvd[0]), "+v"(tvd[1]));
        u16x8 op[kRing];
        auto fetch = [&](int n) __attribute__((always_inline)) {
            if (n < 8) op[n % kRing] = kread(st_c, tkb0, n & 1, n >> 1);
            else if (n < 16) op[n % kRing] = kread(st_c, tkb0, 2 + (n & 1), (n - 8) >> 1);
            else if (n < 24) op[n % kRing] = vread(st_c, tvb0, 0, n - 16);
            else if (n < 32) op[n % kRing] = vread(st_c, tvb0, 1, n - 24);
        };
        auto qk3 = [&](f32x4 (&s)[2][3], int n) __attribute__((always_inline)) {
            const int t = (n & 7) >> 1, kb = n & 1;
#pragma unroll
            for (int qb = 0; qb < 3; qb++)
                s[kb][qb] = MF::run(__builtin_bit_cast(V8, op[n % kRing]), qv[qb][t],
                                    t == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : s[kb][qb]);
        };
        auto pv3 = [&](const u16x8 (&pw)[3], int n) __attribute__((always_inline)) {
            const int db = n & 7;
#pragma unroll
            for (int qb = 0; qb < 3; qb++)
                o[db][qb] = MF::run(__builtin_bit_cast(V8, op[n % kRing]), __builtin_bit_cast(V8, pw[qb]), o[db][qb]);
        };
        f32x4 sa[2][3], sb[2][3];
        u16x8 pa[3], pb[3];

        // ---- R1: QK a (+ the next tile's copies) ----
#pragma unroll
        for (int n = 0; n < kLook; n++) fetch(n);
#pragma unroll
        for (int n = 0; n < 8; n++) {
            fetch(n + kLook);
            qk3(sa, n);
            if (do_issue) {   // copy c = n/2 of the next tile's K rows (n even) or V rows
                if (n & 1) dma16_buf(nrv, voff(tvd, n >> 1), nl0 + kTileBytes + 4 * (n >> 1) * 256);
                else dma16_buf(nrk, koff(tkd, tkx, n >> 1), nl0 + 4 * (n >> 1) * 256);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (general) general_x(sa, key0);
        __builtin_amdgcn_sched_barrier(0);

        // ---- R2: QK b | softmax a (speculative) ----
        float mneg0[3], mxa[3];
#pragma unroll
        for (int qb = 0; qb < 3; qb++) mneg0[qb] = (m2[qb] == -INFINITY) ? 0.0f : -m2[qb];
#pragma unroll
        for (int n = 0; n < 8; n++) {
            fetch(8 + n + kLook);
            qk3(sb, 8 + n);
            if (n == 0) {
#pragma unroll
                for (int qb = 0; qb < 3; qb++) mxa[qb] = max8(sa, qb);
            } else if (n <= 6) {
                probs(sa, (n - 1) >> 1, (n - 1) & 1, gs, mneg0[(n - 1) >> 1], pa);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        float la[3];
#pragma unroll
        for (int qb = 0; qb < 3; qb++) {
            la[qb] = sum8<T>(pa[qb], 0.0f);
        }
        // keep the speculative softmax here, overlapped with QK b (it is
        // redone on the rare path, so it would otherwise sink past R3)
        asm volatile("" ::"v"(pa[0]), "v"(pa[1]), "v"(pa[2]), "v"(la[0]), "v"(la[1]), "v"(la[2]), "v"(mxa[0]),
                     "v"(mxa[1]), "v"(mxa[2]));
        if (general) general_x(sb, key0 + 32);
        __builtin_amdgcn_sched_barrier(0);

        // ---- R3: tile max, reference update (rare) ----
        float bmax[3];
        bool need = false;
#pragma unroll
        for (int qb = 0; qb < 3; qb++) {
            bmax[qb] = fmaxf(mxa[qb], max8(sb, qb)) * gs;
            need |= bmax[qb] > m2[qb] + 8.0f;
        }
        if (__builtin_amdgcn_ballot_w64(need) != 0) {   // wave-uniform
#pragma unroll
            for (int qb = 0; qb < 3; qb++) {
                const float rmax = max_pair16(max_half32(bmax[qb]));   // over lanes n, n+16, n+32, n+48
                const float mnew = fmaxf(m2[qb], rmax);
                const float alpha = (m2[qb] == -INFINITY) ? 1.0f : fast_exp2(m2[qb] - mnew);
                m2[qb] = mnew;
                lsum[qb] *= alpha;
#pragma unroll
                for (int db = 0; db < 8; db++) o[db][qb] *= alpha;
            }
            // S of half a again (K of half a is still in this stage), then P
#pragma unroll
            for (int n = 0; n < 8; n++) {
                op[n % kRing] = kread(st_c, tkb0, n & 1, n >> 1);
                qk3(sa, n);
            }
            if (general) general_x(sa, key0);
#pragma unroll
            for (int qb = 0; qb < 3; qb++) {
                const float mn = (m2[qb] == -INFINITY) ? 0.0f : -m2[qb];
                probs(sa, qb, 0, gs, mn, pa);
                probs(sa, qb, 1, gs, mn, pa);
                la[qb] = sum8<T>(pa[qb], 0.0f);
            }
            // (the operand ring restarts at V^T of half a)
#pragma unroll
            for (int n = 16; n < 16 + kLook; n++) fetch(n);
        }
        float mneg[3];
#pragma unroll
        for (int qb = 0; qb < 3; qb++) mneg[qb] = (m2[qb] == -INFINITY) ? 0.0f : -m2[qb];
        __builtin_amdgcn_sched_barrier(0);

        // ---- R4: PV a | softmax b ----
#pragma unroll
        for (int n = 0; n < 8; n++) {
            fetch(16 + n + kLook);
            pv3(pa, 16 + n);
            if (n < 6) probs(sb, n >> 1, n & 1, gs, mneg[n >> 1], pb);
            __builtin_amdgcn_sched_barrier(0);
        }
        float lb[3];
#pragma unroll
        for (int qb = 0; qb < 3; qb++) {
            lb[qb] = sum8<T>(pb[qb], 0.0f);
        }
        __builtin_amdgcn_sched_barrier(0);

        // ---- R5: PV b ----
#pragma unroll
        for (int n = 0; n < 8; n++) {
            fetch(24 + n + kLook);
            pv3(pb, 24 + n);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int qb = 0; qb < 3; qb++) lsum[qb] += la[qb] + lb[qb];
    };

    // Double-buffered loop over the live tiles: wait for this wave's copies
    // of the tile, one barrier (every wave's copies have landed and every
    // wave is done with the other stage), compute, with the next live
    // tile's copies into the other stage spread over R1.
    std::integral_constant<int, 0> st0;
    std::integral_constant<int, 1> st1;
    int ofree = 1;   // the stage no tile still reads at the end
    while (kt < n_kt) {
        int kn = next_live(kt + 1);
        MXFA_WAIT_VMCNT(0);
        __builtin_amdgcn_s_barrier();
        tile(st0, kt, st1, kn);
        ofree = 1;
        kt = kn;
        if (kt >= n_kt) break;
        kn = next_live(kt + 1);
        MXFA_WAIT_VMCNT(0);
        __builtin_amdgcn_s_barrier();
        tile(st1, kt, st0, kn);
        ofree = 0;
        kt = kn;
    }

    // Row sums over the four lanes of a query; O leaves as whole rows
    // through the stage the last tile did not read (every wave was past its
    // last read of it at that tile's barrier, and no copy has gone into it
    // since): per query block, each wave writes its 16 rows (8 KB, 16-byte
    // chunk c of a row at slot c ^ row) and stores 2 rows per 16-byte store.
    float inv[3];
#pragma unroll
    for (int qb = 0; qb < 3; qb++) {
        const float l = sum_pair16(sum_pair32(lsum[qb]));
        inv[qb] = (l == 0.0f) ? 0.0f : 1.0f / l;
    }
    uint8_t *ost = smem + ofree * kStageBytes + wave * 8192;
    float *drow = a.dst + ((int64_t)b * a.Sq * a.Nh + head) * kD;   // + q * Nh * kD per row
#pragma unroll
    for (int qb = 0; qb < 3; qb++) {
#pragma unroll
        for (int db = 0; db < 8; db++) {
            const int c = 4 * db + g;   // dims 4c .. 4c+3 of row n
            *(f32x4 *)(ost + n16 * 512 + 16 * (c ^ n16)) = o[db][qb] * inv[qb];
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int rl = 2 * i + (lane >> 5), c = lane & 31;
            const f32x4 v = *(const f32x4 *)(ost + rl * 512 + 16 * (c ^ rl));
            const int q = q0w + 16 * qb + rl;
            if (q < a.Sq) *(f32x4 *)(drow + (int64_t)q * a.Nh * kD + 4 * c) = v;
        }
    }
}

template <int T, int MODE>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
fa_wide_kernel(const FaArgs a) {
    fa_wide_body<T, MODE>(a);
}

hipError_t launch_fa_wide(const FaArgs &a, int ktype, hipStream_t stream) {
    dim3 grid((uint32_t)a.n_qt_w * (uint32_t)a.Nh * (uint32_t)a.B);
    if (ktype != T_F16) return hipErrorInvalidValue;   // (F16 only: see mxfa_api.cpp)
    if (a.sm_flags) hipLaunchKernelGGL((fa_wide_kernel<T_F16, kWideSm>), grid, dim3(256), kPfLds, stream, a);
    else if (a.mask) hipLaunchKernelGGL((fa_wide_kernel<T_F16, kWideDense>), grid, dim3(256), kPfLds, stream, a);
    else hipLaunchKernelGGL((fa_wide_kernel<T_F16, kWideNone>), grid, dim3(256), kPfLds, stream, a);
    return hipGetLastError();
}

}  // namespace mxfa
