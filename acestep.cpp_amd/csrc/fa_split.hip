// fa_split.hip -- split-KV flash attention for gfx950 (decode and the
// general path).
//
// Serves the decode call sites of the reference: single-sequence decode
// (src/qwen3-lm.h:465, n_tokens = 1) and batched CFG decode
// (src/qwen3-lm.h:789-794, q [D,1,Nh,N] against a 4D KV-cache view with a
// per-sequence padding mask built at :872-883), and any shape the MFMA
// prefill kernel does not take.
//
// Work decomposition.  One workgroup = 4 waves = one (batch b, KV head,
// 16-row tile, KV split).  A row is one (query, q head) pair; the G = Nh/Nkv
// q heads of a KV head (and the Sq queries) are packed as MFMA columns, so
// each K/V byte streamed from HBM serves all of them (GQA reuse).  The split
// of `chunk` keys is walked by the 4 waves in interleaved 32-key blocks.
//
// Per 32-key block a wave:
//   1. reads the additive mask of its 8 (row, key) entries and skips the
//      block when every entry is -inf (ragged lengths cost nothing past the
//      end of each sequence: the reference pads the window to 256 keys and
//      masks the tail, qwen3-lm.h:496-500, :875-881);
//   2. loads K straight from HBM into the MFMA A operand (16 B per lane:
//      8 dims of one key) and V rows (16 B per lane);
//   3. S^T = K . Q^T with v_mfma_f32_16x16x32_{f16,bf16} (4 per 16 keys);
//   4. online softmax in fp32 registers (exp2 domain), row max/sum reduced
//      across the 4 lane groups that hold a row;
//   5. stages V transposed into a per-wave LDS tile (XOR-swizzled 8-byte
//      chunks, conflict-free for both the transposing writes and the
//      operand reads) and accumulates O^T += V^T . P^T with the same MFMA.
// The 4 waves then merge (m, l, O) through LDS.  With one split the
// workgroup writes the normalised output; otherwise it writes an
// unnormalised partial plus (m, l) and fa_combine_kernel merges the splits
// with a log-sum-exp reduction.
//
// Masked keys are never allowed to contribute: a score whose mask entry is
// -inf is replaced by -inf (not added to), and V rows of keys that are dead
// for every row of the tile are zeroed before the PV product, so non-finite
// data in masked cache slots cannot leak into the output (ggml's CPU kernel
// skips such keys entirely).

#include "mxfa_common.h"
#include "mxfa_internal.h"

namespace mxfa {

constexpr int kSplitWaves = 4;
constexpr int kVtStride = 36;  // halfs per V^T row: 32 keys + 4 pad (72 B)

template <int T>
__global__ void __launch_bounds__(256) fa_split_kernel(const FaArgs a) {
    using MF = Mfma16<T>;
    using V8 = typename MF::v8;
    static_assert(kD == 128, "kernel is written for D = 128");

    __shared__ __attribute__((aligned(16))) uint16_t vt_lds[kSplitWaves * kD * kVtStride];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int c16 = lane & 15, g16 = lane >> 4;
    const int split = blockIdx.x;
    const int kvh = blockIdx.y / a.row_tiles, rt = blockIdx.y % a.row_tiles;
    const int b = blockIdx.z;
    const int bk = b / a.rk3;

    // The row this lane owns as an MFMA column.
    const int r = rt * 16 + c16;
    const bool row_ok = r < a.M;
    const int iq1 = row_ok ? r / a.G : 0;
    const int head = kvh * a.G + (row_ok ? r % a.G : 0);

    // Q^T operand: Q[row][32t + 8*g16 + e], converted like ggml converts Q
    // to K's vec-dot type (F16 or BF16, round to nearest even).
    V8 qb[4];
    {
        const float *qp = (const float *)(a.q + (int64_t)iq1 * a.q_nb1 + (int64_t)head * a.q_nb2 +
                                          (int64_t)b * a.q_nb3);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            f32x4 x0 = {0.f, 0.f, 0.f, 0.f}, x1 = {0.f, 0.f, 0.f, 0.f};
            if (row_ok) {
                x0 = *(const f32x4 *)(qp + 32 * t + 8 * g16);
                x1 = *(const f32x4 *)(qp + 32 * t + 8 * g16 + 4);
            }
            qb[t] = __builtin_bit_cast(V8, cvt8<T>(x0, x1));
        }
    }
    const float slope_l2 = alibi_slope(a, head) * kLog2e;
    const uint16_t *mrow =
        a.mask ? (const uint16_t *)(a.mask + (int64_t)iq1 * a.m_nb1 + (int64_t)(head % a.m_ne2) * a.m_nb2 +
                                    (int64_t)(b % a.m_ne3) * a.m_nb3)
               : nullptr;
    const char *kbase = a.k + (int64_t)kvh * a.k_nb2 + (int64_t)bk * a.k_nb3;
    const char *vbase = a.v + (int64_t)kvh * a.v_nb2 + (int64_t)bk * a.v_nb3;
    const float sl2 = a.scale * kLog2e;
    const bool use_softcap = a.softcap != 0.0f;
    const float sc_in = use_softcap ? a.scale / a.softcap : 0.0f;

    f32x4 o[8];
#pragma unroll
    for (int dt = 0; dt < 8; dt++) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m2 = -INFINITY;   // running max of this lane's row (exp2 domain)
    float lsum = 0.0f;      // this lane's share of the row sum

    const int k0 = split * a.chunk;
    const int k1 = min(a.Skv, k0 + a.chunk);
    uint16_t *vt = vt_lds + wave * kD * kVtStride;

    for (int kb = k0 + wave * 32; kb < k1; kb += 32 * kSplitWaves) {
        // 1. mask entries of (row c16, keys kb + 16*sb + 4*g16 + i)
        float mk[2][4];
        int live = 0;
#pragma unroll
        for (int sb = 0; sb < 2; sb++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int key = kb + 16 * sb + 4 * g16 + i;
                float mv = -INFINITY;
                if (row_ok && key < k1) mv = mrow ? h2f_bits(mrow[key]) * slope_l2 : 0.0f;
                mk[sb][i] = mv;
                live |= (mv != -INFINITY);
            }
        if (!__any(live)) continue;

        // keys dead for every row of the tile (AND over the 16 rows)
        uint32_t dead = 0;
#pragma unroll
        for (int sb = 0; sb < 2; sb++)
#pragma unroll
            for (int i = 0; i < 4; i++) dead |= (mk[sb][i] == -INFINITY ? 1u : 0u) << (4 * sb + i);
        dead &= __shfl_xor(dead, 1);
        dead &= __shfl_xor(dead, 2);
        dead &= __shfl_xor(dead, 4);
        dead &= __shfl_xor(dead, 8);

        // 2. loads.  K: key kb+16sb+c16, dims 32t+8g16..+8.  V: keys
        // kb+4g16+16j+kk, dims 8c16..+8.  Keys past Skv are clamped to a
        // valid row (their scores are -inf and their V rows zeroed).
        u16x8 kr[2][4];
#pragma unroll
        for (int sb = 0; sb < 2; sb++) {
            const int key = min(kb + 16 * sb + c16, a.Skv - 1);
            const char *kp = kbase + (int64_t)key * a.k_nb1 + 16 * g16;
#pragma unroll
            for (int t = 0; t < 4; t++) kr[sb][t] = *(const u16x8 *)(kp + 64 * t);
        }
        u16x8 vr[2][4];
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                const int key = min(kb + 4 * g16 + 16 * j + kk, a.Skv - 1);
                vr[j][kk] = *(const u16x8 *)(vbase + (int64_t)key * a.v_nb1 + 16 * c16);
            }

        // 3. S^T tile: lane holds S^T[key 16sb+4g16+i][row c16]
        f32x4 s[2];
#pragma unroll
        for (int sb = 0; sb < 2; sb++) {
            s[sb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < 4; t++)
                s[sb] = MF::run(__builtin_bit_cast(V8, kr[sb][t]), qb[t], s[sb]);
        }

        // 4. online softmax (exp2 domain)
        float x[2][4];
        float bmax = -INFINITY;
#pragma unroll
        for (int sb = 0; sb < 2; sb++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float sv = s[sb][i];
                float xv;
                if (use_softcap) xv = (a.softcap * tanhf(sv * sc_in)) * kLog2e + mk[sb][i];
                else xv = fmaf(sv, sl2, mk[sb][i]);
                xv = (mk[sb][i] == -INFINITY) ? -INFINITY : xv;
                x[sb][i] = xv;
                bmax = fmaxf(bmax, xv);
            }
        bmax = fmaxf(bmax, __shfl_xor(bmax, 16));
        bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
        const float mnew = fmaxf(m2, bmax);
        const float alpha = (mnew == -INFINITY) ? 1.0f : fast_exp2(m2 - mnew);
        m2 = mnew;
        float p[2][4];
#pragma unroll
        for (int sb = 0; sb < 2; sb++)
#pragma unroll
            for (int i = 0; i < 4; i++) p[sb][i] = (x[sb][i] == -INFINITY) ? 0.0f : fast_exp2(x[sb][i] - mnew);
#pragma unroll
        for (int dt = 0; dt < 8; dt++) o[dt] *= alpha;
        const u16x8 pbits =
            cvt8<T>(f32x4{p[0][0], p[0][1], p[0][2], p[0][3]}, f32x4{p[1][0], p[1][1], p[1][2], p[1][3]});
        lsum = sum8<T>(pbits, lsum * alpha);
        const V8 pb = __builtin_bit_cast(V8, pbits);

        // 5. V^T into this wave's LDS tile.  Chunk kc (4 keys) of row d is
        // stored at chunk slot kc ^ ((d >> 4) & 7).
#pragma unroll
        for (int j = 0; j < 2; j++) {
#pragma unroll
            for (int kk = 0; kk < 4; kk++)
                if (dead & (1u << (4 * j + kk))) vr[j][kk] = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
            const int kc = g16 + 4 * j;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int d = 8 * c16 + e;
                u16x4 w = {vr[j][0][e], vr[j][1][e], vr[j][2][e], vr[j][3][e]};
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
            u16x4 lo = *(const u16x4 *)(row + 4 * (g16 ^ dt));
            u16x4 hi = *(const u16x4 *)(row + 4 * ((g16 + 4) ^ dt));
            u16x8 av = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            o[dt] = MF::run(__builtin_bit_cast(V8, av), pb, o[dt]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    // Merge the 4 waves.
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
    __syncthreads();
    float *mo = (float *)vt_lds;                 // [wave][d][16 rows]
    float *mm = mo + kSplitWaves * kD * 16;      // [wave][16] max
    float *ml = mm + kSplitWaves * 16;           // [wave][16] sum
#pragma unroll
    for (int dt = 0; dt < 8; dt++)
#pragma unroll
        for (int i = 0; i < 4; i++) mo[(wave * kD + 16 * dt + 4 * g16 + i) * 16 + c16] = o[dt][i];
    if (g16 == 0) {
        mm[wave * 16 + c16] = m2;
        ml[wave * 16 + c16] = lsum;
    }
    __syncthreads();

    const int rr = tid & 15;
    const int dd0 = (tid >> 4) * 8;
    const int rglob = rt * 16 + rr;
    if (rglob >= a.M) return;
    float mw[kSplitWaves];
    float mstar = -INFINITY;
#pragma unroll
    for (int w = 0; w < kSplitWaves; w++) {
        mw[w] = mm[w * 16 + rr];
        mstar = fmaxf(mstar, mw[w]);
    }
    float fw[kSplitWaves];
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < kSplitWaves; w++) {
        fw[w] = (mw[w] == -INFINITY) ? 0.0f : fast_exp2(mw[w] - mstar);
        L += fw[w] * ml[w * 16 + rr];
    }
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        float sacc = 0.0f;
#pragma unroll
        for (int w = 0; w < kSplitWaves; w++) sacc += fw[w] * mo[(w * kD + dd0 + e) * 16 + rr];
        acc[e] = sacc;
    }
    if (a.n_splits == 1) {
        const float inv = (L == 0.0f) ? 0.0f : 1.0f / L;
        const int iq1o = rglob / a.G, heado = kvh * a.G + rglob % a.G;
        float *dp = a.dst + (((int64_t)b * a.Sq + iq1o) * a.Nh + heado) * kD + dd0;
        *(f32x4 *)dp = f32x4{acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
        *(f32x4 *)(dp + 4) = f32x4{acc[4] * inv, acc[5] * inv, acc[6] * inv, acc[7] * inv};
    } else {
        const int64_t pr = ((int64_t)b * a.Nkv + kvh) * a.M + rglob;
        float *po = a.part_o + (pr * a.n_splits + split) * kD + dd0;
        *(f32x4 *)po = f32x4{acc[0], acc[1], acc[2], acc[3]};
        *(f32x4 *)(po + 4) = f32x4{acc[4], acc[5], acc[6], acc[7]};
        if (dd0 == 0) {
            a.part_ml[(pr * a.n_splits + split) * 2 + 0] = mstar;
            a.part_ml[(pr * a.n_splits + split) * 2 + 1] = L;
        }
    }
}

// Log-sum-exp merge of the splits: one 128-thread block per row.
__global__ void __launch_bounds__(128) fa_combine_kernel(const FaArgs a) {
    const int64_t pr = blockIdx.x;
    const int d = threadIdx.x;
    const int r = (int)(pr % a.M);
    const int kvh = (int)((pr / a.M) % a.Nkv);
    const int b = (int)(pr / ((int64_t)a.M * a.Nkv));
    const float *ml = a.part_ml + pr * a.n_splits * 2;
    float mstar = -INFINITY;
    for (int s = 0; s < a.n_splits; s++) mstar = fmaxf(mstar, ml[2 * s]);
    float L = 0.0f, acc = 0.0f;
    if (mstar != -INFINITY) {
        const float *po = a.part_o + pr * a.n_splits * kD + d;
        for (int s = 0; s < a.n_splits; s++) {
            const float ms = ml[2 * s];
            if (ms == -INFINITY) continue;
            const float f = fast_exp2(ms - mstar);
            L = fmaf(f, ml[2 * s + 1], L);
            acc = fmaf(f, po[(int64_t)s * kD], acc);
        }
    }
    const float inv = (L == 0.0f) ? 0.0f : 1.0f / L;
    const int iq1 = r / a.G, head = kvh * a.G + r % a.G;
    a.dst[(((int64_t)b * a.Sq + iq1) * a.Nh + head) * kD + d] = acc * inv;
}

hipError_t launch_fa_split(const FaArgs &a, int ktype, hipStream_t stream) {
    if (ktype != T_F16 && ktype != T_BF16) return hipErrorInvalidValue;
    const dim3 grid(a.n_splits, a.Nkv * a.row_tiles, a.B);
    hipError_t e = timed_launch("fa_split", stream, [&] {
        if (ktype == T_F16) hipLaunchKernelGGL(fa_split_kernel<T_F16>, grid, dim3(256), 0, stream, a);
        else hipLaunchKernelGGL(fa_split_kernel<T_BF16>, grid, dim3(256), 0, stream, a);
        return hipGetLastError();
    });
    if (e != hipSuccess || a.n_splits == 1) return e;
    const int64_t rows = (int64_t)a.B * a.Nkv * a.M;
    return timed_launch("fa_combine", stream, [&] {
        hipLaunchKernelGGL(fa_combine_kernel, dim3((unsigned)rows), dim3(128), 0, stream, a);
        return hipGetLastError();
    });
}

}  // namespace mxfa
