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

#include "mxfa_common.h"
#include "mxfa_internal.h"


namespace mxfa {

constexpr int kTileBytes = 16384;            // one K or one V^T tile
constexpr int kStageBytes = 2 * kTileBytes;  // K + V^T
constexpr int kPfLds = 2 * kStageBytes;      // double buffered: 64 KB

__global__ void __launch_bounds__(256) mask_classify_kernel(const FaArgs a, uint8_t *cls) {
    const int kt = blockIdx.x, qt = blockIdx.y, plane = blockIdx.z;
    const int m2i = plane % a.m_ne2, m3i = plane / a.m_ne2;
    const char *base = a.mask + (int64_t)m2i * a.m_nb2 + (int64_t)m3i * a.m_nb3;
    const int q_lo = qt * kPfBM, k_lo = kt * kPfBN;
    int all_ninf = 1, all_zero = 1;
    for (int i = threadIdx.x; i < kPfBM * kPfBN; i += 256) {
        const int q = q_lo + (i >> 6), k = k_lo + (i & 63);
        if (q < a.Sq && k < a.Skv) {
            const uint16_t v = *(const uint16_t *)(base + (int64_t)q * a.m_nb1 + 2 * (int64_t)k);
            all_ninf &= (v == 0xFC00u);
            all_zero &= ((v & 0x7FFFu) == 0);
        }
    }
    all_ninf = __syncthreads_and(all_ninf);
    all_zero = __syncthreads_and(all_zero);
    if (threadIdx.x == 0) cls[((int64_t)plane * a.n_qt + qt) * a.n_kt + kt] = all_ninf ? 0 : (all_zero ? 1 : 2);
}

__device__ __forceinline__ int next_live(const uint8_t *cls, int kt, int n) {
    if (!cls) return kt;
    while (kt < n && cls[kt] == 0) kt++;
    return kt;
}

template <int T>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
fa_prefill_kernel(const FaArgs a) {
    using MF = Mfma32<T>;
    using V8 = typename MF::v8;
    static_assert(kD == 128, "kernel is written for D = 128");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
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
    const uint8_t *cls = a.tile_class ? a.tile_class + ((int64_t)plane * a.n_qt + qt) * a.n_kt : nullptr;
    const uint16_t *mrow =
        a.mask ? (const uint16_t *)(a.mask + (int64_t)qrow_c * a.m_nb1 + (int64_t)(head % a.m_ne2) * a.m_nb2 +
                                    (int64_t)(b % a.m_ne3) * a.m_nb3)
               : nullptr;
    const float slope_l2 = alibi_slope(a, head) * kLog2e;
    const float sl2 = a.scale * kLog2e;
    const bool use_softcap = a.softcap != 0.0f;
    const float sc_in = use_softcap ? a.scale / a.softcap : 0.0f;

    const char *kbase = a.k + (int64_t)kvh * a.k_nb2 + (int64_t)bk * a.k_nb3;
    const char *vbase = a.v + (int64_t)kvh * a.v_nb2 + (int64_t)bk * a.v_nb3;

    // staging assignment: 16-byte chunk dc of keys kq+16j (K) / 4kq+kk (V)
    const int dc = tid & 15, kq = tid >> 4;

    f32x16 o[4];
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[dt][r] = 0.0f;
    float m2 = -INFINITY, lsum = 0.0f;

    u16x8 kreg[4], vreg[4];
    auto gload = [&](int kt) {
        const int key0 = kt * kPfBN;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int key = min(key0 + kq + 16 * j, a.Skv - 1);
            kreg[j] = *(const u16x8 *)(kbase + (int64_t)key * a.k_nb1 + 16 * dc);
        }
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            const int key = min(key0 + 4 * kq + kk, a.Skv - 1);
            vreg[kk] = *(const u16x8 *)(vbase + (int64_t)key * a.v_nb1 + 16 * dc);
        }
    };
    auto lstore = [&](int stage) {
        uint8_t *ks = smem + stage * kStageBytes;
        uint8_t *vs = ks + kTileBytes;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int key = kq + 16 * j;
            *(u16x8 *)(ks + key * 256 + 16 * (dc ^ (key & 15))) = kreg[j];
        }
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int d = 8 * dc + e;
            const int slot = kq ^ ((d & 15) ^ ((d >> 4) & 7));
            u16x4 w = {vreg[0][e], vreg[1][e], vreg[2][e], vreg[3][e]};
            *(u16x4 *)(vs + d * 128 + 8 * slot) = w;
        }
    };

    const int n_kt = a.n_kt;
    int kt = next_live(cls, 0, n_kt);
    if (kt < n_kt) {
        gload(kt);
        lstore(0);
    }
    __syncthreads();
    int stage = 0;
    while (kt < n_kt) {
        const int kn = next_live(cls, kt + 1, n_kt);
        if (kn < n_kt) gload(kn);
        const int cl = cls ? cls[kt] : 1;
        const uint8_t *ks = smem + stage * kStageBytes;
        const uint8_t *vs = ks + kTileBytes;

        // One 32-key half-tile: S^T = K . Q^T, online softmax, O^T += V^T . P^T.
        // Interior unmasked tiles only scale the scores; tiles with mask
        // entries, the Skv tail or a softcap take the general transform.
        const int key0 = kt * kPfBN;
        const bool tail = key0 + kPfBN > a.Skv;
        const bool general = cl == 2 || tail || use_softcap;
#pragma unroll 1
        for (int kb = 0; kb < 2; kb++) {
            // lane: query l32, keys 32kb + 8(r/4) + 4h + r%4
            f32x16 s;
#pragma unroll
            for (int r = 0; r < 16; r++) s[r] = 0.0f;
            {
                const int key = 32 * kb + l32;
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    const u16x8 av = *(const u16x8 *)(ks + key * 256 + 16 * ((2 * t + h) ^ (key & 15)));
                    s = MF::run(__builtin_bit_cast(V8, av), qb[t], s);
                }
            }
            // scores -> exp2 domain
            if (!general) {
#pragma unroll
                for (int r = 0; r < 16; r++) s[r] *= sl2;
            } else {
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
                        if (use_softcap) xv = (a.softcap * tanhf(s[r] * sc_in)) * kLog2e + mv[i];
                        else xv = fmaf(s[r], sl2, mv[i]);
                        if (mv[i] == -INFINITY || kbase4 + i >= a.Skv) xv = -INFINITY;
                        s[r] = xv;
                    }
                }
            }
            float bmax = -INFINITY;
#pragma unroll
            for (int r = 0; r < 16; r++) bmax = fmaxf(bmax, s[r]);
            bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
            // Lazy rescale: the reference max m2 is raised only when some
            // row's new max exceeds it by more than 8 (exp2 domain), so
            // p <= 2^8 and O, l are rescaled on few tiles.  O and l always
            // share the same reference, so the softmax is unchanged.
            if (__any(bmax > m2 + 8.0f)) {
                const float mnew = fmaxf(m2, bmax);
                const float alpha = (mnew == -INFINITY) ? 1.0f : fast_exp2(m2 - mnew);
                m2 = mnew;
                lsum *= alpha;
#pragma unroll
                for (int dt = 0; dt < 4; dt++) o[dt] *= alpha;
            }
            const float m_use = (m2 == -INFINITY) ? 0.0f : m2;
#pragma unroll
            for (int r = 0; r < 16; r++) s[r] = fast_exp2(s[r] - m_use);   // exp2(-inf) = 0
            // P^T operands of the two 16-key steps ks = 2kb + u2:
            // k-slot 4u+i <-> key 16ks + 8u + 4h + i = register 8u2 + 4u + i.
            // The row sum adds the same rounded values the MFMA consumes.
            V8 pb[2];
#pragma unroll
            for (int u2 = 0; u2 < 2; u2++) {
                const int rb = 8 * u2;
                const u16x8 bits = cvt8<T>(f32x4{s[rb + 0], s[rb + 1], s[rb + 2], s[rb + 3]},
                                           f32x4{s[rb + 4], s[rb + 5], s[rb + 6], s[rb + 7]});
                lsum = sum8<T>(bits, lsum);
                pb[u2] = __builtin_bit_cast(V8, bits);
            }
#pragma unroll
            for (int dt = 0; dt < 4; dt++) {
                const int d = 32 * dt + l32;
                const int sw = (d & 15) ^ ((d >> 4) & 7);
                const uint8_t *vrow = vs + d * 128;
#pragma unroll
                for (int u2 = 0; u2 < 2; u2++) {
                    const int ksi = 2 * kb + u2;
                    const u16x4 lo = *(const u16x4 *)(vrow + 8 * ((4 * ksi + h) ^ sw));
                    const u16x4 hi = *(const u16x4 *)(vrow + 8 * ((4 * ksi + 2 + h) ^ sw));
                    const u16x8 av = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                    o[dt] = MF::run(__builtin_bit_cast(V8, av), pb[u2], o[dt]);
                }
            }
        }

        if (kn < n_kt) lstore(stage ^ 1);
        __syncthreads();
        stage ^= 1;
        kt = kn;
    }

    lsum += __shfl_xor(lsum, 32);
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
