// qk_norm_rope.hip -- the work between the QKV projections and attention,
// fused into one pass: QK-RMSNorm, NEOX RoPE, the 16-bit cast of Q, K and V,
// and the KV-cache write.
//
// The reference runs it as separate ggml ops per layer (src/qwen3-lm.h:418-454;
// src/dit-graph.h:177-225):
//   q = rope_neox(rms_norm(q, eps) * q_norm, pos);  k likewise with k_norm
//   k, v = cont(permute(...)); v = clamp(v, +-65504) (optional, :438-441)
//   set_rows(cache_k, k, kv_rows); set_rows(cache_v, v, kv_rows)
// after which attention reads Q in F32 and converts it to K's type.  Here
// every row of 128 values is read once in F32 and written once in 16 bits:
// Q into [D, Nh, S, B] (attention takes its permuted view, as the reference
// does), K and V straight into their cache rows.
//
// DiT cross-attention (src/dit-graph.h:317-346) runs the same chain without
// RoPE ("no RoPE for cross-attention", :333) and with K/V from the encoder:
// positions == NULL switches the rotation off, and K/V then have their own
// token count Skv (enc_S) next to Q's S.
//
// Arithmetic as ggml's CPU ops do it:
//   rms_norm: sum of x*x (float products) accumulated in double, mean =
//     sum / 128, scale = 1 / sqrtf(mean + eps), y = x * scale, then * w;
//   rope (NEOX, n_dims = 128, freq_scale 1, no YaRN): the angle of pair i
//     (dims i, i + 64) is theta_i = p * theta_scale^i formed by repeated
//     float multiplication from theta_0 = p, theta_scale = powf(base, -2/128)
//     (host); y_i = x_i cos - x_{i+64} sin, y_{i+64} = x_i sin + x_{i+64} cos;
//   16-bit cast: round to nearest even.

#include "mxfa_common.h"
#include "mxfa_internal.h"

namespace mxfa {

template <int OT>
__device__ __forceinline__ uint16_t to16(float x) {
    return Mfma16<OT>::from_f32(x);
}

// Rows of one token: [0, Nh) Q heads, [Nh, Nh + Nkv) K heads, then V heads.
constexpr int kGroups = 3;   // 16-row groups a workgroup loads before it computes (48-row tokens: one pass)

// One 32-bit half of a double moved across lanes by a DPP pattern.
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)u, CTRL, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(u >> 32), CTRL, 0xF, 0xF, false);
    return __builtin_bit_cast(double, (uint64_t)lo | ((uint64_t)hi << 32));
}

// Sum over the 16 lanes of a row, left in every lane of it: partners 1 and 2
// apart (quad permutations), then the mirrored quads and the mirrored
// halves. Each step adds a value and its partner's, and the partner adds the
// same two (addition commutes), so all 16 lanes hold the same bits.
__device__ __forceinline__ double row16_sum(double v) {
    v += dpp_f64<0xB1>(v);    // quad_perm [1, 0, 3, 2]
    v += dpp_f64<0x4E>(v);    // quad_perm [2, 3, 0, 1]
    v += dpp_f64<0x141>(v);   // row_half_mirror: quad 0 <-> 1, 2 <-> 3
    v += dpp_f64<0x140>(v);   // row_mirror: half 0 <-> 1
    return v;
}

// One workgroup per token (s, b), 4 waves.  A row belongs to 16 lanes: lane
// j of the 16 holds dims 4j..4j+3 and 64+4j..64+4j+3 (the pairs it rotates,
// two 16-byte loads), so a wave covers 4 rows per step.  Row h = 16 g +
// 4 wave + lane / 16 for group g.  Each wave issues all its row loads
// first, non-temporal (the F32 rows are read once; the 16-bit outputs are
// stored normally, attention reads them next).  While they are in flight,
// wave 0 forms the 64 pair angles of the token's position (one chain of
// multiplications and one sincosf per lane) and wave 1 stages the two norm
// weight rows; both go through LDS to the other waves, behind one barrier.
// A group in which the wave has no row of the token (K/V past the encoder's
// tokens in the cross form) is skipped after its loads.
template <int OT>
__global__ void __launch_bounds__(256) qk_norm_rope_kernel(const NormRopeArgs a) {
    // (no contraction into fma: each product and sum rounds as written)
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane & 15, sub = lane >> 4;
    // token s of batch b: its Q rows (s < S) and its K/V rows (s < Skv)
    const int T = a.S > a.Skv ? a.S : a.Skv;
    const int s = (int)(blockIdx.x % (unsigned)T), b = (int)(blockIdx.x / (unsigned)T);
    const int H = a.Nh + 2 * a.Nkv;
    const bool q_on = s < a.S, kv_on = s < a.Skv;

    __shared__ float sin_lds[64], cos_lds[64];   // pair angles' sine and cosine
    __shared__ f32x4 w_lds[64];                  // q_w (32 x 4 floats), then k_w

    // weight rows first, so that the wait for them leaves the row loads in flight
    f32x4 wreg = f32x4{0.f, 0.f, 0.f, 0.f};
    if (wave == 1) wreg = *(const f32x4 *)((lane < 32 ? a.q_w : a.k_w) + 4 * (lane & 31));

    // K/V destination row of this token (uniform); out of range: skipped
    int64_t r = s;
    if (a.rows && kv_on) {
        const char *ip = a.rows + (int64_t)s * a.r_nb0 + (int64_t)(b % a.r_ne1) * a.r_nb1;
        r = a.rows_i64 ? *(const int64_t *)ip : (int64_t)*(const int32_t *)ip;
    }
    const bool kv_ok = kv_on && r >= 0 && r < a.kv_rows;
    const int pos = a.rope ? a.pos[s + (int64_t)(a.pos_per_batch ? b : 0) * a.S] : 0;

    f32x4 sn4 = f32x4{0.f, 0.f, 0.f, 0.f}, cs4 = f32x4{1.f, 1.f, 1.f, 1.f};
    for (int g0 = 0; g0 < H; g0 += 16 * kGroups) {
        f32x4 lo[kGroups], hi[kGroups];
        int kind[kGroups], hh[kGroups];
#pragma unroll
        for (int g = 0; g < kGroups; g++) {
            const int h = g0 + 16 * g + 4 * wave + sub;
            kind[g] = h < a.Nh ? (q_on ? 0 : 3) : (h < H ? (kv_on ? (h < a.Nh + a.Nkv ? 1 : 2) : 3) : 3);
            hh[g] = kind[g] == 0 ? h : (kind[g] == 1 ? h - a.Nh : h - a.Nh - a.Nkv);
            // Base and strides are selected as values (a pointer into the
            // argument block would be read through memory, with a wait), and
            // a row that does not exist reads the weight row instead of
            // branching round its load (the branch's join would wait for the
            // data): the loads of all groups issue back to back.
            const int kd = kind[g];
            const char *src = kd == 0 ? a.q : (kd == 1 ? a.k : a.v);
            const int64_t nb0 = kd == 0 ? a.q_nb[0] : (kd == 1 ? a.k_nb[0] : a.v_nb[0]);
            const int64_t nb1 = kd == 0 ? a.q_nb[1] : (kd == 1 ? a.k_nb[1] : a.v_nb[1]);
            const int64_t nb2 = kd == 0 ? a.q_nb[2] : (kd == 1 ? a.k_nb[2] : a.v_nb[2]);
            const float *x = kd < 3 ? (const float *)(src + (int64_t)hh[g] * nb0 + (int64_t)s * nb1 + (int64_t)b * nb2)
                                    : a.q_w;
            lo[g] = __builtin_nontemporal_load((const f32x4 *)(x + 4 * j));
            hi[g] = __builtin_nontemporal_load((const f32x4 *)(x + 64 + 4 * j));
        }
        if (g0 == 0) {
            if (wave == 1) w_lds[lane] = wreg;
            if (wave == 0 && a.rope) {
                // angle of pair `lane`: `lane` float multiplications from
                // theta_0 = pos, then one sincosf
                float th = 0.f, t = (float)pos;
#pragma unroll
                for (int i = 0; i < 64; i++) {
                    th = i == lane ? t : th;
                    t *= a.theta_scale;
                }
                float sn1, cs1;
                sincosf(th, &sn1, &cs1);
                sin_lds[lane] = sn1;
                cos_lds[lane] = cs1;
            }
            __syncthreads();
            if (a.rope) {
                sn4 = *(const f32x4 *)(sin_lds + 4 * j);   // pairs 4j..4j+3
                cs4 = *(const f32x4 *)(cos_lds + 4 * j);
            }
        }
#pragma unroll
        for (int g = 0; g < kGroups; g++) {
            if (g0 + 16 * g >= H) break;   // wave-uniform
            if (__builtin_amdgcn_ballot_w64(kind[g] < 3) == 0) continue;   // no row of this token here
            float y0[4], y1[4];
            // rms_norm: the row's sum of squares (float products) in double
            double ss = 0.0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                y0[e] = lo[g][e];
                y1[e] = hi[g][e];
                ss += (double)(y0[e] * y0[e]);
                ss += (double)(y1[e] * y1[e]);
            }
            ss = row16_sum(ss);
            const int kd = kind[g];
            if (kd < 2) {
                const float mean = (float)(ss / 128.0);
                const float scale = 1.0f / sqrtf(mean + a.eps);
                const f32x4 w0 = w_lds[32 * kd + j], w1 = w_lds[32 * kd + 16 + j];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float u0 = (y0[e] * scale) * w0[e], u1 = (y1[e] * scale) * w1[e];
                    if (a.rope) {
                        y0[e] = u0 * cs4[e] - u1 * sn4[e];
                        y1[e] = u0 * sn4[e] + u1 * cs4[e];
                    } else {
                        y0[e] = u0;
                        y1[e] = u1;
                    }
                }
            } else if (a.clamp_v) {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    y0[e] = fminf(fmaxf(y0[e], -65504.0f), 65504.0f);
                    y1[e] = fminf(fmaxf(y1[e], -65504.0f), 65504.0f);
                }
            }
            u32x2 w0, w1;
            w0[0] = (uint32_t)to16<OT>(y0[0]) | ((uint32_t)to16<OT>(y0[1]) << 16);
            w0[1] = (uint32_t)to16<OT>(y0[2]) | ((uint32_t)to16<OT>(y0[3]) << 16);
            w1[0] = (uint32_t)to16<OT>(y1[0]) | ((uint32_t)to16<OT>(y1[1]) << 16);
            w1[1] = (uint32_t)to16<OT>(y1[2]) | ((uint32_t)to16<OT>(y1[3]) << 16);
            char *row = nullptr;
            if (kd == 0) row = a.q_out + (((int64_t)b * a.S + s) * a.Nh + hh[g]) * 256;
            else if (kd < 3 && kv_ok)
                row = (kd == 1 ? a.k_out : a.v_out) + r * a.kv_nb1 + (int64_t)hh[g] * a.kv_nb2 + (int64_t)b * a.kv_nb3;
            if (row) {
                *(u32x2 *)(row + 8 * j) = w0;
                *(u32x2 *)(row + 128 + 8 * j) = w1;
            }
        }
    }
}

hipError_t launch_qk_norm_rope(const NormRopeArgs &a, int out_type, hipStream_t stream) {
    const int64_t tokens = (int64_t)(a.S > a.Skv ? a.S : a.Skv) * a.B;
    if (tokens <= 0) return hipSuccess;
    const dim3 grid((unsigned)tokens);
    if (out_type == T_F16) hipLaunchKernelGGL(qk_norm_rope_kernel<T_F16>, grid, dim3(256), 0, stream, a);
    else if (out_type == T_BF16) hipLaunchKernelGGL(qk_norm_rope_kernel<T_BF16>, grid, dim3(256), 0, stream, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace mxfa
