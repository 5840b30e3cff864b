// set_rows.hip -- the KV-cache write before every attention call:
// GGML_OP_SET_ROWS with F32 source rows converted to the cache type.
//
// The reference writes the fresh K and V rows of each step into its caches
// with ggml_set_rows (src/qwen3-lm.h:448-454: [D, S, Nkv] F32 rows into the
// [D, max_seq, Nkv] F16 cache, row ids broadcast over the KV heads;
// :760-777: [D, 1, Nkv, N] rows into N consecutive sets of the 4D cache, one
// row id per set).  Semantics (ggml's set_rows):
//
//   dst[:, rows[i, i2 % R1, i3 % R2], i2, i3] = from_float(src[:, i, i2, i3])
//
// with from_float the destination type's conversion: F32 copy, F16 / BF16
// round to nearest even, Q8_0 as ggml's quantize_row_q8_0 (per 32 values:
// amax, d = amax / 127 stored as F16, q = round_half_even(x * 127 / amax)).
//
// The op is a bandwidth-bound scatter: one thread converts 4 consecutive
// values (one 16-byte load) and writes them to the destination row; a Q8_0
// block is 8 threads of one wave, whose amax is a 3-step DPP max.  Rows
// whose id is out of range ([0, dst ne1)) are skipped (ggml aborts on them).

#include "mxfa_common.h"
#include "mxfa_internal.h"

namespace mxfa {

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

template <int DT>
__global__ void __launch_bounds__(256) set_rows_kernel(const SetRowsArgs a) {
    // 32-bit index math: the host limits a launch to < 2^31 chunks
    const uint32_t t = blockIdx.x * 256u + threadIdx.x;
    const uint32_t r = t / a.cpr, c = t - r * a.cpr;     // source row, 4-value chunk
    const bool active = r < a.n_rows;
    const uint32_t rc = active ? r : 0u;
    const uint32_t i01 = rc % a.ne01, i23 = rc / a.ne01;
    const uint32_t i02 = i23 % a.ne02, i03 = i23 / a.ne02;
    const char *ip = a.rows + (int64_t)i01 * a.r_nb0 + (int64_t)(i02 % a.r_ne1) * a.r_nb1 +
                     (int64_t)(i03 % a.r_ne2) * a.r_nb2;
    // the source row does not depend on the row id: both loads are issued
    // together, so a thread waits for one memory round trip, not two
    f32x4 x = {0.f, 0.f, 0.f, 0.f};
    int64_t idx = -1;
    if (active) {
        x = *(const f32x4 *)(a.src + (int64_t)i01 * a.s_nb1 + (int64_t)i02 * a.s_nb2 + (int64_t)i03 * a.s_nb3 +
                             16 * c);
        idx = a.rows_i64 ? *(const int64_t *)ip : (int64_t)*(const int32_t *)ip;
    }
    const bool ok = idx >= 0 && idx < a.dst_ne1;
    char *drow = a.dst + (ok ? idx : 0) * a.d_nb1 + (int64_t)i02 * a.d_nb2 + (int64_t)i03 * a.d_nb3;
    if constexpr (DT == T_Q8_0) {
        // block of 32 values = chunks 8b .. 8b+7 = 8 consecutive lanes (a
        // row holds a multiple of 8 chunks, so blocks never straddle rows)
        // max over the 8 lanes with DPP moves: quad_perm [1,0,3,2] and
        // [2,3,0,1] give each quad its max, row_half_mirror (lane i <- 7-i
        // within 8 lanes) brings in the other quad's
        float amax = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
        amax = fmaxf(amax, dpp_f32<0xB1>(amax));
        amax = fmaxf(amax, dpp_f32<0x4E>(amax));
        amax = fmaxf(amax, dpp_f32<0x141>(amax));
        if (!ok) return;
        const float d = amax / 127.0f;
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        const uint32_t blk = c >> 3, j = c & 7;
        char *yb = drow + 34 * blk;
        uint8_t q[4];
#pragma unroll
        for (int i = 0; i < 4; i++) q[i] = (uint8_t)(int8_t)(int)__builtin_rintf(x[i] * id);
        // qs bytes 4j .. 4j+3 sit at block offset 2 + 4j: 2-byte aligned
        uint16_t *qs = (uint16_t *)(yb + 2 + 4 * j);
        qs[0] = (uint16_t)(q[0] | (q[1] << 8));
        qs[1] = (uint16_t)(q[2] | (q[3] << 8));
        if (j == 0) *(uint16_t *)yb = __builtin_bit_cast(uint16_t, (_Float16)d);
    } else {
        if (!ok) return;
        if constexpr (DT == T_F32) {
            *(f32x4 *)(drow + 16 * c) = x;
        } else if constexpr (DT == T_F16) {
            const f16x2 lo = {(_Float16)x[0], (_Float16)x[1]}, hi = {(_Float16)x[2], (_Float16)x[3]};
            *(u32x2 *)(drow + 8 * c) = u32x2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
        } else {
            const bf16x2 lo = {(__bf16)x[0], (__bf16)x[1]}, hi = {(__bf16)x[2], (__bf16)x[3]};
            *(u32x2 *)(drow + 8 * c) = u32x2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
        }
    }
}

hipError_t launch_set_rows(const SetRowsArgs &a, int dtype, hipStream_t stream) {
    const int64_t threads = (int64_t)a.n_rows * a.cpr;
    if (threads <= 0) return hipSuccess;
    if (threads >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((threads + 255) / 256));
    switch (dtype) {
        case T_F32: hipLaunchKernelGGL(set_rows_kernel<T_F32>, grid, dim3(256), 0, stream, a); break;
        case T_F16: hipLaunchKernelGGL(set_rows_kernel<T_F16>, grid, dim3(256), 0, stream, a); break;
        case T_BF16: hipLaunchKernelGGL(set_rows_kernel<T_BF16>, grid, dim3(256), 0, stream, a); break;
        case T_Q8_0: hipLaunchKernelGGL(set_rows_kernel<T_Q8_0>, grid, dim3(256), 0, stream, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace mxfa
