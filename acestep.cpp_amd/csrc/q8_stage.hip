// q8_stage.hip -- the K/V rows of a prefill over a Q8_0 KV cache, staged in
// F16 for the MFMA prefill kernel.
//
// ggml's CPU flash_attn_ext over a Q8_0 cache
// (ggml_compute_forward_flash_attn_ext_f16_one_chunk; ggml is the
// reference's submodule, not vendored) quantises each Q row to Q8_0 (the
// vec_dot type of Q8_0) and forms q . k as integer block dots scaled by
// d_q d_k; V rows are dequantised to F32 (q * d) and accumulated in F32.
// The reference reaches it from src/qwen3-lm.h's prompt path over a Q8_0
// cache (a prompt continued at kv_pos > 0).  This pass writes
//   K' = f16(q_k * d_k),  V' = f16(q_v * d_v)
// each product exact in F32 (8-bit times 11-bit) and rounded once to F16;
// the prefill kernel quantises Q to Q8_0 on load as ggml does and uses
// Q' = f16(q_q * d_q) (fa_prefill_q8q_kernel).  Its F16 products of Q' and
// K' are exact in its F32 accumulators, so the scores differ from ggml's
// integer dots only by the two F16 roundings (relative 2^-11 per factor),
// and P V by V's rounding, as in the decode kernel, which dequantises V to
// F16 the same way.  Values beyond F16's range (|q d| > 65504) become
// infinite.
//
// One thread writes 8 values (16 bytes) of one staged row: 16 threads per
// row of 128.  Rows [0, n_kv) are K rows, [n_kv, 2 n_kv) V rows.

#include "mxfa_common.h"
#include "mxfa_internal.h"

namespace mxfa {

__global__ void __launch_bounds__(256) q8_stage_kernel(const Q8StageArgs a) {
    const uint32_t t = blockIdx.x * 256u + threadIdx.x;
    const uint32_t row = t >> 4, j = t & 15;   // staged row, 8-value chunk
    if (row >= 2 * a.n_kv) return;
    float y[8];
    char *dst;
    {
        const bool is_v = row >= a.n_kv;
        const uint32_t r = is_v ? row - a.n_kv : row;
        const uint32_t key = r % a.Skv, rest = r / a.Skv, kvh = rest % a.Nkv, bk = rest / a.Nkv;
        const char *src = is_v ? a.v + (int64_t)key * a.v_nb1 + (int64_t)kvh * a.v_nb2 + (int64_t)bk * a.v_nb3
                               : a.k + (int64_t)key * a.k_nb1 + (int64_t)kvh * a.k_nb2 + (int64_t)bk * a.k_nb3;
        // block j / 4 (34 bytes: fp16 d, 32 int8), its values 8 (j % 4) ..
        const char *bp = src + 34 * (j >> 2);
        const float d = (float)__builtin_bit_cast(_Float16, *(const uint16_t *)bp);
        // the 8 bytes at bp + 2 + 8 (j % 4) start 2 bytes past a 4-byte
        // boundary in even blocks and on one in odd blocks (rows are 4-byte
        // aligned): read the dwords that cover them and shift
        const char *qp = bp + 2 + 8 * (j & 3);
        const uint32_t sh = (uint32_t)(uintptr_t)qp & 3u;
        const uint32_t *wp = (const uint32_t *)(qp - sh);
        const uint32_t w0 = wp[0], w1 = wp[1];
        const uint32_t w2 = sh ? wp[2] : 0u;
        // ({w1, w0} >> 8 sh bytes): the shift operand counts bytes
        const uint32_t lo = __builtin_amdgcn_alignbyte(w1, w0, sh);
        const uint32_t hi = __builtin_amdgcn_alignbyte(w2, w1, sh);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            y[e] = (float)(int8_t)(lo >> (8 * e)) * d;
            y[4 + e] = (float)(int8_t)(hi >> (8 * e)) * d;
        }
        dst = (is_v ? a.vs : a.ks) + (int64_t)r * 256 + 16 * j;
    }
    u32x4 w;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const f16x2 p = {(_Float16)y[2 * e], (_Float16)y[2 * e + 1]};
        w[e] = __builtin_bit_cast(uint32_t, p);
    }
    *(u32x4 *)dst = w;
}

hipError_t launch_q8_stage(const Q8StageArgs &a, hipStream_t stream) {
    const int64_t threads = 16 * (int64_t)2 * a.n_kv;
    if (threads <= 0) return hipSuccess;
    if (threads >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(q8_stage_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace mxfa
