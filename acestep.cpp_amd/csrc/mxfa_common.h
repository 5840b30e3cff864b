// mxfa_common.h -- shared device types and helpers for the gfx950 kernels.
//
// Layout conventions used by every kernel (ggml order, ne[0] innermost):
//   q   F32  [D, Sq, Nh, B]   strided view (q_nb1..3)
//   k,v F16/BF16 [D, Skv, Nkv, Bk] (k_nb1..3 / v_nb1..3), or Q8_0 blocks
//   mask F16 [>=Skv, >=Sq, Nm2, Nm3] (m_nb1..3), broadcast by modulo
//   dst F32 [D, Nh, Sq, B] contiguous
// A "row" of the attention problem is one (query iq1, q head) pair; the
// rows that share one KV head (GQA) are packed together into MFMA tiles.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mxfa {

constexpr int kD = 128;                 // head size handled by the kernels
constexpr float kLog2e = 1.4426950408889634f;

enum : int { T_F32 = 0, T_F16 = 1, T_Q8_0 = 8, T_BF16 = 30 };

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// Structured masks (mxfa_flash_attn_ext_masked): the mask as metadata.  Key
// j is live for query row i of batch b iff
//   j < len[b % n_len]            (kSmLengths: padding, qwen3-lm.h:879,
//                                  dit-sampler.h:303)
//   j <= pos0 + i                 (kSmCausal: qwen3-lm.h:605, qwen3-enc.h:433)
//   |pos0 + i - j| <= window      (kSmWindow: dit-sampler.h:282,
//                                  cond-enc.h:317, :341)
// -- the same as a dense F16 mask holding 0 there and -inf elsewhere.
// kSmDevice: lengths (and pos0 when sm_pos0_dev is set) live in device
// memory and are read by the kernels when they run, so a captured launch
// follows values the host rewrites between graph replays.
constexpr int kSmCausal = 1, kSmWindow = 2, kSmLengths = 4, kSmDevice = 8;
constexpr int kSmMaxLen = 64;   // per-batch lengths carried in the arguments

// Arguments shared by the attention kernels (passed by value).
struct FaArgs {
    const char *q, *k, *v, *mask;
    float *dst;
    int64_t q_nb1, q_nb2, q_nb3;
    int64_t k_nb1, k_nb2, k_nb3;
    int64_t v_nb1, v_nb2, v_nb3;
    int64_t m_nb1, m_nb2, m_nb3;
    int32_t m_ne2, m_ne3;
    int32_t Sq, Nh, B, Skv, Nkv, G, rk3;  // G = Nh/Nkv, rk3 = B/Bk
    int32_t M;                            // rows per (b, kv head) = Sq*G
    int32_t row_tiles;                    // decode kernel: ceil(M/16)
    float scale, softcap;                 // softcap == 0: off
    float max_bias, l2m0, l2m1;           // ALiBi (max_bias == 0: off): log2 of ggml's m0, m1
    float softcap_in;                     // scale / softcap (softcap != 0)
    uint32_t n_head_log2;
    // mask row alignment (8 / 16 bytes for every row start); mask_vec4:
    // 8-byte aligned rows holding at least round_up(Skv, 4) entries;
    // mask_vec16: the same with at least 16 entries (16-key DMA blocks)
    int32_t mask_al8, mask_al16, mask_vec4, mask_vec16;
    uint32_t m_plane_bytes;               // prefill: bytes of one mask plane, (ne1 - 1) * nb1 + 2 * ne0
    // split-KV
    int32_t n_splits, chunk;
    int32_t dec_live;                     // > 0: decode grid is the list of live splits (structured masks)
    int32_t dec_pair;                     // > 0: paired splits, the even split of a pair streams dec_pair keys
    float *part_o, *part_ml;
    int *tickets;                         // one per (b, kv head, row tile), zero between calls
    // prefill: per (mask plane, q tile, k tile) class (see fa_mfma.hip), and
    // for the mixed tiles whose values are all 0 or -inf (class 3) one 64-bit
    // liveness word per query row (NULL: no words, no class 3)
    const uint8_t *tile_class;
    uint64_t *tile_bits;
    int32_t n_qt, n_kt;                   // tiles along Sq and Skv
    int32_t n_qt_w;                       // fa_wide.hip: 192-query tiles along Sq (0: not used)
    int32_t n_kt_pad;                     // class row stride (n_kt rounded up to 4)
    // structured mask (sm_flags == 0: none; then `mask` may hold a dense one)
    int32_t q16;                          // Q stored in K's 16-bit type (no conversion on load)
    int32_t sm_flags, sm_window, sm_pos0, sm_nlen;
    const int32_t *sm_len_dev;            // kSmDevice: lengths in device memory (else sm_len)
    const int32_t *sm_pos0_dev;           // kSmDevice: pos0 in device memory, or NULL (sm_pos0)
    int32_t sm_len[kSmMaxLen];
};

// Cross-lane steps at VALU latency (DPP, v_permlane*_swap) instead of LDS
// crossbar permutes (ds_bpermute, ~100 cycles each).
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, false);
}
// AND over the 16 lanes of each row: quad_perm [1,0,3,2] and [2,3,0,1]
// combine each quad, row_half_mirror (i <- 7-i) the two quads of each 8,
// row_mirror (i <- 15-i) the two 8s.  Needs every lane active.
__device__ __forceinline__ uint32_t and_rows16(uint32_t v) {
    v &= dpp_u32<0xB1>(v);
    v &= dpp_u32<0x4E>(v);
    v &= dpp_u32<0x141>(v);
    v &= dpp_u32<0x140>(v);
    return v;
}
// OR over the 16 lanes of each row (the same DPP steps as and_rows16).
__device__ __forceinline__ uint32_t or_rows16(uint32_t v) {
    v |= dpp_u32<0xB1>(v);
    v |= dpp_u32<0x4E>(v);
    v |= dpp_u32<0x141>(v);
    v |= dpp_u32<0x140>(v);
    return v;
}
// max of x over lanes l and l ^ 16 (v_permlane16_swap pairs rows r, r ^ 1)
// and over lanes l and l ^ 32 (v_permlane32_swap pairs the two halves)
__device__ __forceinline__ float max_pair16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                    false, false);
    return fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}
__device__ __forceinline__ float max_half32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                    false, false);
    return fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}

// Live keys [lo, hi) of query row iq1 of batch b under the structured mask
// (both ends are non-decreasing in iq1, so the rows of a tile cover
// [lo(first row), hi(last row)) and all of them see [lo(last), hi(first))).
// With kSmDevice the values come from device memory (the host never calls
// this for such a spec); they are clamped here, as the host checks the
// others: pos0 to [0, 2^30), a negative length to 0.
// The device values are read with relaxed agent-scope atomic loads: a plain
// load would let the compiler fold "device pointer or kernel-argument array"
// into one flat load through a selected pointer, which read wrong lengths.
__device__ __forceinline__ int sm_dev_load(const int32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__host__ __device__ __forceinline__ void sm_row_range(const FaArgs &a, int b, int iq1, int &lo, int &hi) {
    int p0 = a.sm_pos0;
#if defined(__HIP_DEVICE_COMPILE__)
    if (a.sm_pos0_dev) {
        const int d = sm_dev_load(a.sm_pos0_dev);
        p0 = d < 0 ? 0 : (d > (1 << 30) - 1 ? (1 << 30) - 1 : d);
    }
#endif
    const int p = p0 + iq1;
    lo = 0;
    hi = a.Skv;
    if (a.sm_flags & kSmLengths) {
        int len = a.sm_len[b % a.sm_nlen];
#if defined(__HIP_DEVICE_COMPILE__)
        if (a.sm_len_dev) len = sm_dev_load(a.sm_len_dev + b % a.sm_nlen);
#endif
        len = len < 0 ? 0 : len;
        hi = hi < len ? hi : len;
    }
    if (a.sm_flags & kSmCausal) hi = hi < p + 1 ? hi : p + 1;
    if (a.sm_flags & kSmWindow) {
        lo = lo > p - a.sm_window ? lo : p - a.sm_window;
        hi = hi < p + a.sm_window + 1 ? hi : p + a.sm_window + 1;
    }
}

// MFMA 16x16x32 for the two 16-bit float formats (8 k-values per lane).
template <int T> struct Mfma16;
template <> struct Mfma16<T_F16> {
    typedef f16x8 v8;
    static __device__ __forceinline__ f32x4 run(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint16_t from_f32(float x) {
        return __builtin_bit_cast(uint16_t, (_Float16)x);
    }
};
template <> struct Mfma16<T_BF16> {
    typedef bf16x8 v8;
    static __device__ __forceinline__ f32x4 run(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint16_t from_f32(float x) {
        return __builtin_bit_cast(uint16_t, (__bf16)x);
    }
};

// MFMA 32x32x16 for the two 16-bit float formats (8 k-values per lane).
template <int T> struct Mfma32;
template <> struct Mfma32<T_F16> {
    typedef f16x8 v8;
    static __device__ __forceinline__ f32x16 run(v8 a, v8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};
template <> struct Mfma32<T_BF16> {
    typedef bf16x8 v8;
    static __device__ __forceinline__ f32x16 run(v8 a, v8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};

__device__ __forceinline__ float h2f_bits(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// Convert 8 floats to 8 16-bit values of format T (round to nearest even),
// returned as the raw bits.
template <int T>
__device__ __forceinline__ u16x8 cvt8(f32x4 lo, f32x4 hi) {
    u16x8 r;
    r[0] = Mfma16<T>::from_f32(lo[0]);
    r[1] = Mfma16<T>::from_f32(lo[1]);
    r[2] = Mfma16<T>::from_f32(lo[2]);
    r[3] = Mfma16<T>::from_f32(lo[3]);
    r[4] = Mfma16<T>::from_f32(hi[0]);
    r[5] = Mfma16<T>::from_f32(hi[1]);
    r[6] = Mfma16<T>::from_f32(hi[2]);
    r[7] = Mfma16<T>::from_f32(hi[3]);
    return r;
}

// bf16 keeps 8 significant bits: a probability rounded once to bf16 for the
// PV product is off by up to 2^-9 relative, which on short or peaked rows
// moves the output by ~1e-3.  The bf16 kernels therefore feed the PV MFMA
// twice, with hi = RNE_bf16(p) and lo = RNE_bf16(p - hi): hi + lo carries
// p to ~2^-17 relative.  bf16_lo returns the raw bits of lo for the hi
// part `h` (raw bits) of p; p - hi is exact in fp32.
__device__ __forceinline__ uint16_t bf16_lo(float p, uint16_t h) {
    return __builtin_bit_cast(uint16_t, (__bf16)(p - __builtin_bit_cast(float, (uint32_t)h << 16)));
}
__device__ __forceinline__ u16x8 bf16_lo8(f32x4 lo4, f32x4 hi4, u16x8 hi) {
    u16x8 r;
#pragma unroll
    for (int i = 0; i < 8; i++) r[i] = bf16_lo(i < 4 ? lo4[i] : hi4[i - 4], hi[i]);
    return r;
}

// Sum of 8 16-bit values of format T (the rounded probabilities that feed
// the PV product) with v_dot2 against (1, 1): the softmax denominator then
// sums exactly the weights the numerator uses.
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
template <int T>
__device__ __forceinline__ float sum8(u16x8 p, float acc) {
    const u32x4 w = __builtin_bit_cast(u32x4, p);
    if constexpr (T == T_F16) {
        const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t wi = w[i];   // bit_cast of a vector element lvalue reads element 0
            acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, wi), one, acc, false);
        }
    } else {
        const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t wi = w[i];
            acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, wi), one, acc, false);
        }
    }
    return acc;
}

// ALiBi slope of head h (ggml's formula m0^(h+1), or m1^(2(h - n_head_log2)
// + 1); 1 when max_bias == 0), as exp2(e * log2 m) with the host's log2 of
// m0 and m1 (inline: a libm pow call would cost a register save per call
// site).
__device__ __forceinline__ float alibi_slope(const FaArgs &a, int h) {
    if (a.max_bias <= 0.0f) return 1.0f;
    const uint32_t hu = (uint32_t)h;
    return hu < a.n_head_log2 ? __builtin_amdgcn_exp2f(a.l2m0 * (float)(hu + 1))
                              : __builtin_amdgcn_exp2f(a.l2m1 * (float)(2 * (hu - a.n_head_log2) + 1));
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// tanh(x) = 1 - 2 / (e^(2x) + 1) with the hardware exp2 and reciprocal
// (absolute error ~1e-7; saturates to +-1, e^(2x) = inf gives 1).  Inline
// on purpose: a library call inside the attention loops costs a full
// register save per call site.
__device__ __forceinline__ float fast_tanh(float x) {
    const float e = fast_exp2(x * (2.0f * kLog2e));
    return 1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f);
}

// s_waitcnt immediates (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] |
// lgkmcnt[11:8] | vmcnt[5:4] << 14).
#define MXFA_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4) | (0xF << 8))
#define MXFA_WAIT_LGKMCNT0() __builtin_amdgcn_s_waitcnt(0xC07F)

typedef __attribute__((address_space(3))) void lds_void;
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// Direct HBM -> LDS copy of 16 bytes per lane: lane l's bytes land at
// lds_base + 16*l (lds_base must be the same for the whole wave).
//
// Issued as inline assembly on purpose: the compiler's own wait insertion
// treats every LDS read after such a copy as a possible alias and drains
// all outstanding copies (vmcnt(0)) before it, which serialises a
// multi-buffer prefetch.  Callers wait with MXFA_WAIT_VMCNT before reading a
// buffer.  Compiler-generated waits for other vector loads stay correct: a
// copy unknown to the compiler only makes them wait longer (counters retire
// in order).
__device__ __forceinline__ void dma16(const void *g, void *lds_base) {
    const uint32_t lds_addr = (uint32_t)(uintptr_t)(lds_void *)lds_base;
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(g)
                 : "memory", "m0");
}

// Direct HBM -> LDS copy of 4 bytes per lane (4-byte aligned source): lane
// l's bytes land at lds_base + 4*l.  Same contract as dma16.
__device__ __forceinline__ void dma4(const void *g, void *lds_base) {
    const uint32_t lds_addr = (uint32_t)(uintptr_t)(lds_void *)lds_base;
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(g)
                 : "memory", "m0");
}

// Buffer resource over `bytes` bytes from `base`, offset addressed (stride
// 0): a load at or past `bytes` returns zeros and touches no memory.
__device__ __forceinline__ i32x4 buf_rsrc(const void *base, uint32_t bytes) {
    const uint64_t b = (uint64_t)(uintptr_t)base;
    i32x4 r;
    r[0] = (int)__builtin_amdgcn_readfirstlane((uint32_t)b);
    r[1] = (int)((uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) & 0xFFFFu);
    r[2] = (int)__builtin_amdgcn_readfirstlane(bytes);
    r[3] = 0x00020000;   // 32-bit data format, no swizzle, no stride
    return r;
}

// HBM -> LDS copy of 16 bytes per lane through a buffer resource: lane l
// reads base + voff(l) (zeros, and no memory access, when voff(l) + 16
// exceeds the resource's size) and its bytes land at LDS address
// lds_addr + 16*l.  Same wait contract as dma16 (callers wait with
// MXFA_WAIT_VMCNT before reading the buffer).
__device__ __forceinline__ void dma16_buf(const i32x4 &rsrc, uint32_t voff, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds_addr), "v"(voff), "s"(rsrc)
                 : "memory", "m0");
}

// LDS transpose read of four 16-bit values.  Within each group of 16 lanes,
// lane j receives element (j % 4) of the 8-byte chunks addressed by lanes
// j/4 + 4e, e = 0..3 (gfx950 ds_read_b64_tr_b16).
__device__ __forceinline__ u16x4 lds_read_tr16(const void *p) {
    return __builtin_bit_cast(u16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)p));
}

// XOR swizzles of the 16-byte chunks of a 256-byte K or V row stored in
// LDS (key k, logical chunk c at slot c ^ swz(k)).  K: consecutive keys
// read the same chunk (MFMA A operand), k & 15 spreads them over all banks.
// V: transpose reads fetch 4 consecutive keys x 32 bytes per 16 lanes;
// swz_v keeps those (and the neighbouring 16-lane group) conflict-free.
__device__ __forceinline__ int swz_k(int k) { return k & 15; }
__device__ __forceinline__ int swz_v(int k) { return (((k & 3) << 1) ^ ((k & 1) << 3)) ^ (((k >> 2) & 1) << 1); }

}  // namespace mxfa
