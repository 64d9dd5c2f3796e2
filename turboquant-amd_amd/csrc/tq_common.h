// Shared device helpers for the TurboQuant gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "turboquant_hip.h"

#define TQ_ABI_VERSION 4
#define TQ_HEAD_DIM 128
#define TQ_WAVE 64

typedef _Float16 tq_half8 __attribute__((ext_vector_type(8)));
typedef _Float16 tq_half4 __attribute__((ext_vector_type(4)));
typedef float tq_floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t tq_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t tq_u32x2 __attribute__((ext_vector_type(2)));

// ---- scalar conversions ---------------------------------------------------------

__device__ __forceinline__ float tq_bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

__device__ __forceinline__ float tq_f16_to_f32(uint32_t bits16) {
    _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits16);
    return (float)h;
}

// fp32 -> fp16 bits, round to nearest even (hardware v_cvt_f16_f32).
__device__ __forceinline__ uint32_t tq_f32_to_f16_bits(float f) {
    _Float16 h = (_Float16)f;
    return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

// fp32 -> bf16 bits, round to nearest even, NaN kept quiet.
__device__ __forceinline__ uint32_t tq_f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

__device__ __forceinline__ uint32_t tq_pack_half2(float lo, float hi) {
    return tq_f32_to_f16_bits(lo) | (tq_f32_to_f16_bits(hi) << 16);
}

// Load 8 consecutive elements of dtype `dt` starting at element `off` of `base` as fp32.
// The address of element `off` must be 16-byte aligned for f16/bf16 and 32-byte for f32.
__device__ __forceinline__ void tq_load8(const void* base, int64_t off, int dt, float v[8]) {
    if (dt == TQ_F32) {
        const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + off);
        float4 a = p[0], b = p[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
        tq_u32x4 w = *reinterpret_cast<const tq_u32x4*>(static_cast<const uint16_t*>(base) + off);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            uint32_t lo = w[k] & 0xffffu, hi = w[k] >> 16;
            if (dt == TQ_BF16) {
                v[2 * k] = tq_bf16_to_f32(lo);
                v[2 * k + 1] = tq_bf16_to_f32(hi);
            } else {
                v[2 * k] = tq_f16_to_f32(lo);
                v[2 * k + 1] = tq_f16_to_f32(hi);
            }
        }
    }
}

__device__ __forceinline__ float tq_load1(const void* base, int64_t off, int dt) {
    if (dt == TQ_F32) return static_cast<const float*>(base)[off];
    uint32_t b = static_cast<const uint16_t*>(base)[off];
    return dt == TQ_BF16 ? tq_bf16_to_f32(b) : tq_f16_to_f32(b);
}

__device__ __forceinline__ void tq_store1(void* base, int64_t off, int dt, float v) {
    if (dt == TQ_F32) {
        static_cast<float*>(base)[off] = v;
    } else {
        uint32_t b = dt == TQ_BF16 ? tq_f32_to_bf16_bits(v) : tq_f32_to_f16_bits(v);
        static_cast<uint16_t*>(base)[off] = (uint16_t)b;
    }
}

// ---- bit-field extraction from a little-endian array of 32-bit words -----------------
// Returns bits [pos, pos+width) of the stream w[]; pos/width are compile-time after unrolling.
template <int N>
__device__ __forceinline__ uint32_t tq_field(const uint32_t (&w)[N], int pos, int width) {
    const int wi = pos >> 5, sh = pos & 31;
    const uint32_t mask = (width >= 32) ? 0xffffffffu : ((1u << width) - 1u);
    if (sh + width <= 32 || wi + 1 >= N) return (w[wi] >> sh) & mask;
    return __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh) & mask;
}

// ---- division by a runtime divisor as a multiply-high and a shift ---------------------------
// For 2 <= d < 2^31 with l = ceil(log2 d) and m = ceil(2^(31 + l) / d) (which fits 32 bits),
// floor(n / d) = floor(n m / 2^(31 + l)) for every n < 2^31: m = 2^(31 + l) / d + e with
// 0 <= e < 1, so the excess n e / 2^(31 + l) stays below 1 / d because 2^(31 + l) / d >= 2^31 > n.
// d = 1 is m = 0 (q = n).
struct tq_udiv {
    uint32_t m;
    int32_t sh;  // l - 1
};
inline tq_udiv tq_make_udiv(uint32_t d) {
    tq_udiv v = {0u, 0};
    if (d <= 1) return v;
    int l = 0;
    while ((1ull << l) < d) ++l;
    v.m = (uint32_t)(((1ull << (31 + l)) + d - 1) / d);
    v.sh = l - 1;
    return v;
}
__device__ __forceinline__ uint32_t tq_udiv_apply(uint32_t n, tq_udiv v) {
    return v.m ? (__umulhi(n, v.m) >> v.sh) : n;
}

// ---- correctly rounded quotient by a per-row divisor ------------------------------
// q = RN(x / d) given rcp = RN(1/d): one residual correction of the product (Markstein).
// The residual uses d clamped to FLT_MAX, so d = inf gives x * 0 = 0 for finite x (as x / inf
// does) instead of NaN; the clamp is the same for every x of a row and is computed once.
__device__ __forceinline__ float tq_div_rn(float x, float d, float rcp) {
    float q0 = x * rcp;
    float e = __builtin_fmaf(-q0, __builtin_fminf(d, 3.40282347e38f), x);
    return __builtin_fmaf(e, rcp, q0);
}

// ---- Walsh-Hadamard butterflies: x -> x H for the Sylvester matrix H[i][j] = (-1)^popcount(i & j)
// (unscaled; the caller multiplies by 1/sqrt(128)).  Each stage pairs the elements whose
// index differs in one bit, so the stages may run in any order and over any mix of register
// index bits and lane bits, as long as every index bit gets exactly one stage.
template <int N>
__device__ __forceinline__ void tq_wht_regs(float (&x)[N]) {
    constexpr int kStages = N >= 32 ? 5 : N >= 16 ? 4 : N >= 8 ? 3 : N >= 4 ? 2 : 1;
    static_assert(N == (1 << kStages), "N must be a power of two in 2..32");
#pragma unroll
    for (int st = 0; st < kStages; ++st)
#pragma unroll
        for (int j = 0; j < N / 2; ++j) {
            // j-th pair of stage st: indices i (bit st clear) and i + 2^st
            const int i = ((j >> st) << (st + 1)) | (j & ((1 << st) - 1));
            const float a = x[i], b = x[i + (1 << st)];
            x[i] = a + b;
            x[i + (1 << st)] = a - b;
        }
}
// The stage across lanes l and l ^ m (m a power of two below 64): the lower lane gets a + b, the
// upper a - b, where a is the lower lane's value.  Every lane of the wave must take part.
__device__ __forceinline__ float tq_wht_lane(float x, int m) {
    const float y = __shfl_xor(x, m, 64);
    return (__lane_id() & m) ? y - x : x + y;
}
// A 128-element row spread over lanes l, l^16, l^32, l^48, 32 elements each (lane group
// g = l / 16 holds elements 32g + i in x[i], or any layout that maps the element bits 5-6 to
// lane bits 4-5): x <- (x H) * h.
__device__ __forceinline__ void tq_wht_row_g4(float (&x)[32], float h) {
    tq_wht_regs(x);
#pragma unroll
    for (int i = 0; i < 32; ++i) x[i] = tq_wht_lane(tq_wht_lane(x[i], 16), 32) * h;
}
// Paged tile geometry (must match tq_tile_bytes / tq_tile_offsets on the host).
struct tq_tile_geom {
    int64_t off_signs, off_norm, off_rnorm, bytes;
};
__host__ __device__ inline tq_tile_geom tq_make_tile_geom(int block_size, int bits, int qjl) {
    tq_tile_geom g;
    const int64_t idx_bytes = (int64_t)block_size * 16 * bits;
    g.off_signs = idx_bytes;
    g.off_norm = idx_bytes + (qjl ? (int64_t)block_size * 16 : 0);
    g.off_rnorm = g.off_norm + (int64_t)block_size * 2;
    g.bytes = g.off_norm + (int64_t)block_size * 2 + (qjl ? (int64_t)block_size * 2 : 0);
    return g;
}
