// PolarQuant compression kernels for gfx950.
//
// A wave64 works on 16 rows and a 256-thread workgroup on 64 rows, 32 dims of a row per lane.
// 16-bit rows of the paged kernels are rotated on the matrix cores (one row per lane and lane
// group, rotate_mfma); fp32 rows and polarquant_compress keep 4 consecutive lanes per row and a
// Walsh-Hadamard rotation of 5 in-register butterfly stages (dim bits 0-4) plus 2 cross-lane
// stages (DPP, no LDS).  Indices come from an LDS cell table of the boundaries (129 cells in the
// paged kernels, 257 for polarquant_compress; one compare per value); each lane stores its
// 4 * bits packed bytes at once.
// Row math follows turboquant/core/quantizer.py:141-174:
//   x_rot = x @ H; norm = |x_rot|; x_n = x_rot / (norm + 1e-8); idx = #{b < x_n};
//   r = (x_n - c[idx]) * norm; rnorm = |r|; sign = r >= 0.
#include "tq_common.h"

namespace {

enum { MODE_UNPACKED = 0, MODE_PAGED = 1 };

struct CompressParams {
    const void* x;
    int x_dtype;
    int64_t x_stride_token;  // elements
    int64_t x_stride_head;   // elements
    int64_t num_tokens;
    int num_heads;
    int64_t tok_rows;        // rows per head: num_tokens, rounded up to 4 in paged mode
    int64_t n_rows;          // tok_rows * num_heads
    int rotate;
    float wht_scale;
    const float* centroids;
    const float* boundaries;
    // paged output
    const void* slot_mapping;
    int slot_i64;
    uint8_t* cache;
    int64_t stride_block, stride_head, num_blocks;
    int block_size;
    int idx32;  // rows and slots below 2^31: 32-bit index arithmetic
    tq_udiv tok_div, blk_div;  // by tok_rows and block_size (32-bit index arithmetic)
    int tile_layout;  // TQ_TILE_ROWS / TQ_TILE_KEYS / TQ_TILE_VALUES
    int64_t off_signs, off_norm, off_rnorm;  // region offsets from the tile (or idx region) base
    int64_t rs_idx, rs_sig, rs_norm;          // row strides of the index, sign and norm regions
    int narrow;                               // index / sign rows only 2-byte aligned: 16-bit stores
    // unpacked output
    int64_t* indices;
    float* norms;
    float* k_mse;
    float* signs;
    float* rnorm;
};

// Lane layout: 4 lanes per 128-dim row, lane q = L & 3 of the row holding dims 32q..32q+31;
// a wave works on 16 rows and a 256-thread workgroup on 64.  Five Hadamard stages (dims bits
// 0-4) run in registers, two (dims bits 5, 6 = lane bits 0, 1) through DPP quad_perm.
constexpr int kRowsPerWG = 64;
// Grid of the grid-stride compress launches: one round of the workgroups the device holds at
// once (CUs x resident 256-thread workgroups of the kernel instance, from the occupancy query),
// so every workgroup builds its LDS table once and no second, partial round is left over.
// Measured on config 2 (fused K + V, 4 resident workgroups per CU): 512 per tensor (one round)
// 23.8 us, 1024 (two rounds) 23.9-24.1 us, 768 24.6 us, 1536 25.1 us, 2048 25.8 us.
template <typename K>
int resident_grid(K kernel) {
    int dev = 0, cus = 0, per = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, 256, 0) != hipSuccess || per <= 0 || cus <= 0)
        return 1024;
    return per * cus;
}
constexpr int kDppXor1 = 0xB1;  // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;  // quad_perm [2, 3, 0, 1]
template <int CTRL>
__device__ __forceinline__ float dppf(float x) {
    // bound_ctrl with a zero old value: lets the compiler fold the move into a consuming add
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, true));
}

// Sum of x[k]^2 over the row, associated as an 8-term fma chain per 8 dims followed by an xor
// butterfly over dims bits 3, 4, 5, 6 (the order is part of the result: every lane of the row
// gets the same bits, and the same bits as a 16-lanes-per-row butterfly would).
__device__ __forceinline__ float row_sumsq(const float (&x)[32]) {
    float s[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        s[j] = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k) s[j] = __builtin_fmaf(x[8 * j + k], x[8 * j + k], s[j]);
    }
    float t = (s[0] + s[1]) + (s[2] + s[3]);
    t += dppf<kDppXor1>(t);
    t += dppf<kDppXor2>(t);
    return t;
}

// v[k] += s * (v[k] of lane L ^ 1 (CTRL = quad_perm [1,0,3,2]) or L ^ 2 ([2,3,0,1])), 32 values:
// one fma per value on the DPP-moved partner (s = +-1, so the product is exact and the fma rounds
// once, as a v_fmac_f32_dpp would).  The moves are compiler builtins, so the wait states between
// a VALU write and a DPP read of the same register are the compiler's to place.
template <int CTRL>
__device__ __forceinline__ void fmac_dpp32(float (&v)[32], float s) {
    static_assert(CTRL == kDppXor1 || CTRL == kDppXor2, "quad_perm xor 1 or xor 2");
#pragma unroll
    for (int k = 0; k < 32; ++k) v[k] = __builtin_fmaf(dppf<CTRL>(v[k]), s, v[k]);
}

// Normalised Hadamard transform of the row (dims 32q + k in v[k]): butterflies
// (u, w) -> (u + w, u - w) over dims bits 0..6, then the scale h.  A cross-lane stage computes
// own + s * partner (s = -1 in the upper lane): the upper lane then holds -(u - w), exactly;
// partners of a later stage agree in the earlier stage bits, so the negations collect into the
// per-lane sign (-1)^(q bit 0 + q bit 1) that the final scale undoes.
__device__ __forceinline__ void wht_row(float (&v)[32], int q, float h) {
#pragma unroll
    for (int b = 1; b < 32; b <<= 1) {
#pragma unroll
        for (int k = 0; k < 32; ++k) {
            if (!(k & b)) {
                const float u = v[k], w = v[k | b];
                v[k] = u + w;
                v[k | b] = u - w;
            }
        }
    }
    const float s0 = (q & 1) ? -1.f : 1.f, s1 = (q & 2) ? -1.f : 1.f;
    fmac_dpp32<kDppXor1>(v, s0);
    fmac_dpp32<kDppXor2>(v, s1);
    const float hs = (s0 * s1) * h;
#pragma unroll
    for (int k = 0; k < 32; ++k) v[k] *= hs;
}

// A lane's 32 input elements of a row as raw words: 4 x 16 bytes for 16-bit types, 8 x 16 for fp32.
template <int DT>
struct RawRow {
    tq_u32x4 w[DT == TQ_F32 ? 8 : 4];
};
template <int DT>
__device__ __forceinline__ void load_raw(const void* base, int64_t off, RawRow<DT>& r) {
    constexpr int N = DT == TQ_F32 ? 8 : 4;
    const tq_u32x4* p = DT == TQ_F32 ? reinterpret_cast<const tq_u32x4*>(static_cast<const float*>(base) + off)
                                     : reinterpret_cast<const tq_u32x4*>(static_cast<const uint16_t*>(base) + off);
#pragma unroll
    for (int i = 0; i < N; ++i) r.w[i] = p[i];
}
template <int DT>
__device__ __forceinline__ void raw_to_float(const RawRow<DT>& r, float (&v)[32]) {
#pragma unroll
    for (int i = 0; i < (DT == TQ_F32 ? 8 : 4); ++i)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t w = r.w[i][k];
            if (DT == TQ_F32) {
                v[4 * i + k] = __uint_as_float(w);
            } else if (DT == TQ_BF16) {
                v[8 * i + 2 * k] = tq_bf16_to_f32(w & 0xffffu);
                v[8 * i + 2 * k + 1] = tq_bf16_to_f32(w >> 16);
            } else {
                v[8 * i + 2 * k] = tq_f16_to_f32(w & 0xffffu);
                v[8 * i + 2 * k + 1] = tq_f16_to_f32(w >> 16);
            }
        }
}

// The paged kernels' rotation of fp32 rows without its scale: v <- x H (H the +-1 Sylvester
// matrix), so that y = h v.  The lane's inputs enter multiplied by sigma = (-1)^(q bit 0 + q bit 1);
// the cross-lane stages then compute own - partner in the lower lane and own + partner in the
// upper, and each leaves the right sign (a lower lane's partner arrives negated relative to it,
// stage by stage), so no final negation or scale pass is needed.  (16-bit rows take the
// matrix-core rotation below.)
__device__ __forceinline__ void rotate_unscaled_f32(const RawRow<TQ_F32>& r, int q, float (&v)[32]) {
    const bool neg = ((q ^ (q >> 1)) & 1) != 0;
    raw_to_float<TQ_F32>(r, v);
    const float sg = neg ? -1.f : 1.f;
#pragma unroll
    for (int k = 0; k < 32; ++k) v[k] *= sg;
#pragma unroll
    for (int b = 1; b < 32; b <<= 1) {
#pragma unroll
        for (int k = 0; k < 32; ++k) {
            if (!(k & b)) {
                const float u = v[k], w = v[k | b];
                v[k] = u + w;
                v[k | b] = u - w;
            }
        }
    }
    fmac_dpp32<kDppXor1>(v, (q & 1) ? 1.f : -1.f);
    fmac_dpp32<kDppXor2>(v, (q & 2) ? 1.f : -1.f);
}

// ---- 16-bit paged rows on the matrix cores ----
// A wave holds 16 rows; lane l works on row l & 15 with lane group G = l >> 4.  The rotation
// z^T = H x^T runs as 32 v_mfma_f32_16x16x32 (bf16 / f16 products are exact, fp32 accumulation)
// with the +-1 matrix as the A operand and the rows as B: lane l's B operand of K step kk is the
// 16-byte load of row l & 15 at dims 32 kk + 8 G + (0..7), and its output tile t = 2 s + u
// (s = 0..3, u = 0..1) holds dims 32 s + 8 G + 4 u + (0..3) of that row, in v[4 t .. 4 t + 3].
// So a lane holds 8 consecutive dims of each 32-dim quarter s: group s of the lane is dims
// 32 s + 8 G .. + 7.  A[o][in] = (-1)^popcount(o & in) with o = 32 s + 8 (m >> 2) + 4 u + (m & 3)
// (m = l & 15, A's row) and in = 32 kk + 8 G + j: the sign factors into a per-lane pattern that
// depends on u only and the lane-uniform (-1)^popcount(s & kk), so four fragments serve all 32
// products.  Packed bits leave the kernel per quarter: a 4 x 4 transpose across the row's lanes
// (two permlane32 and two permlane16 swaps per four words) gives lane G the words of dims
// 32 G .. 32 G + 31, which the tile stores expect.
typedef __bf16 tq_bf16x8 __attribute__((ext_vector_type(8)));
template <int DT>
struct HadamardFrags {
    tq_u32x4 f[2][2];  // [u][negated]
};
template <int DT>
__device__ __forceinline__ HadamardFrags<DT> hadamard_frags(int lane) {
    const uint32_t one = DT == TQ_BF16 ? 0x3F80u : 0x3C00u;
    const int m = lane & 15, g = lane >> 4;
    const int e0 = __builtin_popcount((m >> 2) & g);
    HadamardFrags<DT> h;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int pw = 0; pw < 4; ++pw) {
            uint32_t w = 0;
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int j = 2 * pw + hh;
                const int e = e0 + __builtin_popcount((m & 3) & (j & 3)) + (u & (j >> 2));
                w |= (one | ((e & 1) ? 0x8000u : 0u)) << (16 * hh);
            }
            h.f[u][0][pw] = w;
            h.f[u][1][pw] = w ^ 0x80008000u;
        }
    return h;
}
template <int DT>
__device__ __forceinline__ tq_floatx4 mfma_rows(const tq_u32x4& a, const tq_u32x4& b, const tq_floatx4& c) {
    if constexpr (DT == TQ_BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(tq_bf16x8, a), __builtin_bit_cast(tq_bf16x8, b),
                                                       c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(tq_half8, a), __builtin_bit_cast(tq_half8, b), c,
                                                      0, 0, 0);
}
// v <- x H (unscaled) of the lane's row, in the group order above; r.w[kk] = the K step kk operand
template <int DT>
__device__ __forceinline__ void rotate_mfma(const RawRow<DT>& r, const HadamardFrags<DT>& h, float (&v)[32]) {
    tq_floatx4 acc[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = tq_floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int t = 0; t < 8; ++t) acc[t] = mfma_rows<DT>(h.f[t & 1][__builtin_popcount((t >> 1) & kk) & 1], r.w[kk], acc[t]);
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) v[4 * t + i] = acc[t][i];
}
// A lane's four K-step operands: 16 bytes at dims 32 kk + 8 G of its row (off includes 8 G)
template <int DT>
__device__ __forceinline__ void load_raw_groups(const void* base, int64_t off, RawRow<DT>& r) {
    const tq_u32x4* p = reinterpret_cast<const tq_u32x4*>(static_cast<const uint16_t*>(base) + off);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) r.w[kk] = p[4 * kk];
}
// g[s] of lane G (the row's lane groups G = 0..3, 16 lanes apart) becomes g[s] of lane s's
// slot G: after the two stages lane G slot w holds what lane w held in slot G.
__device__ __forceinline__ void transpose_groups(uint32_t (&g)[4]) {
    auto a = __builtin_amdgcn_permlane32_swap(g[0], g[2], false, false);  // lanes 32 apart: slots 0 <-> 2
    auto b = __builtin_amdgcn_permlane32_swap(g[1], g[3], false, false);
    g[0] = a[0];
    g[2] = a[1];
    g[1] = b[0];
    g[3] = b[1];
    auto c = __builtin_amdgcn_permlane16_swap(g[0], g[1], false, false);  // lanes 16 apart: slots 0 <-> 1
    auto d = __builtin_amdgcn_permlane16_swap(g[2], g[3], false, false);
    g[0] = c[0];
    g[1] = c[1];
    g[2] = d[0];
    g[3] = d[1];
}
// Sum of squares of the row held by the four lanes l, l ^ 16, l ^ 32, l ^ 48 (8-term fma chain
// per group, then (s0 + s1) + (s2 + s3), then the two cross-lane sums: every lane of the row
// gets the same bits).
__device__ __forceinline__ float row_sumsq_groups(const float (&x)[32]) {
    float s[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        s[j] = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k) s[j] = __builtin_fmaf(x[8 * j + k], x[8 * j + k], s[j]);
    }
    const float t = (s[0] + s[1]) + (s[2] + s[3]);
    auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(t), __float_as_uint(t), false, false);
    const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
template <bool GROUPS>
__device__ __forceinline__ float row_sumsq_of(const float (&x)[32]) {
    if constexpr (GROUPS) return row_sumsq_groups(x);
    else return row_sumsq(x);
}

// Left searchsorted over NB sorted boundaries (count of boundaries < x) for |x| <= 1 through a
// table of 256 cells of width 1/128 over [-1, 1] (plus one cell for x = 1): cell k holds
// c0 = #{b < edge_k - eps} and the one boundary inside [edge_k - eps, edge_k+1 + eps] (or +inf),
// so idx = c0 + (b < x).  The cell is trunc(128 x + 128), exact to 2^-16 in cell units (eps =
// 1e-5 is 160 times that).  A codebook with two boundaries in one such cell sets `bad`, and the
// kernel then counts linearly.  NaN is handled by the caller.
constexpr int kCells = 257;
template <int NB>
__device__ __forceinline__ void build_cells(const float (&bd)[NB], const float* boundaries, uint2* tab, int* bad) {
    constexpr float eps = 1e-5f;
    for (int k = threadIdx.x; k < kCells; k += blockDim.x) {
        const float e0 = -1.f + (float)k * (1.f / 128.f) - eps, e1 = -1.f + (float)(k + 1) * (1.f / 128.f) + eps;
        int c0 = 0, c1 = 0;
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            c0 += bd[i] < e0 ? 1 : 0;
            c1 += bd[i] <= e1 ? 1 : 0;
        }
        if (c1 - c0 > 1) atomicOr(bad, 1);
        const float b = c1 > c0 ? boundaries[c0] : __builtin_huge_valf();
        tab[k] = make_uint2(__float_as_uint(b), (uint32_t)c0);
    }
}
__device__ __forceinline__ int quant_cell(float x, const uint2* tab) {
    const uint2 e = tab[(int)__builtin_fmaf(x, 128.f, 128.f)];
    return (int)e.y + (__uint_as_float(e.x) < x ? 1 : 0);
}
template <int NB>
__device__ __forceinline__ int quant_linear(float x, const float (&bd)[NB]) {
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < NB; ++i) cnt += (bd[i] < x) ? 1 : 0;
    return x != x ? NB : cnt;
}

// Paged mode: round-to-nearest cells and decisions on z itself.  Cell k (0..128) covers
// 64 x + 64 in [k - 1/2, k + 1/2] and holds c0 = #{b < lo_k - eps} and the one boundary inside
// [lo_k - eps, hi_k + eps] (or +inf); the cell of x = z / den is the low mantissa bits of
// fl(z (64 / den) + 64 + 1.5 * 2^23) (one fma; a tie lands in either neighbour, both cover it,
// and the approximate 64 / den moves x by far less than eps).  The decision b < z / den is the
// sign of b den - z, one fma of the exact product (den > 0): exact for this z, with no rounded
// quotient in between.  Cells of width 1/64 (the d = 128 codebooks keep at least 0.023 between
// boundaries): the cells a row's values fall in (x ~ N(0, 1/128)) then lie within one period of
// the LDS banks, which the 1/128 table's lookups did not (measured: 2.5 % faster on config 2).
constexpr int kCellsRn = 129;
constexpr float kCellsRnScale = 64.f;
constexpr float kCellMagic = 12583040.f - 64.f;   // 1.5 * 2^23 + 64
constexpr uint32_t kCellMagicBase = 0x4B400000u;  // bits of 1.5 * 2^23
template <int NB>
__device__ __forceinline__ void build_cells_rn(const float (&bd)[NB], const float* boundaries, uint2* tab, int* bad) {
    constexpr float eps = 1e-5f;
    for (int k = threadIdx.x; k < kCellsRn; k += blockDim.x) {
        const float lo = ((float)k - 64.5f) * (1.f / 64.f) - eps, hi = ((float)k - 63.5f) * (1.f / 64.f) + eps;
        int c0 = 0, c1 = 0;
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            c0 += bd[i] < lo ? 1 : 0;
            c1 += bd[i] <= hi ? 1 : 0;
        }
        if (c1 - c0 > 1) atomicOr(bad, 1);
        const float b = c1 > c0 ? boundaries[c0] : __builtin_huge_valf();
        tab[k] = make_uint2(__float_as_uint(b), (uint32_t)c0);
    }
}
__device__ __forceinline__ int quant_cell_y(float z, float den, float rscale, const uint2* tab) {
    const uint2 e = tab[__float_as_uint(__builtin_fmaf(z, rscale, kCellMagic)) - kCellMagicBase];
    return (int)e.y + (__builtin_fmaf(__uint_as_float(e.x), den, -z) < 0.f ? 1 : 0);
}

// The lane's 32 indices as 4 * BITS bytes of the little-endian BITS-bit stream.  2 and 4 bits
// (fields never straddle a word): a tree of v_lshl_or_b32, one per field after the first of
// each word (the compiler's form took a shift per field and an or3 per two).
__device__ __forceinline__ uint32_t lshl_or(uint32_t a, int sh, uint32_t b) {
    uint32_t r;
    asm("v_lshl_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "i"(sh), "v"(b));
    return r;
}
template <int BITS>
__device__ __forceinline__ void pack_stream(const int (&idx)[32], uint32_t (&w)[BITS]) {
    if constexpr (BITS == 4 || BITS == 2) {
        constexpr int F = 32 / BITS;  // fields per word
#pragma unroll
        for (int j = 0; j < BITS; ++j) {
            uint32_t t[F];
#pragma unroll
            for (int k = 0; k < F; ++k) t[k] = (uint32_t)idx[F * j + k];
#pragma unroll
            for (int span = 1, sh = BITS; span < F; span *= 2, sh *= 2)
#pragma unroll
                for (int k = 0; k < F; k += 2 * span) t[k] = lshl_or(t[k + span], sh, t[k]);
            w[j] = t[0];
        }
    } else {
#pragma unroll
        for (int j = 0; j < BITS; ++j) w[j] = 0;
#pragma unroll
        for (int k = 0; k < 32; ++k) {
            const int pos = BITS * k, wi = pos >> 5, sh = pos & 31;
            w[wi] |= (uint32_t)idx[k] << sh;
            if (sh + BITS > 32) w[wi + 1] |= (uint32_t)idx[k] >> (32 - sh);
        }
    }
}
// The same bytes from the group order of the matrix-core rows: each group's 8 fields packed
// (8 BITS bits), the groups transposed across the row's lanes, then joined into the stream.
template <int BITS>
__device__ __forceinline__ void pack_stream_groups(const int (&idx)[32], uint32_t (&w)[BITS]) {
    uint32_t g[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        uint32_t t[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) t[k] = (uint32_t)idx[8 * s + k];
#pragma unroll
        for (int span = 1, sh = BITS; span < 8; span *= 2, sh *= 2)
#pragma unroll
            for (int k = 0; k < 8; k += 2 * span) t[k] = lshl_or(t[k + span], sh, t[k]);
        g[s] = t[0];
    }
    transpose_groups(g);
    if constexpr (BITS == 4) {
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = g[j];
    } else if constexpr (BITS == 2) {
        w[0] = lshl_or(g[1], 16, g[0]);
        w[1] = lshl_or(g[3], 16, g[2]);
    } else if constexpr (BITS == 1) {
        w[0] = lshl_or(g[3], 24, lshl_or(g[2], 16, lshl_or(g[1], 8, g[0])));
    } else {
        w[0] = lshl_or(g[1], 24, g[0]);
        w[1] = lshl_or(g[2], 16, g[1] >> 8);
        w[2] = lshl_or(g[3], 8, g[2] >> 16);
    }
}
// 32 sign bits (bit k of the lane's element k, group order) -> the bits of dims 32 G .. 32 G + 31
__device__ __forceinline__ uint32_t sign_bits_groups(uint32_t sb) {
    uint32_t g[4] = {sb & 0xffu, (sb >> 8) & 0xffu, (sb >> 16) & 0xffu, sb >> 24};
    transpose_groups(g);
    return lshl_or(g[3], 24, lshl_or(g[2], 16, lshl_or(g[1], 8, g[0])));
}

// ---- values tile layout ----
// Chunk 16g + n of a 16-row sub-tile (4 * BITS bytes) holds, at field 4j + r (BITS bits each,
// little-endian), dim 8n + j of row 4g + r: the four rows' fields of one dim are adjacent, so a
// decode lane turns one field group into one PV operand with one table lookup.  A row's lane q
// (dims 32q..32q+31) owns fields of chunks n = 4q + i, i = 0..3.  Its slice i holds fields 8i + j
// at bits 4 BITS j (BITS words): room for the other three rows' fields in between.
template <int BITS>
struct ValueSlices {
    uint32_t w[4][BITS];
};
template <int BITS>
__device__ __forceinline__ ValueSlices<BITS> value_slices(const int (&idx)[32]) {
    ValueSlices<BITS> s;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int k = 0; k < BITS; ++k) s.w[i][k] = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int pos = 4 * BITS * j;  // a field never straddles two words here
            s.w[i][pos >> 5] |= (uint32_t)idx[8 * i + j] << (pos & 31);
        }
    }
    return s;
}
// The fields of one slice (every 4th field position), as words.
template <int BITS>
__device__ __forceinline__ uint32_t value_field_mask(int k) {
    if (BITS == 2) return 0x03030303u;
    if (BITS == 4) return 0x000F000Fu;
    return k == 0 ? 0x07007007u : (k == 1 ? 0x70070070u : 0x00700700u);  // fields at 12 j
}
// a << s over BITS words (s = BITS r, r = 0..3; for 2 and 4 bits no field crosses a word)
template <int BITS>
__device__ __forceinline__ void shl_words(const uint32_t (&a)[BITS], uint32_t s, uint32_t (&o)[BITS]) {
#pragma unroll
    for (int k = 0; k < BITS; ++k) {
        if (BITS == 3 && k > 0)
            // (a[k]:a[k-1]) >> (32 - s), one funnel shift (a 64-bit shift of the pair kept the
            // slices in scratch memory)
            o[k] = s == 0 ? a[k] : __builtin_amdgcn_alignbit(a[k], a[k - 1], 32 - s);
        else
            o[k] = a[k] << s;
    }
}

// Writes this lane's fields into the values layout.  Rows 4a..4a+3 of a workgroup that land on
// slots 4k..4k+3 fill whole chunks: their slices are exchanged through this group's part of
// xchg and each lane stores one chunk.  Any other row sets its own fields with atomic and / or on
// the chunk words (other rows of the chunk, written by other launches or workgroups, are
// untouched).  Lane layouts: 4 consecutive lanes per row (a group of 4 rows is lanes
// 16a'..16a'+15 of one wave, slice i of lane q is chunk 4q + i), or GROUPS, the matrix-core
// rows (row l & 15, lane group q = l >> 4: a group of 4 rows is lanes 4a' + {0..3} + 16 {0..3},
// slice i of lane q is chunk 4i + q).
template <int BITS, bool GROUPS>
__device__ __forceinline__ void store_values(const ValueSlices<BITS>& vs, bool write, int64_t slot, uint8_t* tile,
                                             int64_t r_in_blk, int q, uint32_t* xchg) {
    constexpr int VS = BITS == 3 ? 4 : BITS;  // words per slice in the exchange (b64 / b128 access)
    const int lane = threadIdx.x & 63;
    const int rr = GROUPS ? (lane & 3) : ((threadIdx.x >> 2) & 3);  // row of the lane within its group of 4 rows
    const int64_t s0 = __shfl(slot, GROUPS ? (lane & 12) : (lane & ~12));
    const bool ok = write && (s0 & 3) == 0 && slot == s0 + rr;
    const uint64_t bal = __builtin_amdgcn_ballot_w64(ok);
    const bool full = GROUPS ? ((bal >> (lane & 12)) & 0x000F000F000F000Full) == 0x000F000F000F000Full
                             : ((bal >> (lane & 48)) & 0xffffull) == 0xffffull;
    uint8_t* sub = tile + (r_in_blk & ~(int64_t)15) * (16 * BITS);
    const int g = (int)((r_in_blk & 15) >> 2);
    if (full) {
        const int grp = GROUPS ? ((threadIdx.x >> 6) * 4 + ((lane & 15) >> 2)) : (threadIdx.x >> 4);
        uint32_t* gx = xchg + grp * (64 * VS);  // this group: [chunk][row][VS]
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t* d = gx + ((GROUPS ? 4 * i + q : q * 4 + i) * 4 + rr) * VS;
            if (VS == 2) {
                *reinterpret_cast<tq_u32x2*>(d) = tq_u32x2{vs.w[i][0], vs.w[i][1 % BITS]};
            } else {
                *reinterpret_cast<tq_u32x4*>(d) =
                    tq_u32x4{vs.w[i][0], vs.w[i][1 % BITS], vs.w[i][2 % BITS], BITS == 4 ? vs.w[i][3 % BITS] : 0u};
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        // chunk n = 4q + rr: slice rr of the group's rows 0..3
        uint32_t out[BITS];
#pragma unroll
        for (int k = 0; k < BITS; ++k) out[k] = 0;
        const uint32_t* src = gx + ((q * 4 + rr) * 4) * VS;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            uint32_t a[BITS], sh[BITS];
            if (VS == 2) {
                const tq_u32x2 v = *reinterpret_cast<const tq_u32x2*>(src + r * VS);
                a[0] = v[0];
                a[1 % BITS] = v[1];
            } else {
                const tq_u32x4 v = *reinterpret_cast<const tq_u32x4*>(src + r * VS);
#pragma unroll
                for (int k = 0; k < BITS; ++k) a[k] = v[k];
            }
            shl_words<BITS>(a, (uint32_t)(BITS * r), sh);
#pragma unroll
            for (int k = 0; k < BITS; ++k) out[k] |= sh[k];
        }
        uint32_t* ch = reinterpret_cast<uint32_t*>(sub + (16 * g + 4 * q + rr) * (4 * BITS));
#pragma unroll
        for (int k = 0; k < BITS; ++k) ch[k] = out[k];
    } else if (write) {
        const uint32_t sh = (uint32_t)(BITS * (r_in_blk & 3));
        uint32_t m0[BITS];
#pragma unroll
        for (int k = 0; k < BITS; ++k) m0[k] = value_field_mask<BITS>(k);
        uint32_t m[BITS];
        shl_words<BITS>(m0, sh, m);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t b[BITS];
            shl_words<BITS>(vs.w[i], sh, b);
            uint32_t* ch = reinterpret_cast<uint32_t*>(sub + (16 * g + (GROUPS ? 4 * i + q : 4 * q + i)) * (4 * BITS));
#pragma unroll
            for (int k = 0; k < BITS; ++k) {
                __hip_atomic_fetch_and(ch + k, ~m[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_fetch_or(ch + k, b[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
}

// The body of the compression kernels: workgroup wg of nwg takes 64-row groups wg, wg + nwg, ...
template <int BITS, bool QJL, int MODE, int DT>
__device__ __forceinline__ void compress_rows(const CompressParams& p, int wg, int nwg) {
    constexpr int NC = 1 << BITS;
    constexpr int NB = NC - 1;
    __shared__ float s_cent[NC];
    __shared__ uint2 s_cells[kCells];
    __shared__ int s_bad;
    // values layout: slices exchanged within each group of 4 rows (16 groups x 64 slices)
    __shared__ __align__(16) uint32_t s_xchg[MODE == MODE_PAGED ? 1024 * (BITS == 3 ? 4 : BITS) : 1];
    if (threadIdx.x < NC) s_cent[threadIdx.x] = p.centroids[threadIdx.x];
    if (threadIdx.x == 0) s_bad = 0;
    // Boundaries are uniform: the loads below become scalar loads kept in SGPRs.
    float bd[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) bd[i] = p.boundaries[i];
    __syncthreads();
    if (MODE == MODE_PAGED) build_cells_rn<NB>(bd, p.boundaries, s_cells, &s_bad);
    else build_cells<NB>(bd, p.boundaries, s_cells, &s_bad);
    __syncthreads();
    const bool cells = s_bad == 0;
    // 1e-8 in the units of the unscaled rotation (paged mode)
    const float den_eps = (MODE == MODE_PAGED && p.rotate) ? 1e-8f / p.wht_scale : 1e-8f;

    // 16-bit paged rows run on the matrix cores (row l & 15 of the wave, lane group q = l >> 4);
    // the others keep 4 consecutive lanes per row.  Either way the row's words leave lane q for
    // dims 32q..32q+31.
    constexpr bool GR = MODE == MODE_PAGED && DT != TQ_F32;
    const int lane = threadIdx.x & 63;
    const int q = GR ? (lane >> 4) : (threadIdx.x & 3);
    const int row_in_wg = GR ? ((threadIdx.x >> 6) * 16 + (lane & 15)) : (threadIdx.x >> 2);  // 0..63
    HadamardFrags<DT> hf;
    if constexpr (GR) hf = hadamard_frags<DT>(lane);

    for (int64_t row0 = (int64_t)wg * kRowsPerWG; row0 < p.n_rows; row0 += (int64_t)nwg * kRowsPerWG) {
        const int64_t row = row0 + row_in_wg;
        bool row_ok = row < p.n_rows;
        // Paged rows are head-major so that a workgroup's rows are consecutive tokens; each
        // head's rows are padded to a multiple of 4, so rows 4a..4a+3 (one 16-lane group of a
        // wave) are tokens 4k..4k+3 of one head.
        int64_t tok, head;
        if (MODE == MODE_PAGED) {
            if (p.idx32) {
                const uint32_t r = row_ok ? (uint32_t)row : 0u, nt = (uint32_t)p.tok_rows;
                const uint32_t h = tq_udiv_apply(r, p.tok_div);
                head = h;
                tok = r - h * nt;
            } else {
                head = row_ok ? row / p.tok_rows : 0;
                tok = row_ok ? row - head * p.tok_rows : 0;
            }
            row_ok = row_ok && tok < p.num_tokens;
            tok = row_ok ? tok : 0;
            head = row_ok ? head : 0;
        } else {
            head = 0;
            tok = row_ok ? row : 0;
        }

        // Rows that are not written (padding, past the end) read token 0 of head 0, a row of the
        // same launch, and their results are dropped: no separate zero fill.
        int64_t off;
        const uint32_t lane_off = GR ? 8u * q : 32u * q;
        if (p.idx32) off = (uint32_t)tok * (uint32_t)p.x_stride_token + (uint32_t)head * (uint32_t)p.x_stride_head + lane_off;
        else off = tok * p.x_stride_token + head * p.x_stride_head + lane_off;
        RawRow<DT> raw;
        if constexpr (GR) load_raw_groups<DT>(p.x, off, raw);
        else load_raw<DT>(p.x, off, raw);
        // the slot goes out with the row (token 0's for rows that are not written, whose result
        // is dropped): its round trip overlaps the row's instead of following the quantisation
        uint32_t slo = 0, shi = 0;
        if (MODE == MODE_PAGED) {
            const uint32_t* sp = reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(p.slot_mapping) +
                                                                   tok * (p.slot_i64 ? 8 : 4));
            slo = sp[0];
            shi = sp[p.slot_i64 ? 1 : 0];
        }
        float v[32];
        float norm, den, rcp;
        bool fast;
        if (MODE == MODE_PAGED) {
            // v = z, y = scale z (the rotation's scale h, or 1 without rotation)
            if (p.rotate) {
                if constexpr (GR) rotate_mfma<DT>(raw, hf, v);
                else if constexpr (DT == TQ_F32) rotate_unscaled_f32(raw, q, v);
            } else {
                raw_to_float<DT>(raw, v);
            }
            const float scale = p.rotate ? p.wht_scale : 1.f;
            const float nz = __builtin_sqrtf(row_sumsq_of<GR>(v));
            fast = cells && !__builtin_amdgcn_ballot_w64(!(nz < __builtin_huge_valf()));
            if (fast) {
                // x_n = y / (|y| + 1e-8) = z / (|z| + 1e-8 / scale): decisions on z and this
                // denominator; 128 / den only places the lookup cell, an approximate reciprocal
                // does (it moves x by far less than the cells' eps)
                norm = nz * scale;
                den = nz + den_eps;
                rcp = __builtin_amdgcn_rcpf(den);
            } else {
#pragma unroll
                for (int k = 0; k < 32; ++k) v[k] *= scale;
                norm = __builtin_sqrtf(row_sumsq_of<GR>(v));
                den = norm + 1e-8f;
                rcp = 1.0f / den;
            }
        } else {
            raw_to_float<DT>(raw, v);
            if (p.rotate) wht_row(v, q, p.wht_scale);
            norm = __builtin_sqrtf(row_sumsq(v));
            den = norm + 1e-8f;
            rcp = 1.0f / den;
            // |x| <= 1 unless the norm is not finite (then x may be NaN: searchsorted puts it last)
            fast = cells && !__builtin_amdgcn_ballot_w64(!(norm < __builtin_huge_valf()));
        }

        int idx[32];
        float rn = 0.f;
        uint32_t sbits = 0;
        if (MODE == MODE_PAGED && fast) {
            // decisions on z itself (x_n = z / den is never formed); with QJL the residual
            // r = (x_n - c) norm = (z - c den) (norm / den), its sign that of one fma
            const float rscale = kCellsRnScale * rcp;
#pragma unroll
            for (int k = 0; k < 32; ++k) idx[k] = quant_cell_y(v[k], den, rscale, s_cells);
            if (QJL) {
                float r[32];
#pragma unroll
                for (int k = 0; k < 32; ++k) {
                    r[k] = __builtin_fmaf(-s_cent[idx[k]], den, v[k]);
                    sbits |= (r[k] >= 0.f ? 1u : 0u) << k;
                }
                rn = __builtin_sqrtf(row_sumsq_of<GR>(r)) * (norm / den);
                if (norm == 0.f) sbits = 0xffffffffu;  // r = (0 - c) 0 = +-0: sign(0) counts as +1
            }
        } else {
#pragma unroll
            for (int k = 0; k < 32; ++k) v[k] = tq_div_rn(v[k], den, rcp);  // x / (norm + 1e-8)
            if (fast) {
#pragma unroll
                for (int k = 0; k < 32; ++k) idx[k] = quant_cell(v[k], s_cells);
            } else {
#pragma unroll
                for (int k = 0; k < 32; ++k) idx[k] = quant_linear<NB>(v[k], bd);
            }
            if (QJL) {
                float r[32];
#pragma unroll
                for (int k = 0; k < 32; ++k) {
                    r[k] = (v[k] - s_cent[idx[k]]) * norm;
                    sbits |= (r[k] >= 0.f ? 1u : 0u) << k;
                }
                rn = __builtin_sqrtf(row_sumsq_of<GR>(r));
            }
        }

        if (MODE == MODE_UNPACKED) {
            if (row_ok) {
                int64_t* ip = p.indices + row * TQ_HEAD_DIM + 32 * q;
                float* kp = p.k_mse + row * TQ_HEAD_DIM + 32 * q;
#pragma unroll
                for (int k = 0; k < 32; ++k) {
                    ip[k] = idx[k];
                    kp[k] = s_cent[idx[k]] * norm;
                }
                if (QJL) {
                    float* sp = p.signs + row * TQ_HEAD_DIM + 32 * q;
#pragma unroll
                    for (int k = 0; k < 32; ++k) sp[k] = ((sbits >> k) & 1u) ? 1.f : -1.f;
                }
                if (q == 0) {
                    p.norms[row] = norm;
                    if (QJL) p.rnorm[row] = rn;
                }
            }
        } else {
            const int64_t slot =
                !row_ok ? -1 : (p.slot_i64 ? (int64_t)(((uint64_t)shi << 32) | slo) : (int64_t)(int32_t)slo);
            const bool write = row_ok && slot >= 0 && slot < p.num_blocks * p.block_size;
            int64_t blk, r_in_blk;
            if (p.idx32) {
                const uint32_t sl = write ? (uint32_t)slot : 0u, bs = (uint32_t)p.block_size;
                const uint32_t b = tq_udiv_apply(sl, p.blk_div);
                blk = b;
                r_in_blk = sl - b * bs;
            } else {
                blk = write ? slot / p.block_size : 0;
                r_in_blk = write ? slot - blk * p.block_size : 0;
            }
            uint8_t* tile = p.cache + blk * p.stride_block + head * p.stride_head;
            if (p.tile_layout == TQ_TILE_VALUES) {
                if (BITS >= 2)
                    store_values<BITS < 2 ? 2 : BITS, GR>(value_slices<BITS < 2 ? 2 : BITS>(idx), write, slot, tile,
                                                          r_in_blk, q, s_xchg);
                if (write && q == 0)
                    *reinterpret_cast<uint16_t*>(tile + p.off_norm + r_in_blk * p.rs_norm) = (uint16_t)tq_f32_to_f16_bits(norm);
                continue;
            }
            // this lane's 32 indices: 4 * BITS bytes of the row's little-endian bit stream
            uint32_t w[BITS];
            if constexpr (GR) {
                pack_stream_groups<BITS>(idx, w);
                if (QJL) sbits = sign_bits_groups(sbits);
            } else {
                pack_stream<BITS>(idx, w);
            }
            if (write) {
                if (p.tile_layout == TQ_TILE_KEYS) {
                    // chunk (4n + q) of the row's 16-row sub-tile: index bytes, then sign bytes
                    constexpr int P = 16 * BITS + (QJL ? 16 : 0), C = 4 * BITS + (QJL ? 4 : 0);
                    uint32_t* ch = reinterpret_cast<uint32_t*>(tile + (r_in_blk & ~(int64_t)15) * P +
                                                               (4 * (r_in_blk & 15) + q) * C);
#pragma unroll
                    for (int j = 0; j < BITS; ++j) ch[j] = w[j];
                    if (QJL) ch[BITS] = sbits;
                } else {
                    // row-major regions (this library's rows layout, or caller-described regions
                    // such as the reference's array-of-slots cache)
                    uint8_t* ip = tile + r_in_blk * p.rs_idx + 4 * BITS * q;
                    uint8_t* sp = tile + p.off_signs + r_in_blk * p.rs_sig + 4 * q;
                    if (!p.narrow) {
#pragma unroll
                        for (int j = 0; j < BITS; ++j) reinterpret_cast<uint32_t*>(ip)[j] = w[j];
                        if (QJL) *reinterpret_cast<uint32_t*>(sp) = sbits;
                    } else {
#pragma unroll
                        for (int j = 0; j < BITS; ++j) {
                            reinterpret_cast<uint16_t*>(ip)[2 * j] = (uint16_t)w[j];
                            reinterpret_cast<uint16_t*>(ip)[2 * j + 1] = (uint16_t)(w[j] >> 16);
                        }
                        if (QJL) {
                            reinterpret_cast<uint16_t*>(sp)[0] = (uint16_t)sbits;
                            reinterpret_cast<uint16_t*>(sp)[1] = (uint16_t)(sbits >> 16);
                        }
                    }
                }
                if (q == 0) {
                    *reinterpret_cast<uint16_t*>(tile + p.off_norm + r_in_blk * p.rs_norm) =
                        (uint16_t)tq_f32_to_f16_bits(norm);
                    if (QJL)
                        *reinterpret_cast<uint16_t*>(tile + p.off_rnorm + r_in_blk * p.rs_norm) =
                            (uint16_t)tq_f32_to_f16_bits(rn);
                }
            }
        }
    }
}

// Resident waves per SIMD the kernel is compiled for: the matrix-core rows (16-bit paged input)
// without QJL fit 4 (128 registers: the Hadamard fragments, the accumulators and the row), the
// others keep the compiler's own choice.
template <int MODE, int DT, bool QJL>
constexpr int compress_min_waves() {
    return (MODE == MODE_PAGED && DT != TQ_F32 && !QJL) ? 4 : 1;
}

template <int BITS, bool QJL, int MODE, int DT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(compress_min_waves<MODE, DT, QJL>(), 8)))
void compress_kernel(CompressParams p) {
    compress_rows<BITS, QJL, MODE, DT>(p, blockIdx.x, gridDim.x);
}

// K and V of one layer in one launch (same bits; V without QJL): workgroups [0, gk) take K, the
// rest V.  One launch instead of two halves the fixed cost of a K + V cache update.
template <int BITS, bool QJL_K, int DT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(compress_min_waves<MODE_PAGED, DT, QJL_K>(), 8)))
void compress_kv_kernel(CompressParams pk, CompressParams pv, int gk) {
    if ((int)blockIdx.x < gk) compress_rows<BITS, QJL_K, MODE_PAGED, DT>(pk, blockIdx.x, gk);
    else compress_rows<BITS, false, MODE_PAGED, DT>(pv, blockIdx.x - gk, gridDim.x - gk);
}

template <int MODE>
int launch_compress(const CompressParams& p, int bits, int qjl, hipStream_t stream) {
    if (p.n_rows <= 0) return TQ_OK;
    // Workgroups loop over 64-row groups; at most as many workgroups as are resident at once.
    const int64_t groups = (p.n_rows + kRowsPerWG - 1) / kRowsPerWG;
#define TQ_LAUNCH_DT(B, Q, DT)                                                                       \
    do {                                                                                             \
        static const int res = resident_grid(compress_kernel<B, Q, MODE, DT>);                       \
        const int grid = (int)(groups < res ? groups : res);                                         \
        hipLaunchKernelGGL((compress_kernel<B, Q, MODE, DT>), dim3(grid), dim3(256), 0, stream, p);  \
    } while (0)
#define TQ_LAUNCH(B, Q)                                   \
    do {                                                  \
        if (p.x_dtype == TQ_BF16) TQ_LAUNCH_DT(B, Q, TQ_BF16); \
        else if (p.x_dtype == TQ_F16) TQ_LAUNCH_DT(B, Q, TQ_F16); \
        else TQ_LAUNCH_DT(B, Q, TQ_F32);                  \
    } while (0)
    switch (bits * 2 + (qjl ? 1 : 0)) {
        case 2: TQ_LAUNCH(1, false); break;
        case 3: TQ_LAUNCH(1, true); break;
        case 4: TQ_LAUNCH(2, false); break;
        case 5: TQ_LAUNCH(2, true); break;
        case 6: TQ_LAUNCH(3, false); break;
        case 7: TQ_LAUNCH(3, true); break;
        case 8: TQ_LAUNCH(4, false); break;
        case 9: TQ_LAUNCH(4, true); break;
        default: return TQ_ERR_BITS;
    }
#undef TQ_LAUNCH
#undef TQ_LAUNCH_DT
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TQ_OK : (int)e;
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

int check_x(const void* x, int x_dtype) {
    if (x_dtype != TQ_F32 && x_dtype != TQ_F16 && x_dtype != TQ_BF16) return TQ_ERR_DTYPE;
    if (!aligned(x, x_dtype == TQ_F32 ? 32 : 16)) return TQ_ERR_ALIGNMENT;
    return TQ_OK;
}

}  // namespace

extern "C" int tq_polarquant_compress(const void* x, int x_dtype, int64_t x_row_stride, int64_t n_rows,
                                      int head_dim, int rotate, float wht_scale,
                                      const float* centroids, const float* boundaries, int bits, int use_qjl,
                                      int64_t* indices, float* norms, float* k_mse, float* signs, float* rnorm,
                                      tq_stream_t stream) {
    if (head_dim != TQ_HEAD_DIM) return TQ_ERR_HEAD_DIM;
    if (bits < 1 || bits > 4) return TQ_ERR_BITS;
    if (n_rows < 0 || x_row_stride < TQ_HEAD_DIM) return TQ_ERR_INVALID_ARGUMENT;
    if (n_rows == 0) return TQ_OK;
    if (!x || !centroids || !boundaries || !indices || !norms || !k_mse) return TQ_ERR_INVALID_ARGUMENT;
    if (use_qjl && (!signs || !rnorm)) return TQ_ERR_INVALID_ARGUMENT;
    int rc = check_x(x, x_dtype);
    if (rc) return rc;
    if (x_row_stride % 8) return TQ_ERR_ALIGNMENT;
    CompressParams p = {};
    p.x = x;
    p.x_dtype = x_dtype;
    p.x_stride_token = x_row_stride;
    p.x_stride_head = 0;
    p.num_tokens = n_rows;
    p.tok_rows = n_rows;
    p.num_heads = 1;
    p.n_rows = n_rows;
    p.rotate = rotate ? 1 : 0;
    p.wht_scale = wht_scale;
    p.centroids = centroids;
    p.boundaries = boundaries;
    p.indices = indices;
    p.norms = norms;
    p.k_mse = k_mse;
    p.signs = signs;
    p.rnorm = rnorm;
    p.idx32 = (n_rows * x_row_stride < (1ll << 31)) ? 1 : 0;
    return launch_compress<MODE_UNPACKED>(p, bits, use_qjl, (hipStream_t)stream);
}

extern "C" int64_t tq_tile_bytes(int block_size, int bits, int use_qjl) {
    if (block_size <= 0 || block_size % 16 || bits < 2 || bits > 4) return -1;
    return tq_make_tile_geom(block_size, bits, use_qjl).bytes;
}

extern "C" int tq_tile_offsets(int block_size, int bits, int use_qjl, int64_t* off_idx, int64_t* off_signs,
                               int64_t* off_norm, int64_t* off_rnorm) {
    if (block_size <= 0 || block_size % 16) return TQ_ERR_BLOCK_SIZE;
    if (bits < 2 || bits > 4) return TQ_ERR_BITS;
    tq_tile_geom g = tq_make_tile_geom(block_size, bits, use_qjl);
    if (off_idx) *off_idx = 0;
    if (off_signs) *off_signs = use_qjl ? g.off_signs : -1;
    if (off_norm) *off_norm = g.off_norm;
    if (off_rnorm) *off_rnorm = use_qjl ? g.off_rnorm : -1;
    return TQ_OK;
}

namespace {

// Validates one paged compression and fills its parameters (TQ_OK, or the error to return;
// *empty when there is nothing to write).
int paged_params(const void* x, int x_dtype, int64_t x_stride_token, int64_t x_stride_head, int64_t num_tokens,
                 int num_heads, int head_dim, const void* slot_mapping, int slot_dtype, void* cache,
                 int64_t cache_stride_block, int64_t cache_stride_head, int64_t num_blocks, int block_size, int bits,
                 int use_qjl, int tile_layout, int rotate, float wht_scale, const float* centroids,
                 const float* boundaries, CompressParams* out, bool* empty, const tq_kv_view* regions = nullptr) {
    *empty = false;
    if (head_dim != TQ_HEAD_DIM) return TQ_ERR_HEAD_DIM;
    if (bits < 2 || bits > 4) return TQ_ERR_BITS;
    if (block_size <= 0 || block_size % 16) return TQ_ERR_BLOCK_SIZE;
    if (num_tokens < 0 || num_heads <= 0 || num_blocks < 0) return TQ_ERR_INVALID_ARGUMENT;
    if (slot_dtype != TQ_I32 && slot_dtype != TQ_I64) return TQ_ERR_DTYPE;
    if (tile_layout != TQ_TILE_ROWS && tile_layout != TQ_TILE_KEYS && tile_layout != TQ_TILE_VALUES)
        return TQ_ERR_INVALID_ARGUMENT;
    if (tile_layout == TQ_TILE_VALUES && use_qjl) return TQ_ERR_INVALID_ARGUMENT;
    if (num_tokens == 0 || num_blocks == 0) {
        *empty = true;
        return TQ_OK;
    }
    if (!x || !slot_mapping || !cache || !centroids || !boundaries) return TQ_ERR_INVALID_ARGUMENT;
    int rc = check_x(x, x_dtype);
    if (rc) return rc;
    if (x_stride_token % 8 || x_stride_head % 8) return TQ_ERR_ALIGNMENT;
    const tq_tile_geom g = tq_make_tile_geom(block_size, bits, use_qjl);
    if (!regions) {
        if (!aligned(cache, 16) || cache_stride_block % 16 || cache_stride_head % 16) return TQ_ERR_ALIGNMENT;
        if (cache_stride_head < g.bytes && num_heads > 1) return TQ_ERR_INVALID_ARGUMENT;
    }
    CompressParams p = {};
    p.x = x;
    p.x_dtype = x_dtype;
    p.x_stride_token = x_stride_token;
    p.x_stride_head = x_stride_head;
    p.num_tokens = num_tokens;
    p.num_heads = num_heads;
    p.tok_rows = (num_tokens + 3) & ~(int64_t)3;
    p.n_rows = p.tok_rows * num_heads;
    p.rotate = rotate ? 1 : 0;
    p.wht_scale = wht_scale;
    p.centroids = centroids;
    p.boundaries = boundaries;
    p.slot_mapping = slot_mapping;
    p.slot_i64 = slot_dtype == TQ_I64;
    p.cache = static_cast<uint8_t*>(cache);
    p.stride_block = cache_stride_block;
    p.stride_head = cache_stride_head;
    p.num_blocks = num_blocks;
    p.block_size = block_size;
    p.tile_layout = tile_layout;
    p.off_signs = g.off_signs;
    p.off_norm = g.off_norm;
    p.off_rnorm = g.off_rnorm;
    p.rs_idx = 16 * bits;
    p.rs_sig = 16;
    p.rs_norm = 2;
    p.narrow = 0;
    if (regions) {
        // caller-described row-major regions sharing one (block, head) base: offsets from the
        // index region, per-region row strides
        const tq_region& ri = regions->idx;
        const uint8_t* b0 = static_cast<const uint8_t*>(ri.ptr);
        auto off = [&](const tq_region& r) { return static_cast<int64_t>(static_cast<const uint8_t*>(r.ptr) - b0); };
        p.off_norm = off(regions->norm);
        p.rs_idx = ri.stride_row;
        p.rs_norm = regions->norm.stride_row;
        if (use_qjl) {
            p.off_signs = off(regions->signs);
            p.off_rnorm = off(regions->rnorm);
            p.rs_sig = regions->signs.stride_row;
        } else {
            p.off_signs = p.off_rnorm = 0;
        }
        const bool four = aligned(ri.ptr, 4) && ri.stride_block % 4 == 0 && ri.stride_head % 4 == 0 &&
                          ri.stride_row % 4 == 0 && (!use_qjl || (p.off_signs % 4 == 0 && p.rs_sig % 4 == 0));
        p.narrow = four ? 0 : 1;
    }
    // rows, slots and x element offsets all below 2^31
    p.idx32 = (p.n_rows < (1ll << 31) && num_blocks * (int64_t)block_size < (1ll << 31) &&
               num_tokens * x_stride_token + (int64_t)num_heads * x_stride_head < (1ll << 31))
                  ? 1
                  : 0;
    if (p.idx32) {
        p.tok_div = tq_make_udiv((uint32_t)p.tok_rows);
        p.blk_div = tq_make_udiv((uint32_t)block_size);
    }
    *out = p;
    return TQ_OK;
}

int paged_target_params(const tq_paged_target* t, int x_dtype, int64_t num_tokens, int num_heads, int head_dim,
                        const void* slot_mapping, int slot_dtype, int64_t num_blocks, int block_size, int rotate,
                        float wht_scale, CompressParams* out, bool* empty) {
    if (!t) return TQ_ERR_INVALID_ARGUMENT;
    return paged_params(t->x, x_dtype, t->x_stride_token, t->x_stride_head, num_tokens, num_heads, head_dim,
                        slot_mapping, slot_dtype, t->cache, t->cache_stride_block, t->cache_stride_head, num_blocks,
                        block_size, t->bits, t->use_qjl, t->tile_layout, rotate, wht_scale, t->centroids,
                        t->boundaries, out, empty);
}

}  // namespace

extern "C" int tq_compress_paged(const void* x, int x_dtype, int64_t x_stride_token, int64_t x_stride_head,
                                 int64_t num_tokens, int num_heads, int head_dim,
                                 const void* slot_mapping, int slot_dtype,
                                 void* cache, int64_t cache_stride_block, int64_t cache_stride_head,
                                 int64_t num_blocks, int block_size,
                                 int bits, int use_qjl, int tile_layout, int rotate, float wht_scale,
                                 const float* centroids, const float* boundaries,
                                 tq_stream_t stream) {
    CompressParams p;
    bool empty;
    const int rc = paged_params(x, x_dtype, x_stride_token, x_stride_head, num_tokens, num_heads, head_dim, slot_mapping,
                                slot_dtype, cache, cache_stride_block, cache_stride_head, num_blocks, block_size, bits,
                                use_qjl, tile_layout, rotate, wht_scale, centroids, boundaries, &p, &empty);
    if (rc || empty) return rc;
    return launch_compress<MODE_PAGED>(p, bits, use_qjl, (hipStream_t)stream);
}

extern "C" int tq_compress_regions(const void* x, int x_dtype, int64_t x_stride_token, int64_t x_stride_head,
                                   int64_t num_tokens, int num_heads, int head_dim, const void* slot_mapping,
                                   int slot_dtype, const tq_kv_view* dst, const float* boundaries,
                                   int64_t num_blocks, int block_size, int rotate, float wht_scale,
                                   tq_stream_t stream) {
    if (!dst || dst->layout != TQ_TILE_ROWS || dst->signs_permuted) return TQ_ERR_INVALID_ARGUMENT;
    const int qjl = dst->qjl ? 1 : 0;
    const tq_region& ri = dst->idx;
    auto same_base = [&](const tq_region& r) {
        return r.stride_block == ri.stride_block && r.stride_head == ri.stride_head;
    };
    auto two = [](const tq_region& r) {
        return aligned(r.ptr, 2) && r.stride_block % 2 == 0 && r.stride_head % 2 == 0 && r.stride_row % 2 == 0;
    };
    if (num_tokens > 0 && num_blocks > 0) {
        if (!ri.ptr || !dst->norm.ptr || (qjl && (!dst->signs.ptr || !dst->rnorm.ptr))) return TQ_ERR_INVALID_ARGUMENT;
        if (!same_base(dst->norm) || (qjl && (!same_base(dst->signs) || !same_base(dst->rnorm))))
            return TQ_ERR_INVALID_ARGUMENT;
        if (qjl && dst->rnorm.stride_row != dst->norm.stride_row) return TQ_ERR_INVALID_ARGUMENT;
        if (!two(ri) || !two(dst->norm) || (qjl && (!two(dst->signs) || !two(dst->rnorm)))) return TQ_ERR_ALIGNMENT;
    }
    CompressParams p;
    bool empty;
    const int rc = paged_params(x, x_dtype, x_stride_token, x_stride_head, num_tokens, num_heads, head_dim, slot_mapping,
                                slot_dtype, const_cast<void*>(ri.ptr), ri.stride_block, ri.stride_head, num_blocks,
                                block_size, dst->bits, qjl, TQ_TILE_ROWS, rotate, wht_scale, dst->centroids, boundaries,
                                &p, &empty, dst);
    if (rc || empty) return rc;
    return launch_compress<MODE_PAGED>(p, dst->bits, qjl, (hipStream_t)stream);
}

extern "C" int tq_compress_paged_kv(const tq_paged_target* k, const tq_paged_target* v, int x_dtype,
                                    int64_t num_tokens, int num_heads, int head_dim,
                                    const void* slot_mapping, int slot_dtype, int64_t num_blocks, int block_size,
                                    int rotate, float wht_scale, tq_stream_t stream) {
    CompressParams pk, pv;
    bool ek, ev;
    int rc = paged_target_params(k, x_dtype, num_tokens, num_heads, head_dim, slot_mapping, slot_dtype, num_blocks,
                                 block_size, rotate, wht_scale, &pk, &ek);
    if (rc) return rc;
    rc = paged_target_params(v, x_dtype, num_tokens, num_heads, head_dim, slot_mapping, slot_dtype, num_blocks,
                             block_size, rotate, wht_scale, &pv, &ev);
    if (rc || ek) return rc;  // both are empty together (same tokens, same blocks)
    const hipStream_t st = (hipStream_t)stream;
    if (k->bits != v->bits || v->use_qjl) {
        // not one kernel: two launches
        rc = launch_compress<MODE_PAGED>(pk, k->bits, k->use_qjl, st);
        return rc ? rc : launch_compress<MODE_PAGED>(pv, v->bits, v->use_qjl, st);
    }
    // K workgroups first, then as many V workgroups: half the resident workgroups each
    const int64_t groups = (pk.n_rows + kRowsPerWG - 1) / kRowsPerWG;
#define TQ_KV_DT(B, Q, DT)                                                                          \
    do {                                                                                            \
        static const int res = resident_grid(compress_kv_kernel<B, Q, DT>) / 2;                     \
        const int gk = (int)(groups < res ? groups : (res > 0 ? res : 1));                          \
        hipLaunchKernelGGL((compress_kv_kernel<B, Q, DT>), dim3(2 * gk), dim3(256), 0, st, pk, pv, gk); \
    } while (0)
#define TQ_KV(B, Q)                                             \
    do {                                                        \
        if (x_dtype == TQ_BF16) TQ_KV_DT(B, Q, TQ_BF16);        \
        else if (x_dtype == TQ_F16) TQ_KV_DT(B, Q, TQ_F16);     \
        else TQ_KV_DT(B, Q, TQ_F32);                            \
    } while (0)
    switch (k->bits * 2 + (k->use_qjl ? 1 : 0)) {
        case 4: TQ_KV(2, false); break;
        case 5: TQ_KV(2, true); break;
        case 6: TQ_KV(3, false); break;
        case 7: TQ_KV(3, true); break;
        case 8: TQ_KV(4, false); break;
        case 9: TQ_KV(4, true); break;
        default: return TQ_ERR_BITS;
    }
#undef TQ_KV
#undef TQ_KV_DT
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? TQ_OK : (int)e;
}
