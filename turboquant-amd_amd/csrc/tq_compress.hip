// PolarQuant compression kernels for gfx950.
//
// One 128-dim row per 16 lanes (8 dims each), so a wave64 works on 4 rows and a 256-thread
// workgroup on 16 rows.  The Walsh-Hadamard rotation is 3 in-register butterfly stages (dim
// bits 0-2) plus 4 cross-lane stages (DPP / permlane16_swap, no LDS); indices come from a
// 256-cell LDS table of the boundaries (one compare per value).
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
    int64_t n_rows;          // num_tokens * num_heads
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
    int64_t off_signs, off_norm, off_rnorm;
    // unpacked output
    int64_t* indices;
    float* norms;
    float* k_mse;
    float* signs;
    float* rnorm;
};

// Lane layout: lane L of a wave holds dims 8c..8c+7 of row rho of the wave's 4 rows, with
//   c = L bits {0, 1, 3, 4},  rho = L bits {2, 5}.
// The 16 lanes of a row then differ in lane bits 0, 1, 3, 4, and every exchange inside a row is
// a DPP quad_perm (bits 0, 1), a DPP row_ror:8 (bit 3) or a permlane16_swap (bit 4): no LDS.
__device__ __forceinline__ int lane_dims(int L) { return (L & 3) | ((L >> 1) & 12); }
__device__ __forceinline__ int lane_row(int L) { return ((L >> 2) & 1) | ((L >> 4) & 2); }

constexpr int kDppXor1 = 0xB1;   // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;   // quad_perm [2, 3, 0, 1]
constexpr int kDppXor8 = 0x128;  // row_ror:8 (lane l <- l ^ 8 inside a row of 16)
template <int CTRL>
__device__ __forceinline__ float dppf(float x) {
    // bound_ctrl with a zero old value: lets the compiler fold the move into the consuming add
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, true));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dppu(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, CTRL, 0xf, 0xf, false);
}
// Values of lanes L & ~16 and L | 16.
__device__ __forceinline__ void rows16(float x, float& even, float& odd) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    even = __uint_as_float(r[0]);
    odd = __uint_as_float(r[1]);
}

// Sum over the 16 lanes of a row, in the order of an xor butterfly over dims bits 3, 4, 5, 6:
// every lane of the row gets the same bits.
__device__ __forceinline__ float row_sum16(float v) {
    v += dppf<kDppXor1>(v);
    v += dppf<kDppXor2>(v);
    v += dppf<kDppXor8>(v);
    float e, o;
    rows16(v, e, o);
    return e + o;
}

// Normalised Hadamard transform of a row in the lane layout above (dims 8c + k in v[k]):
// butterflies (u, w) -> (u + w, u - w) over dims bits 0..6, then the scale h.  A cross-lane
// stage computes partner + s * own with s = -1 in the upper lane (u - w there, exactly), the
// partner read through DPP or permlane16_swap.
__device__ __forceinline__ void wht_row(float (&v)[8], int L, float h) {
#pragma unroll
    for (int b = 1; b < 8; b <<= 1) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            if (!(k & b)) {
                const float u = v[k], w = v[k | b];
                v[k] = u + w;
                v[k | b] = u - w;
            }
        }
    }
    auto stage = [&](auto dpp, float s) {
        float t[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) t[k] = v[k] * s;
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = dpp(v[k]) + t[k];
    };
    stage([](float x) { return dppf<kDppXor1>(x); }, (L & 1) ? -1.f : 1.f);
    stage([](float x) { return dppf<kDppXor2>(x); }, (L & 2) ? -1.f : 1.f);
    stage([](float x) { return dppf<kDppXor8>(x); }, (L & 8) ? -1.f : 1.f);
    const float s4 = (L & 16) ? -1.f : 1.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        float e, o;
        rows16(v[k], e, o);
        v[k] = __builtin_fmaf(o, s4, e);  // lower lane: e + o, upper lane: e - o
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] *= h;
}

// Left searchsorted over NB sorted boundaries (count of boundaries < x; NaN -> NB) through a
// table of 256 equal cells over [lo, hi] (one cell of margin past the outer boundaries): cell k
// holds c0 = #{b < edge_k - eps} and the one boundary inside [edge_k - eps, edge_k+1 + eps] (or
// +inf), so idx = c0 + (b < x) for any x whose computed cell is within eps of its true cell
// (|x| <= 1 here, the cell arithmetic errs by < 1e-6 * (hi - lo) = eps / 10).  A codebook with two
// boundaries in one such cell sets `bad` and the kernel counts linearly instead.
constexpr int kCells = 256;
struct CellQuant {
    float inv_w, c;  // cell = trunc(x * inv_w + c)
};
template <int NB>
__device__ __forceinline__ CellQuant build_cells(const float (&bd)[NB], const float* boundaries, uint2* tab,
                                                 int* bad) {
    float span = bd[NB - 1] - bd[0];
    span = span > 0.f ? span : 1.f;
    const float lo = bd[0] - span * (1.f / 64.f);
    const float hi = bd[NB - 1] + span * (1.f / 64.f);
    const float w = (hi - lo) * (1.f / kCells);
    const float eps = (hi - lo) * 1e-5f;
    for (int k = threadIdx.x; k < kCells; k += blockDim.x) {
        const float e0 = lo + (float)k * w - eps, e1 = lo + (float)(k + 1) * w + eps;
        int c0 = 0, c1 = 0;
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            c0 += bd[i] < e0 ? 1 : 0;
            c1 += bd[i] <= e1 ? 1 : 0;
        }
        if (c1 - c0 > 1 || !(w > 0.f)) atomicOr(bad, 1);
        const float b = c1 > c0 ? boundaries[c0] : __builtin_huge_valf();
        tab[k] = make_uint2(__float_as_uint(b), (uint32_t)c0);
    }
    CellQuant q;
    q.inv_w = (float)kCells / (hi - lo);
    q.c = -lo * q.inv_w;
    return q;
}
template <int NB>
__device__ __forceinline__ int quant_cell(float x, const CellQuant& q, const uint2* tab) {
    int cell = (int)__builtin_fmaf(x, q.inv_w, q.c);
    cell = cell < 0 ? 0 : (cell > kCells - 1 ? kCells - 1 : cell);
    const uint2 e = tab[cell];
    const int idx = (int)e.y + (__uint_as_float(e.x) < x ? 1 : 0);
    return x != x ? NB : idx;  // searchsorted puts NaN last
}
template <int NB>
__device__ __forceinline__ int quant_linear(float x, const float (&bd)[NB]) {
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < NB; ++i) cnt += (bd[i] < x) ? 1 : 0;
    return x != x ? NB : cnt;
}

template <int BITS, bool QJL, int MODE>
__global__ __launch_bounds__(256) void compress_kernel(CompressParams p) {
    constexpr int NC = 1 << BITS;
    constexpr int NB = NC - 1;
    __shared__ float s_cent[NC];
    __shared__ uint2 s_cells[kCells];
    __shared__ int s_bad;
    if (threadIdx.x < NC) s_cent[threadIdx.x] = p.centroids[threadIdx.x];
    if (threadIdx.x == 0) s_bad = 0;
    // Boundaries are uniform: the loads below become scalar loads kept in SGPRs.
    float bd[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) bd[i] = p.boundaries[i];
    __syncthreads();
    const CellQuant cq = build_cells<NB>(bd, p.boundaries, s_cells, &s_bad);
    __syncthreads();
    const bool cells = s_bad == 0;

    const int L = threadIdx.x & 63;
    const int c = lane_dims(L);                                      // dims 8c..8c+7
    const int row_in_wg = 4 * (int)(threadIdx.x >> 6) + lane_row(L);  // 0..15

    for (int64_t row0 = (int64_t)blockIdx.x * 16; row0 < p.n_rows; row0 += (int64_t)gridDim.x * 16) {
        const int64_t row = row0 + row_in_wg;
        const bool row_ok = row < p.n_rows;
        // Paged rows are head-major so that a workgroup's 16 rows are 16 consecutive tokens.
        int64_t tok, head;
        if (MODE == MODE_PAGED) {
            if (p.idx32) {
                const uint32_t r = row_ok ? (uint32_t)row : 0u, nt = (uint32_t)p.num_tokens;
                const uint32_t h = r / nt;
                head = h;
                tok = r - h * nt;
            } else {
                head = row_ok ? row / p.num_tokens : 0;
                tok = row_ok ? row - head * p.num_tokens : 0;
            }
        } else {
            head = 0;
            tok = row_ok ? row : 0;
        }

        float v[8];
        if (row_ok) {
            tq_load8(p.x, tok * p.x_stride_token + head * p.x_stride_head + 8 * c, p.x_dtype, v);
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = 0.f;
        }
        if (p.rotate) wht_row(v, L, p.wht_scale);

        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k) ss = __builtin_fmaf(v[k], v[k], ss);
        ss = row_sum16(ss);
        const float norm = __builtin_sqrtf(ss);
        const float den = norm + 1e-8f;
        const float rcp = 1.0f / den;

        int idx[8];
        float xn[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) xn[k] = tq_div_rn(v[k], den, rcp);
        if (cells) {
#pragma unroll
            for (int k = 0; k < 8; ++k) idx[k] = quant_cell<NB>(xn[k], cq, s_cells);
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) idx[k] = quant_linear<NB>(xn[k], bd);
        }

        float rn = 0.f;
        uint32_t sbits = 0;
        float cv[8];
        if (QJL || MODE == MODE_UNPACKED) {
#pragma unroll
            for (int k = 0; k < 8; ++k) cv[k] = s_cent[idx[k]];
        }
        if (QJL) {
            float rs = 0.f;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                float r = (xn[k] - cv[k]) * norm;
                rs = __builtin_fmaf(r, r, rs);
                sbits |= (r >= 0.f ? 1u : 0u) << k;
            }
            rn = __builtin_sqrtf(row_sum16(rs));
        }

        if (MODE == MODE_UNPACKED) {
            if (row_ok) {
                int64_t* ip = p.indices + row * TQ_HEAD_DIM + 8 * c;
                float* kp = p.k_mse + row * TQ_HEAD_DIM + 8 * c;
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    ip[k] = idx[k];
                    kp[k] = cv[k] * norm;
                }
                if (QJL) {
                    float* sp = p.signs + row * TQ_HEAD_DIM + 8 * c;
#pragma unroll
                    for (int k = 0; k < 8; ++k) sp[k] = ((sbits >> k) & 1u) ? 1.f : -1.f;
                }
                if (c == 0) {
                    p.norms[row] = norm;
                    if (QJL) p.rnorm[row] = rn;
                }
            }
        } else {
            int64_t slot = -1;
            if (row_ok) {
                slot = p.slot_i64 ? static_cast<const int64_t*>(p.slot_mapping)[tok]
                                  : (int64_t) static_cast<const int32_t*>(p.slot_mapping)[tok];
            }
            const bool write = row_ok && slot >= 0 && slot < p.num_blocks * p.block_size;
            int64_t blk, r_in_blk;
            if (p.idx32) {
                const uint32_t sl = write ? (uint32_t)slot : 0u, bs = (uint32_t)p.block_size;
                const uint32_t b = sl / bs;
                blk = b;
                r_in_blk = sl - b * bs;
            } else {
                blk = write ? slot / p.block_size : 0;
                r_in_blk = write ? slot - blk * p.block_size : 0;
            }
            uint8_t* tile = p.cache + blk * p.stride_block + head * p.stride_head;

            uint32_t w = 0;
#pragma unroll
            for (int k = 0; k < 8; ++k) w |= (uint32_t)idx[k] << (BITS * k);
            uint8_t* irow = tile + r_in_blk * (16 * BITS);
            // lanes c..c+3 of a row (c % 4 == 0) are one quad: the first lane gathers the others
            const bool quad0 = (L & 3) == 0;
            if (BITS == 3) {
                // 24 bits per lane: the quad's four lanes make 12 aligned bytes.
                const uint32_t w1 = dppu<0x55>(w), w2 = dppu<0xAA>(w), w3 = dppu<0xFF>(w);
                if (write && quad0) {
                    uint32_t* dst = reinterpret_cast<uint32_t*>(irow + 12 * (c >> 2));
                    dst[0] = w | (w1 << 24);
                    dst[1] = (w1 >> 8) | (w2 << 16);
                    dst[2] = (w2 >> 16) | (w3 << 8);
                }
            } else if (BITS == 4) {
                if (write) reinterpret_cast<uint32_t*>(irow)[c] = w;
            } else if (BITS == 2) {
                if (write) reinterpret_cast<uint16_t*>(irow)[c] = (uint16_t)w;
            } else {
                if (write) irow[c] = (uint8_t)w;
            }
            if (QJL) {
                const uint32_t s1 = dppu<0x55>(sbits), s2 = dppu<0xAA>(sbits), s3 = dppu<0xFF>(sbits);
                if (write && quad0) {
                    uint32_t* dst = reinterpret_cast<uint32_t*>(tile + p.off_signs + r_in_blk * 16 + 4 * (c >> 2));
                    *dst = sbits | (s1 << 8) | (s2 << 16) | (s3 << 24);
                }
            }
            if (write && c == 0) {
                reinterpret_cast<uint16_t*>(tile + p.off_norm)[r_in_blk] = (uint16_t)tq_f32_to_f16_bits(norm);
                if (QJL)
                    reinterpret_cast<uint16_t*>(tile + p.off_rnorm)[r_in_blk] = (uint16_t)tq_f32_to_f16_bits(rn);
            }
        }
    }
}

template <int MODE>
int launch_compress(const CompressParams& p, int bits, int qjl, hipStream_t stream) {
    if (p.n_rows <= 0) return TQ_OK;
    // Workgroups loop over 16-row groups; 2048 of them (8 per CU) amortise the LDS set-up.
    int64_t groups = (p.n_rows + 15) / 16;
    int grid = (int)(groups < 2048 ? groups : 2048);
#define TQ_LAUNCH(B, Q)                                                                     \
    hipLaunchKernelGGL((compress_kernel<B, Q, MODE>), dim3(grid), dim3(256), 0, stream, p)
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

extern "C" int tq_compress_paged(const void* x, int x_dtype, int64_t x_stride_token, int64_t x_stride_head,
                                 int64_t num_tokens, int num_heads, int head_dim,
                                 const void* slot_mapping, int slot_dtype,
                                 void* cache, int64_t cache_stride_block, int64_t cache_stride_head,
                                 int64_t num_blocks, int block_size,
                                 int bits, int use_qjl, int rotate, float wht_scale,
                                 const float* centroids, const float* boundaries,
                                 tq_stream_t stream) {
    if (head_dim != TQ_HEAD_DIM) return TQ_ERR_HEAD_DIM;
    if (bits < 2 || bits > 4) return TQ_ERR_BITS;
    if (block_size <= 0 || block_size % 16) return TQ_ERR_BLOCK_SIZE;
    if (num_tokens < 0 || num_heads <= 0 || num_blocks < 0) return TQ_ERR_INVALID_ARGUMENT;
    if (slot_dtype != TQ_I32 && slot_dtype != TQ_I64) return TQ_ERR_DTYPE;
    if (num_tokens == 0 || num_blocks == 0) return TQ_OK;
    if (!x || !slot_mapping || !cache || !centroids || !boundaries) return TQ_ERR_INVALID_ARGUMENT;
    int rc = check_x(x, x_dtype);
    if (rc) return rc;
    if (x_stride_token % 8 || x_stride_head % 8) return TQ_ERR_ALIGNMENT;
    const tq_tile_geom g = tq_make_tile_geom(block_size, bits, use_qjl);
    if (!aligned(cache, 16) || cache_stride_block % 16 || cache_stride_head % 16) return TQ_ERR_ALIGNMENT;
    if (cache_stride_head < g.bytes && num_heads > 1) return TQ_ERR_INVALID_ARGUMENT;
    CompressParams p = {};
    p.x = x;
    p.x_dtype = x_dtype;
    p.x_stride_token = x_stride_token;
    p.x_stride_head = x_stride_head;
    p.num_tokens = num_tokens;
    p.num_heads = num_heads;
    p.n_rows = num_tokens * num_heads;
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
    p.off_signs = g.off_signs;
    p.off_norm = g.off_norm;
    p.off_rnorm = g.off_rnorm;
    p.idx32 = (p.n_rows < (1ll << 31) && num_blocks * (int64_t)block_size < (1ll << 31)) ? 1 : 0;
    return launch_compress<MODE_PAGED>(p, bits, use_qjl, (hipStream_t)stream);
}
