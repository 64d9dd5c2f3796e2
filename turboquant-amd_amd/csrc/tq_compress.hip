// PolarQuant compression kernels for gfx950.
//
// One 128-dim row per 16 lanes: lane c holds dims 8c..8c+7, so a wave64 works on 4 rows
// and a 256-thread workgroup on 16 rows.  The Walsh-Hadamard rotation is 3 in-register
// butterfly stages (dim bits 0-2) plus 4 cross-lane stages (dim bits 3-6 = lane bits 0-3).
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
    int64_t off_signs, off_norm, off_rnorm;
    // unpacked output
    int64_t* indices;
    float* norms;
    float* k_mse;
    float* signs;
    float* rnorm;
};

__device__ __forceinline__ float xor_sum16(float v) {
    v += __shfl_xor(v, 1);
    v += __shfl_xor(v, 2);
    v += __shfl_xor(v, 4);
    v += __shfl_xor(v, 8);
    return v;
}

template <int BITS, bool QJL, int MODE>
__global__ __launch_bounds__(256) void compress_kernel(CompressParams p) {
    constexpr int NC = 1 << BITS;
    constexpr int NB = NC - 1;
    __shared__ float s_cent[NC];
    if (threadIdx.x < NC) s_cent[threadIdx.x] = p.centroids[threadIdx.x];
    __syncthreads();

    // Boundaries are uniform: the loads below become scalar loads kept in SGPRs.
    float bd[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) bd[i] = p.boundaries[i];

    const int lane = threadIdx.x & 63;
    const int c = lane & 15;                       // dims 8c..8c+7
    const int row_in_wg = (threadIdx.x >> 4);      // 0..15

    for (int64_t row0 = (int64_t)blockIdx.x * 16; row0 < p.n_rows; row0 += (int64_t)gridDim.x * 16) {
        const int64_t row = row0 + row_in_wg;
        const bool row_ok = row < p.n_rows;
        // Paged rows are head-major so that a workgroup's 16 rows are 16 consecutive tokens.
        int64_t tok, head;
        if (MODE == MODE_PAGED) {
            head = row_ok ? row / p.num_tokens : 0;
            tok = row_ok ? row - head * p.num_tokens : 0;
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

        if (p.rotate) {
            // Natural-order Hadamard: stage for index bit b maps (u, v) -> (u + v, u - v).
#pragma unroll
            for (int b = 1; b < 8; b <<= 1) {
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    if (!(k & b)) {
                        float u = v[k], w = v[k | b];
                        v[k] = u + w;
                        v[k | b] = u - w;
                    }
                }
            }
#pragma unroll
            for (int m = 1; m < 16; m <<= 1) {
                const bool upper = (c & m) != 0;
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    float o = __shfl_xor(v[k], m);
                    v[k] = upper ? (o - v[k]) : (v[k] + o);
                }
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] *= p.wht_scale;
        }

        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k) ss = __builtin_fmaf(v[k], v[k], ss);
        ss = xor_sum16(ss);
        const float norm = __builtin_sqrtf(ss);
        const float den = norm + 1e-8f;
        const float rcp = 1.0f / den;

        int idx[8];
        float xn[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            xn[k] = tq_div_rn(v[k], den, rcp);
            int cnt = 0;
#pragma unroll
            for (int i = 0; i < NB; ++i) cnt += (bd[i] < xn[k]) ? 1 : 0;
            idx[k] = (xn[k] != xn[k]) ? NB : cnt;  // searchsorted puts NaN last
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
            rn = __builtin_sqrtf(xor_sum16(rs));
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
            const int64_t blk = write ? slot / p.block_size : 0;
            const int64_t r_in_blk = write ? slot - blk * p.block_size : 0;
            uint8_t* tile = p.cache + blk * p.stride_block + head * p.stride_head;

            uint32_t w = 0;
#pragma unroll
            for (int k = 0; k < 8; ++k) w |= (uint32_t)idx[k] << (BITS * k);
            uint8_t* irow = tile + r_in_blk * (16 * BITS);
            if (BITS == 3) {
                // 24 bits per lane: lanes 4j..4j+3 assemble 12 aligned bytes.
                uint32_t w1 = __shfl_down(w, 1), w2 = __shfl_down(w, 2), w3 = __shfl_down(w, 3);
                if (write && (c & 3) == 0) {
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
                uint32_t s1 = __shfl_down(sbits, 1), s2 = __shfl_down(sbits, 2), s3 = __shfl_down(sbits, 3);
                if (write && (c & 3) == 0) {
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
    int64_t groups = (p.n_rows + 15) / 16;
    int grid = (int)(groups < 65536 ? groups : 65536);
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
    return launch_compress<MODE_PAGED>(p, bits, use_qjl, (hipStream_t)stream);
}
