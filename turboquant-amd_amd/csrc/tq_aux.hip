// Bit-level helpers of the packed format and the ABI utilities.
#include "tq_common.h"

namespace {

// One thread per 16-byte sign row: out bit 32c+k = in bit 4k+c (c < 4, k < 32).
// Follows permute_signs_for_chunked (turboquant/kernels/packed_compress.py:180-216).
__global__ __launch_bounds__(256) void permute_signs_kernel(const uint8_t* in, uint8_t* out, int64_t n_rows) {
    for (int64_t row = (int64_t)blockIdx.x * 256 + threadIdx.x; row < n_rows; row += (int64_t)gridDim.x * 256) {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint8_t* b = in + row * 16 + 4 * i;
            w[i] = (uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) | ((uint32_t)b[3] << 24);
        }
        uint32_t o[4] = {0, 0, 0, 0};
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
#pragma unroll
            for (int k = 0; k < 32; ++k) {
                const int src = 4 * k + cc;
                o[cc] |= ((w[src >> 5] >> (src & 31)) & 1u) << k;
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint8_t* b = out + row * 16 + 4 * i;
            b[0] = (uint8_t)o[i];
            b[1] = (uint8_t)(o[i] >> 8);
            b[2] = (uint8_t)(o[i] >> 16);
            b[3] = (uint8_t)(o[i] >> 24);
        }
    }
}

// One thread per (row, dim): field d of a little-endian stream of b-bit fields.
// Follows unpack_2bit / unpack_1bit (turboquant/kernels/packed_compress.py:145-154).
__global__ __launch_bounds__(256) void unpack_kernel(const uint8_t* in, int8_t* out, int64_t n_rows, int bits) {
    const int64_t total = n_rows * TQ_HEAD_DIM;
    const int row_bytes = 16 * bits;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t row = i / TQ_HEAD_DIM;
        const int d = (int)(i - row * TQ_HEAD_DIM);
        const int pos = bits * d;
        const uint8_t* r = in + row * row_bytes;
        uint32_t v = r[pos >> 3];
        if ((pos >> 3) + 1 < row_bytes) v |= (uint32_t)r[(pos >> 3) + 1] << 8;
        out[i] = (int8_t)((v >> (pos & 7)) & ((1u << bits) - 1u));
    }
}

// y = x H per 128-element row (H = make_wht_matrix(128)), 16 threads per row: thread t holds
// elements 8t .. 8t+7 (butterflies over element bits 0-2 in registers, bits 3-6 across lanes
// 1, 2, 4, 8 of the row).  Rows of a grid-stride step are block-uniform, so every lane takes
// part in the exchanges; rows past the end carry zeros and store nothing.
// Follows TurboQuantFP8State.rotate_query / rotate_output (integration/vllm_backend.py:158-177).
__global__ __launch_bounds__(256) void wht_rows_kernel(const void* x, int x_dt, int64_t x_ss, int64_t x_sh, int hn,
                                                       int64_t n_rows, int vec, void* y, int y_dt, int64_t y_ss,
                                                       int64_t y_sh, float h) {
    const int t = threadIdx.x & 15;
    for (int64_t r0 = (int64_t)blockIdx.x * 16; r0 < n_rows; r0 += (int64_t)gridDim.x * 16) {
        const int64_t row = r0 + (threadIdx.x >> 4);
        const bool valid = row < n_rows;
        const int64_t sq = valid ? row / hn : 0, hd = valid ? row - sq * hn : 0;
        const int64_t xo = sq * x_ss + hd * x_sh + 8 * t;
        float v[8];
        if (valid && vec) {
            tq_load8(x, xo, x_dt, v);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = valid ? tq_load1(x, xo + i, x_dt) : 0.f;
        }
        tq_wht_regs(v);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float a = v[i];
#pragma unroll
            for (int m = 1; m < 16; m <<= 1) a = tq_wht_lane(a, m);
            v[i] = a * h;
        }
        if (valid) {
            const int64_t yo = sq * y_ss + hd * y_sh + 8 * t;
#pragma unroll
            for (int i = 0; i < 8; ++i) tq_store1(y, yo + i, y_dt, v[i]);
        }
    }
}

int grid_for(int64_t items) {
    int64_t g = (items + 255) / 256;
    return (int)(g < 65536 ? (g > 0 ? g : 1) : 65536);
}

}  // namespace

extern "C" int tq_abi_version(void) { return TQ_ABI_VERSION; }

extern "C" const char* tq_status_string(int status) {
    switch (status) {
        case TQ_OK: return "ok";
        case TQ_ERR_INVALID_ARGUMENT: return "invalid argument";
        case TQ_ERR_HEAD_DIM: return "head_dim must be 128";
        case TQ_ERR_BITS: return "unsupported bit width";
        case TQ_ERR_ALIGNMENT: return "pointer or stride not aligned as required";
        case TQ_ERR_WORKSPACE: return "workspace missing, too small or not 256-byte aligned";
        case TQ_ERR_GQA: return "num_q_heads must be a multiple of num_kv_heads with group size <= 16";
        case TQ_ERR_DTYPE: return "unsupported dtype";
        case TQ_ERR_BLOCK_SIZE: return "block_size must be a positive multiple of 16";
        case TQ_ERR_CHUNK: return "tokens_per_chunk must be 0 (balanced schedule) or a positive multiple of 16";
        case TQ_ERR_SCRATCH_LIMIT:
            return "the call needs more split-K scratch than tq_decode_noalloc's fixed array "
                   "(TQ_NOALLOC_SCRATCH_BYTES): use a larger tokens_per_chunk, or fixed chunks instead of the "
                   "balanced schedule (tokens_per_chunk 0) for very large batches";
        default: break;
    }
    if (status > 0) return hipGetErrorString((hipError_t)status);
    return "unknown status";
}

extern "C" int tq_permute_signs(const uint8_t* in, uint8_t* out, int64_t n_rows, int head_dim, tq_stream_t stream) {
    if (head_dim != TQ_HEAD_DIM) return TQ_ERR_HEAD_DIM;
    if (n_rows < 0) return TQ_ERR_INVALID_ARGUMENT;
    if (n_rows == 0) return TQ_OK;
    if (!in || !out || in == out) return TQ_ERR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(permute_signs_kernel, dim3(grid_for(n_rows)), dim3(256), 0, (hipStream_t)stream, in, out, n_rows);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TQ_OK : (int)e;
}

extern "C" int tq_unpack_bits(const uint8_t* in, int8_t* out, int64_t n_rows, int head_dim, int bits, tq_stream_t stream) {
    if (head_dim != TQ_HEAD_DIM) return TQ_ERR_HEAD_DIM;
    if (bits < 1 || bits > 4) return TQ_ERR_BITS;
    if (n_rows < 0) return TQ_ERR_INVALID_ARGUMENT;
    if (n_rows == 0) return TQ_OK;
    if (!in || !out) return TQ_ERR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(unpack_kernel, dim3(grid_for(n_rows * TQ_HEAD_DIM)), dim3(256), 0, (hipStream_t)stream, in, out,
                       n_rows, bits);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TQ_OK : (int)e;
}

extern "C" int tq_wht_rows(const void* x, int x_dtype, int64_t x_stride_seq, int64_t x_stride_head,
                           int num_seqs, int num_heads, int head_dim,
                           void* y, int y_dtype, int64_t y_stride_seq, int64_t y_stride_head,
                           tq_stream_t stream) {
    if (head_dim != TQ_HEAD_DIM) return TQ_ERR_HEAD_DIM;
    if (num_seqs < 0 || num_heads <= 0) return TQ_ERR_INVALID_ARGUMENT;
    if (x_dtype != TQ_F32 && x_dtype != TQ_F16 && x_dtype != TQ_BF16) return TQ_ERR_DTYPE;
    if (y_dtype != TQ_F32 && y_dtype != TQ_F16 && y_dtype != TQ_BF16) return TQ_ERR_DTYPE;
    if (num_seqs == 0) return TQ_OK;
    if (!x || !y) return TQ_ERR_INVALID_ARGUMENT;
    const int64_t n_rows = (int64_t)num_seqs * num_heads;
    // 8-element vector loads: 16-byte (f16/bf16) or 32-byte (f32) aligned rows
    const uintptr_t al = x_dtype == TQ_F32 ? 32 : 16;
    const int vec = ((uintptr_t)x % al == 0) && x_stride_seq % 8 == 0 && x_stride_head % 8 == 0;
    const int64_t groups = (n_rows + 15) / 16;
    const int grid = (int)(groups < 65536 ? groups : 65536);
    hipLaunchKernelGGL(wht_rows_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, x, x_dtype, x_stride_seq,
                       x_stride_head, num_heads, n_rows, vec, y, y_dtype, y_stride_seq, y_stride_head,
                       0.08838834764831845f);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TQ_OK : (int)e;
}
