// polarquant_compress with a general rotation matrix (fp32), for the entry point that takes an
// arbitrary rotation_matrix instead of the Walsh-Hadamard transform (core/quantizer.py:135-183):
//   x_rot = x @ R; norm = |x_rot|; x_n = x_rot / (norm + 1e-8); idx = #{b < x_n};
//   k_mse = c[idx] * norm; QJL: r = (x_n - c[idx]) * norm, rnorm = |r|, sign = r >= 0 ? +1 : -1.
// The product is fp32 FMAs summed over d = 0..127 in order.
//
// Layout: the matrix (128 x 128 f32, row d holds R[d][0..127]) is staged in LDS once per
// workgroup; each wave handles 4 rows per pass, lane l owns output columns 2l and 2l+1, and the
// 4 input rows are broadcast from LDS.  VALU work (32K FMAs per row), off the paged hot path.
//
// The packed entry point (compress_k / compress_v with PiT and PiST) runs on the matrix cores:
// tq_packed.hip.
#include "tq_common.h"

namespace {

constexpr int kRows = 4;     // rows per wave per pass
constexpr int kD = TQ_HEAD_DIM;

struct RotParams {
    const void* x;
    int x_dtype;
    int64_t x_stride;
    int64_t n_rows;
    const float* rot;
    const float* centroids;
    const float* boundaries;
    int64_t* indices;
    float* norms;
    float* k_mse;
    float* signs;
    float* rnorm;
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// acc[r] (columns 2l, 2l+1) = sum_d rows[r][d] * m[d][2l..2l+1], d ascending.
__device__ __forceinline__ void rows_times_matrix(const float* rows, const float* m, int lane, float2 (&acc)[kRows]) {
#pragma unroll
    for (int r = 0; r < kRows; ++r) acc[r] = make_float2(0.f, 0.f);
    for (int d = 0; d < kD; d += 4) {
        float4 xr[kRows];
#pragma unroll
        for (int r = 0; r < kRows; ++r) xr[r] = *reinterpret_cast<const float4*>(rows + r * kD + d);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float2 mm = *reinterpret_cast<const float2*>(m + (d + k) * kD + 2 * lane);
#pragma unroll
            for (int r = 0; r < kRows; ++r) {
                const float xv = k == 0 ? xr[r].x : k == 1 ? xr[r].y : k == 2 ? xr[r].z : xr[r].w;
                acc[r].x = __builtin_fmaf(xv, mm.x, acc[r].x);
                acc[r].y = __builtin_fmaf(xv, mm.y, acc[r].y);
            }
        }
    }
}

template <int BITS, bool QJL>
__global__ __launch_bounds__(256) void rotate_compress_kernel(RotParams p) {
    constexpr int NC = 1 << BITS;
    constexpr int NB = NC - 1;
    extern __shared__ float s_mem[];
    float* s_rot = s_mem;
    float* s_rows = s_mem + kD * kD;  // [4 waves][kRows][128]

    for (int i = threadIdx.x; i < kD * kD; i += 256) s_rot[i] = p.rot[i];
    __shared__ float s_cent[NC], s_bnd[NB > 0 ? NB : 1];
    if (threadIdx.x < NC) s_cent[threadIdx.x] = p.centroids[threadIdx.x];
    if (threadIdx.x < NB) s_bnd[threadIdx.x] = p.boundaries[threadIdx.x];
    __syncthreads();

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    float* rows = s_rows + wave * kRows * kD;
    const int64_t ngroups = (p.n_rows + kRows - 1) / kRows;

    // Every wave of the workgroup runs the same number of passes (barriers inside).
    for (int64_t base = (int64_t)blockIdx.x * 4; base < ngroups; base += (int64_t)gridDim.x * 4) {
        const int64_t row0 = (base + wave) * kRows;
        float2 xv[kRows];
        bool live[kRows];
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            live[r] = row0 + r < p.n_rows;
            xv[r] = make_float2(0.f, 0.f);
            if (live[r]) {
                const int64_t o = (row0 + r) * p.x_stride + 2 * lane;
                xv[r] = make_float2(tq_load1(p.x, o, p.x_dtype), tq_load1(p.x, o + 1, p.x_dtype));
            }
        }
#pragma unroll
        for (int r = 0; r < kRows; ++r) *reinterpret_cast<float2*>(rows + r * kD + 2 * lane) = xv[r];
        __syncthreads();
        float2 rot[kRows];
        rows_times_matrix(rows, s_rot, lane, rot);
        __syncthreads();  // rows is rewritten by the next pass

#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            const float nrm = __builtin_sqrtf(wave_sum(__builtin_fmaf(rot[r].x, rot[r].x, rot[r].y * rot[r].y)));
            const float den = nrm + 1e-8f;
            const float xn[2] = {rot[r].x / den, rot[r].y / den};
            float rr[2];
            int idx[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                int k = 0;
#pragma unroll
                for (int b = 0; b < NB; ++b) k += s_bnd[b] < xn[e] ? 1 : 0;
                idx[e] = xn[e] != xn[e] ? NB : k;  // searchsorted puts NaN last
                rr[e] = (xn[e] - s_cent[idx[e]]) * nrm;
            }
            float rn = 0.f;
            if (QJL) rn = __builtin_sqrtf(wave_sum(__builtin_fmaf(rr[0], rr[0], rr[1] * rr[1])));
            if (live[r]) {
                const int64_t row = row0 + r;
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const int64_t o = row * kD + 2 * lane + e;
                    p.indices[o] = idx[e];
                    p.k_mse[o] = s_cent[idx[e]] * nrm;
                    if (QJL) p.signs[o] = rr[e] >= 0.f ? 1.f : -1.f;
                }
                if (lane == 0) {
                    p.norms[row] = nrm;
                    if (QJL) p.rnorm[row] = rn;
                }
            }
        }
    }
}

int check_x(const void* x, int dtype) {
    if (dtype != TQ_F32 && dtype != TQ_F16 && dtype != TQ_BF16) return TQ_ERR_DTYPE;
    if (reinterpret_cast<uintptr_t>(x) & (dtype == TQ_F32 ? 3 : 1)) return TQ_ERR_ALIGNMENT;
    return TQ_OK;
}

size_t rot_lds_bytes() { return (size_t)kD * kD * 4 + 4 * kRows * kD * 4; }

int launch_rotate(const RotParams& p, int bits, bool qjl, hipStream_t st) {
    const size_t lds = rot_lds_bytes();
    const void* kern = nullptr;
#define TQ_RK(B)                                                                                       \
    if (bits == B) kern = qjl ? (const void*)rotate_compress_kernel<B, true> : (const void*)rotate_compress_kernel<B, false>;
    TQ_RK(1) TQ_RK(2) TQ_RK(3) TQ_RK(4)
#undef TQ_RK
    if (!kern) return TQ_ERR_BITS;
    int dev = 0, max_lds = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return (int)e;
    if ((size_t)max_lds < lds) return TQ_ERR_WORKSPACE;  // device cannot stage the matrix in LDS
    e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return (int)e;
    const int64_t groups = (p.n_rows + kRows - 1) / kRows;
    int64_t grid = (groups + 3) / 4;
    const int64_t cap = (int64_t)cus * 2;  // resident workgroups (LDS-limited)
    grid = grid < cap ? grid : cap;
    void* args[] = {const_cast<RotParams*>(&p)};
    e = hipLaunchKernel(kern, dim3((unsigned)grid), dim3(256), args, lds, st);
    if (e != hipSuccess) return (int)e;
    e = hipGetLastError();
    return e == hipSuccess ? TQ_OK : (int)e;
}

}  // namespace

// tq_packed.hip
size_t tq_packed_mfma_lds_bytes(bool proj);
int tq_packed_mfma_launch(const void* x, int x_dtype, int64_t x_stride, int64_t n_rows, const float* pit,
                          const float* pist, const float* centroids, const float* boundaries, int bits,
                          uint8_t* idx_out, uint8_t* signs_out, uint16_t* rnorm_out, uint16_t* norm_out,
                          hipStream_t st);

extern "C" int tq_polarquant_compress_matrix(const void* x, int x_dtype, int64_t x_row_stride, int64_t n_rows,
                                             int head_dim, const float* rotation,
                                             const float* centroids, const float* boundaries, int bits,
                                             int use_qjl, int64_t* indices, float* norms, float* k_mse,
                                             float* signs, float* rnorm, tq_stream_t stream) {
    if (head_dim != TQ_HEAD_DIM) return TQ_ERR_HEAD_DIM;
    if (bits < 1 || bits > 4) return TQ_ERR_BITS;
    if (n_rows < 0 || x_row_stride < TQ_HEAD_DIM) return TQ_ERR_INVALID_ARGUMENT;
    if (n_rows == 0) return TQ_OK;
    if (!x || !rotation || !centroids || !boundaries || !indices || !norms || !k_mse) return TQ_ERR_INVALID_ARGUMENT;
    if (use_qjl && (!signs || !rnorm)) return TQ_ERR_INVALID_ARGUMENT;
    int rc = check_x(x, x_dtype);
    if (rc) return rc;
    RotParams p = {};
    p.x = x;
    p.x_dtype = x_dtype;
    p.x_stride = x_row_stride;
    p.n_rows = n_rows;
    p.rot = rotation;
    p.centroids = centroids;
    p.boundaries = boundaries;
    p.indices = indices;
    p.norms = norms;
    p.k_mse = k_mse;
    p.signs = signs;
    p.rnorm = rnorm;
    return launch_rotate(p, bits, use_qjl != 0, (hipStream_t)stream);
}

extern "C" int tq_compress_packed(const void* x, int x_dtype, int64_t x_row_stride, int64_t n_rows, int head_dim,
                                  const float* pit, const float* pist, const float* centroids,
                                  const float* boundaries, int bits, uint8_t* idx_out, uint8_t* signs_out,
                                  uint16_t* rnorm_out, uint16_t* norm_out, tq_stream_t stream) {
    if (head_dim != TQ_HEAD_DIM) return TQ_ERR_HEAD_DIM;
    if (bits < 1 || bits > 4) return TQ_ERR_BITS;
    if (n_rows < 0 || x_row_stride < TQ_HEAD_DIM) return TQ_ERR_INVALID_ARGUMENT;
    if (n_rows == 0) return TQ_OK;
    if (!x || !pit || !centroids || !boundaries || !idx_out || !norm_out) return TQ_ERR_INVALID_ARGUMENT;
    const bool qjl = pist != nullptr;
    if (qjl && (!signs_out || !rnorm_out)) return TQ_ERR_INVALID_ARGUMENT;
    if ((reinterpret_cast<uintptr_t>(idx_out) & 3) || (qjl && (reinterpret_cast<uintptr_t>(signs_out) & 3)) ||
        (reinterpret_cast<uintptr_t>(norm_out) & 1) || (qjl && (reinterpret_cast<uintptr_t>(rnorm_out) & 1)) ||
        (reinterpret_cast<uintptr_t>(pit) & 15) || (qjl && (reinterpret_cast<uintptr_t>(pist) & 15)))
        return TQ_ERR_ALIGNMENT;
    int rc = check_x(x, x_dtype);
    if (rc) return rc;
    return tq_packed_mfma_launch(x, x_dtype, x_row_stride, n_rows, pit, pist, centroids, boundaries, bits, idx_out,
                                 signs_out, rnorm_out, norm_out, (hipStream_t)stream);
}
