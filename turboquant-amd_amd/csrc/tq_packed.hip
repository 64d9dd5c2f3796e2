// Packed K / V compression with explicit rotation matrices on the matrix cores (gfx950).
//
// Replaces compress_k / compress_v (kernels/packed_compress.py:44-142,157-177,226-240):
//   norm = |x|; x_n = x * (1 / (norm + 1e-8)); rot = x_n @ PiT; idx = #{b <= rot};
//   K: resid = (rot - c[idx]) * norm; rnorm = |resid|; sign bit = (resid @ PiST >= 0);
// indices as a little-endian bit stream (2 bits: byte j = sum_c idx[4j+c] << 2c), signs LSB
// first, norms fp16.
//
// Both products run transposed on v_mfma_f32_16x16x32_f16, the matrix as the A operand and 16
// data rows as the B operand:  rot^T[col][row] = sum_d PiT^T[col][d] x^T[d][row].  A lane then
// holds, per 16-column block cb, row (lane % 16) at columns 16cb + 4(lane / 16) + r, r = 0..3:
// four consecutive dims of one row, which is what the bit packing needs, and - with the K
// positions of the second product permuted to match (PiST is staged in LDS in that order) -
// exactly the B operand of resid @ PiST, so the residual never leaves the registers.
//
// Precision: each operand is split into fp16 hi + lo, the product is hi*hi + hi*lo + lo*hi with
// fp32 accumulation.  Error of rot_j = sum_d x_d M_dj against the exact sum, with S = sum_d |x_d
// M_dj| <= ||M_j|| (x_n has unit norm), ||M_j|| the column norm:
//   - the split: |x - hi - lo| <= 2^-22 |x| for normal values and <= 2^-25 where fp16's
//     subnormals take over (|x| < 2^-13), the same for M: 2 * 2^-22 S + 2^-25 (sum_d |M_dj| +
//     sum_d |x_d|) <= 2^-21 S + 2^-25 sqrt(128) (||M_j|| + 1);
//   - the dropped lo*lo term: 2^-22 S;
//   - accumulation: 12 MFMA steps (4 K slices x 3 products), each adding exact fp16 products
//     to the fp32 accumulator with an error of at most 2^-24 of the partial sum (measured:
//     0.445 * 2^-24), partial sums bounded by (1 + 2^-10) S: 12 * 2^-24 * 1.001 S.
// In all |rot_GPU - rot| <= 1.43e-6 S + 3.4e-7 (||M_j|| + 1) <= 1.77e-6 ||M_j|| + 3.4e-7, inside
// the band 2^-19 * max ||M_j|| + 2^-21 (1.91e-6 + 4.8e-7) used below.  Every element within the band of a boundary is decided
// exactly: the whole wave recomputes that element's dot product in fp64 from the input row and
// the fp32 matrix (one element at a time; well under 1e-4 of the elements), so the indices equal
// the float64 restatement of the reference except within fp32 rounding of a boundary.  The row
// norm is an fp64 sum and x_n is rounded once from x * (1 / (norm + 1e-8)) in fp64.  Sign bits
// come from the same hi / lo products of the residual and PiST: they equal float64's except
// where |proj| is within the analogous bound (rot's error times the row norm and the column's
// 1-norm of PiST, plus 2^-19 of the summed terms), which the tests check element by element.
//
// The matrices are staged transposed, hi and lo parts, with one 16-byte LDS store per 8
// consecutive positions of a column (a thread keeps one column).
#include <mutex>
#include <set>
#include <utility>

#include "tq_common.h"

namespace {

constexpr int kD = TQ_HEAD_DIM;
constexpr int kStride = kD + 8;   // fp16 elements per staged matrix row (272 B: no bank conflicts
                                  // among the 16 rows one ds_read_b128 wave phase touches)
// Waves per workgroup: K (PROJ) stages both matrices (139 KB of LDS, one workgroup per CU) and
// runs 8 waves, two per SIMD; V stages one (70 KB, two workgroups per CU) and runs 4.
template <bool PROJ>
constexpr int packed_wg_waves() {
    return PROJ ? 8 : 4;
}
constexpr int kRT = 2;            // 16-row tiles per wave and pass
constexpr float kNearRel = 1.0f / (1 << 19);  // band: kNearRel * max column norm + kNearAbs
constexpr float kNearAbs = 1.0f / (1 << 21);

struct PackedParams {
    const void* x;
    int x_dtype;
    int64_t x_stride;
    int64_t n_rows;
    int x_vec;                 // rows 16-byte aligned: 8-element vector loads
    const float* pit;
    const float* pist;
    const float* centroids;
    const float* boundaries;
    uint8_t* idx_out;          // [n_rows][16 * bits]
    uint8_t* signs_out;        // [n_rows][16]
    uint16_t* rnorm_out;       // fp16
    uint16_t* norm_out;        // fp16
};

__device__ __forceinline__ uint32_t or_over_groups(uint32_t x) {
    auto a = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    const uint32_t y = a[0] | a[1];
    auto b = __builtin_amdgcn_permlane16_swap(y, y, false, false);
    return b[0] | b[1];
}
// Element 2g + h of the 8 (lane group g = 0..3, h = 0, 1) by selects: an array indexed by the
// lane's group would be kept in scratch memory.
template <typename T>
__device__ __forceinline__ T pick_group(const T (&a)[8], int g, int h) {
    const T x01 = g == 1 ? a[2 + h] : a[h];
    const T x23 = g == 3 ? a[6 + h] : a[4 + h];
    return g >= 2 ? x23 : x01;
}
__device__ __forceinline__ float sum_over_groups(float x) {
    auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
__device__ __forceinline__ double wave_sum_f64(double x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, 64);
    return x;
}

// K position p (0..31) of the second product's slice -> dim offset inside the slice: the lane
// of group g holds dims 4g..4g+3 (column block 2ks) and 16 + 4g..16 + 4g + 3 (block 2ks + 1).
__host__ __device__ constexpr int perm2(int p) {
    return (p & 7) < 4 ? 4 * (p >> 3) + (p & 7) : 16 + 4 * (p >> 3) + (p & 7) - 4;
}

template <int BITS, bool PROJ, int DT>
__global__ __launch_bounds__(packed_wg_waves<PROJ>() * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void packed_compress_mfma_kernel(PackedParams p) {
    constexpr int kWaves = packed_wg_waves<PROJ>();
    constexpr int NC = 1 << BITS;
    constexpr int NB = NC - 1;
    extern __shared__ _Float16 s_h[];
    _Float16* s_m1h = s_h;                      // PiT^T hi  [col][d]
    _Float16* s_m1l = s_h + kD * kStride;       // PiT^T lo
    _Float16* s_m2h = s_h + 2 * kD * kStride;   // PiST^T hi [col][32ks + p] = PiST[32ks + perm2(p)][col]
    _Float16* s_m2l = s_h + 3 * kD * kStride;
    __shared__ float s_colss[kWaves * 64];
    __shared__ float s_colmax;
    __shared__ float s_cent[NC];

    const int tid = threadIdx.x;
    // float4 of 4 consecutive columns per thread and step (kWaves * 64 * 4 is a multiple of 128:
    // each thread keeps the same 4 columns and sums their squares)
    // Staging: task t = (column col = t % 128, group j = t / 128 of 8 positions along d) reads
    // 8 floats of the column (consecutive threads: consecutive columns, coalesced) and writes
    // their fp16 hi and lo parts as two 16-byte rows of the transposed matrix.  Thread tid always
    // has column tid % 128 and sums its squares for the column norm.
    constexpr int kThreads = kWaves * 64;
    constexpr int kTasks = kD * (kD / 8) / kThreads;
    float css = 0.f;
#pragma unroll
    for (int k = 0; k < kTasks; ++k) {
        const int t = tid + k * kThreads;
        const int col = t & (kD - 1), j = t >> 7;
        float v[8], w[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v[i] = p.pit[(8 * j + i) * kD + col];
            // PiST: position 8j + i of the permuted K slice holds dim (8j & ~31) + perm2((8j & 31) + i)
            if (PROJ) w[i] = p.pist[((8 * j & ~31) + perm2((8 * j & 31) + i)) * kD + col];
        }
        tq_half8 h, l, hw, lw;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            css = __builtin_fmaf(v[i], v[i], css);
            h[i] = (_Float16)v[i];
            l[i] = (_Float16)(v[i] - (float)h[i]);
            if (PROJ) {
                hw[i] = (_Float16)w[i];
                lw[i] = (_Float16)(w[i] - (float)hw[i]);
            }
        }
        *reinterpret_cast<tq_half8*>(s_m1h + col * kStride + 8 * j) = h;
        *reinterpret_cast<tq_half8*>(s_m1l + col * kStride + 8 * j) = l;
        if (PROJ) {
            *reinterpret_cast<tq_half8*>(s_m2h + col * kStride + 8 * j) = hw;
            *reinterpret_cast<tq_half8*>(s_m2l + col * kStride + 8 * j) = lw;
        }
    }
    if (tid < NC) s_cent[tid] = p.centroids[tid];
    // largest column 2-norm of PiT: the near-boundary threshold scales with it.  Column c's
    // partial sums are at threads c, c + 128, ...
    s_colss[tid] = css;
    __syncthreads();
    if (tid < 64) {
        float m = 0.f;
        for (int c = tid; c < kD; c += 64) {
            float t = 0.f;
            for (int u = c; u < kThreads; u += kD) t += s_colss[u];
            m = fmaxf(m, t);
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        if (tid == 0) s_colmax = m;
    }
    __syncthreads();

    float bd[NB > 0 ? NB : 1];
#pragma unroll
    for (int i = 0; i < NB; ++i) bd[i] = p.boundaries[i];
    const uint32_t near_bits = __float_as_uint(__builtin_fmaf(kNearRel, __builtin_sqrtf(s_colmax), kNearAbs));
    // idx = #{b <= v} and whether some boundary lies within the threshold of v, from the signs
    // and magnitudes of v - b (integer arithmetic: no compare-and-select chains)
    const float near_thr = __uint_as_float(near_bits);
    // near: (nearest boundary distance) - threshold, negative within the band
    auto quantize = [&](float v, uint32_t& k, float& near) {
        uint32_t neg = 0;
        float m = __builtin_huge_valf();
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const float d = v - bd[b];
            neg += __float_as_uint(d) >> 31;
            m = __builtin_fminf(m, __builtin_fabsf(d));
        }
        k = NB - neg;
        near = m - near_thr;
    };

    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15;   // data row within the tile (B column / output column)
    const int g = lane >> 4;   // K group of the operands; output rows 4g..4g+3 of a column block

    const int64_t rows_per_pass = 16 * kRT;
    const int64_t ngroups = (p.n_rows + rows_per_pass - 1) / rows_per_pass;
    for (int64_t grp = (int64_t)blockIdx.x * kWaves + wave; grp < ngroups; grp += (int64_t)gridDim.x * kWaves) {
        const int64_t row0 = grp * rows_per_pass;
        // ---- rows: load, fp64 norm, x_n, fp16 hi / lo B operands ----
        tq_half8 bh[kRT][4], bl[kRT][4];
        float norm32[kRT];
#pragma unroll
        for (int rt = 0; rt < kRT; ++rt) {
            const int64_t row = row0 + 16 * rt + n;
            const bool live = row < p.n_rows;
            float xv[4][8];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const int64_t off = row * p.x_stride + 32 * ks + 8 * g;
                if (live && p.x_vec) {
                    tq_load8(p.x, off, DT, xv[ks]);
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) xv[ks][e] = live ? tq_load1(p.x, off + e, DT) : 0.f;
                }
            }
            // fp64 norm, x_n rounded once from x * (1 / (norm + 1e-8)): an error in the norm
            // would scale rot, whose projection rot @ PiST is much larger than the residual's
            double ss = 0.0;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int e = 0; e < 8; ++e) ss = __builtin_fma((double)xv[ks][e], (double)xv[ks][e], ss);
            ss += __shfl_xor(ss, 16, 64);
            ss += __shfl_xor(ss, 32, 64);
            const double nrm = __builtin_sqrt(ss);
            // the fp16 norm is rounded from this fp32 value (as the reference's .half() of an fp32
            // norm); without the barrier the compiler may round fp64 -> fp16 in one step
            float n32 = (float)nrm;
            asm volatile("" : "+v"(n32));
            norm32[rt] = n32;
            const double inv = 1.0 / (nrm + 1e-8);
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    // x_n rounded to fp32 first (the hi part is then one fp32 -> fp16 conversion;
                    // left to itself the compiler turns fp64 -> fp32 -> fp16 into a software
                    // fp64 -> fp16 rounding of ~25 instructions per element)
                    float xn = (float)((double)xv[ks][e] * inv);
                    asm("" : "+v"(xn));
                    const _Float16 h = (_Float16)xn;
                    bh[rt][ks][e] = h;
                    bl[rt][ks][e] = (_Float16)(xn - (float)h);
                }
        }

        // ---- rot^T = PiT^T x_n^T ----
        // 32 steps (K slice ks = step / 8, column block cb = step % 8); the A fragments of the
        // next step are loaded before this step's products (the barrier keeps the schedule to
        // that one step of look-ahead: hoisting all 64 loads runs out of registers)
        tq_floatx4 acc[kRT][8];
#pragma unroll
        for (int rt = 0; rt < kRT; ++rt)
#pragma unroll
            for (int cb = 0; cb < 8; ++cb) acc[rt][cb] = tq_floatx4{0.f, 0.f, 0.f, 0.f};
        {
            tq_half8 ah[2], al[2];
            auto frag = [&](int step, tq_half8& h, tq_half8& l) {
                const int o = (16 * (step & 7) + n) * kStride + 32 * (step >> 3) + 8 * g;
                h = *reinterpret_cast<const tq_half8*>(s_m1h + o);
                l = *reinterpret_cast<const tq_half8*>(s_m1l + o);
            };
            frag(0, ah[0], al[0]);
#pragma unroll
            for (int step = 0; step < 32; ++step) {
                if (step + 1 < 32) frag(step + 1, ah[(step + 1) & 1], al[(step + 1) & 1]);
                const int ks = step >> 3, cb = step & 7;
#pragma unroll
                for (int rt = 0; rt < kRT; ++rt) {
                    acc[rt][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[step & 1], bh[rt][ks], acc[rt][cb], 0, 0, 0);
                    acc[rt][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[step & 1], bl[rt][ks], acc[rt][cb], 0, 0, 0);
                    acc[rt][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[step & 1], bh[rt][ks], acc[rt][cb], 0, 0, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }

        // ---- indices (BITS-bit fields of the 4 elements of (rt, cb), word 8 rt + cb) and the
        // elements near a boundary.  Element e = 32 rt + 4 cb + r of a lane is
        // rot[row0 + 16 rt + n][16 cb + 4 g + r]. ----
        uint32_t kf[8 * kRT];
        uint32_t nearw[kRT];
#pragma unroll
        for (int rt = 0; rt < kRT; ++rt) {
            nearw[rt] = 0;
#pragma unroll
            for (int cb = 0; cb < 8; ++cb) {
                kf[8 * rt + cb] = 0;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    uint32_t k;
                    float nr;
                    quantize(acc[rt][cb][r], k, nr);
                    kf[8 * rt + cb] |= k << (BITS * r);
                    // shift the sign bit of nr in at bit 0 (one funnel shift): after the 32
                    // elements, element 4 cb + r of the tile sits at bit 31 - (4 cb + r)
                    nearw[rt] = __builtin_amdgcn_alignbit(nearw[rt], __float_as_uint(nr), 31);
                }
            }
            nearw[rt] = __builtin_bitreverse32(nearw[rt]);  // element e at bit e
            if (row0 + 16 * rt + n >= p.n_rows) nearw[rt] = 0;
        }
        uint64_t near = nearw[0] | (kRT > 1 ? ((uint64_t)nearw[kRT > 1 ? 1 : 0] << 32) : 0ull);
        // Exact decisions, one near element at a time (about 1e-5 of them): the whole wave
        // computes that row's norm and dot product in fp64 (x * (1 / (norm + 1e-8)) @ PiT as the
        // reference orders it) and the owning lane rewrites the element's index field.  The
        // residual keeps the fp32 value, which is within the threshold of the boundary.
        while (true) {
            const uint64_t lanes = __builtin_amdgcn_ballot_w64(near != 0);
            if (!lanes) break;
            const int src = __builtin_ctzll(lanes);
            const uint32_t mlo = __builtin_amdgcn_readlane((uint32_t)near, src);
            const uint32_t mhi = __builtin_amdgcn_readlane((uint32_t)(near >> 32), src);
            const int e = mlo ? __builtin_ctz(mlo) : 32 + __builtin_ctz(mhi);
            const int64_t xo = (row0 + 16 * (e >> 5) + (src & 15)) * p.x_stride;
            const int col = 16 * ((e >> 2) & 7) + 4 * (src >> 4) + (e & 3);
            // every lane: dims lane and lane + 64 of the row
            const double x0 = (double)tq_load1(p.x, xo + lane, DT);
            const double x1 = (double)tq_load1(p.x, xo + lane + 64, DT);
            const double dot = wave_sum_f64(__builtin_fma(x1, (double)p.pit[(lane + 64) * kD + col],
                                                          x0 * (double)p.pit[lane * kD + col]));
            const double ss = wave_sum_f64(__builtin_fma(x1, x1, x0 * x0));
            const double exact = dot * (1.0 / (__builtin_sqrt(ss) + 1e-8));
            uint32_t k = 0;
#pragma unroll
            for (int b = 0; b < NB; ++b) k += exact >= (double)bd[b] ? 1u : 0u;
            if (lane == src) {
                const int sh = BITS * (e & 3);
                kf[e >> 2] = (kf[e >> 2] & ~(((1u << BITS) - 1u) << sh)) | (k << sh);
                near &= ~(1ull << e);
            }
        }

        // ---- indices, residuals, packing ----
        tq_half8 rh[kRT][4], rl[kRT][4];
        float rnorm[kRT];
#pragma unroll
        for (int rt = 0; rt < kRT; ++rt) {
            const int64_t row = row0 + 16 * rt + n;
            float rss = 0.f;
            uint32_t seg[8][BITS > 2 ? 2 : 1];
#pragma unroll
            for (int cb = 0; cb < 8; ++cb) {
                uint64_t f = 0;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float v = acc[rt][cb][r];
                    const uint32_t k = (kf[8 * rt + cb] >> (BITS * r)) & ((1u << BITS) - 1u);
                    f |= (uint64_t)k << (BITS * r);
                    if (PROJ) {
                        const float rs = v - s_cent[k];
                        rss = __builtin_fmaf(rs, rs, rss);
                        // B operand of the second product: slice cb / 2, position 8g + 4 (cb & 1) + r
                        const _Float16 h = (_Float16)rs;
                        rh[rt][cb >> 1][4 * (cb & 1) + r] = h;
                        rl[rt][cb >> 1][4 * (cb & 1) + r] = (_Float16)(rs - (float)h);
                    }
                }
                // this lane's 4 fields sit at bit 4 g BITS of the column block's 16-field segment
                f <<= 4 * g * BITS;
                seg[cb][0] = or_over_groups((uint32_t)f);
                if (BITS > 2) seg[cb][BITS > 2 ? 1 : 0] = or_over_groups((uint32_t)(f >> 32));
            }
            if (PROJ) rnorm[rt] = __builtin_sqrtf(sum_over_groups(rss)) * norm32[rt];
            if (row < p.n_rows) {
                // lane group g stores column blocks 2g and 2g + 1: 4 BITS bytes at byte 4 g BITS
                uint32_t w[BITS];
                uint64_t sg64[8];
#pragma unroll
                for (int cb = 0; cb < 8; ++cb)
                    sg64[cb] = BITS > 2 ? ((uint64_t)seg[cb][0] | ((uint64_t)seg[cb][BITS > 2 ? 1 : 0] << 32)) : seg[cb][0];
                const uint64_t s0 = pick_group(sg64, g, 0);
                const uint64_t s1 = pick_group(sg64, g, 1);
                // two 16 BITS-bit segments -> 32 BITS bits
                if (BITS == 1) {
                    w[0] = (uint32_t)(s0 & 0xffffu) | ((uint32_t)(s1 & 0xffffu) << 16);
                } else if (BITS == 2) {
                    w[0] = (uint32_t)s0;
                    w[BITS > 1 ? 1 : 0] = (uint32_t)s1;
                } else if (BITS == 3) {
                    // 48 + 48 bits
                    w[0] = (uint32_t)s0;
                    w[1 % BITS] = (uint32_t)(s0 >> 32) | (uint32_t)(s1 << 16);
                    w[2 % BITS] = (uint32_t)(s1 >> 16);
                } else {
                    w[0] = (uint32_t)s0;
                    w[1 % BITS] = (uint32_t)(s0 >> 32);
                    w[2 % BITS] = (uint32_t)s1;
                    w[3 % BITS] = (uint32_t)(s1 >> 32);
                }
                uint32_t* dst = reinterpret_cast<uint32_t*>(p.idx_out + row * (16 * BITS) + 4 * g * BITS);
#pragma unroll
                for (int j = 0; j < BITS; ++j) dst[j] = w[j];
                if (g == 0) p.norm_out[row] = (uint16_t)tq_f32_to_f16_bits(norm32[rt]);
            }
        }

        if (PROJ) {
            // ---- proj^T = PiST^T resid^T (resid without its factor norm > 0: same signs) ----
            tq_floatx4 pj[kRT][8];
#pragma unroll
            for (int rt = 0; rt < kRT; ++rt)
#pragma unroll
                for (int cb = 0; cb < 8; ++cb) pj[rt][cb] = tq_floatx4{0.f, 0.f, 0.f, 0.f};
            {
                tq_half8 ah[2], al[2];
                auto frag = [&](int step, tq_half8& h, tq_half8& l) {
                    const int o = (16 * (step & 7) + n) * kStride + 32 * (step >> 3) + 8 * g;
                    h = *reinterpret_cast<const tq_half8*>(s_m2h + o);
                    l = *reinterpret_cast<const tq_half8*>(s_m2l + o);
                };
                frag(0, ah[0], al[0]);
#pragma unroll
                for (int step = 0; step < 32; ++step) {
                    if (step + 1 < 32) frag(step + 1, ah[(step + 1) & 1], al[(step + 1) & 1]);
                    const int ks = step >> 3, cb = step & 7;
#pragma unroll
                    for (int rt = 0; rt < kRT; ++rt) {
                        pj[rt][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[step & 1], rh[rt][ks], pj[rt][cb], 0, 0, 0);
                        pj[rt][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[step & 1], rl[rt][ks], pj[rt][cb], 0, 0, 0);
                        pj[rt][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[step & 1], rh[rt][ks], pj[rt][cb], 0, 0, 0);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
#pragma unroll
            for (int rt = 0; rt < kRT; ++rt) {
                const int64_t row = row0 + 16 * rt + n;
                const bool zero = norm32[rt] == 0.f;  // resid = 0: every projection is 0 -> bit 1
                uint32_t seg[8];
#pragma unroll
                for (int cb = 0; cb < 8; ++cb) {
                    uint32_t f = 0;
#pragma unroll
                    for (int r = 0; r < 4; ++r) f |= ((__float_as_uint(pj[rt][cb][r]) >> 31) ^ 1u) << r;
                    f = zero ? 0xfu : f;
                    seg[cb] = or_over_groups(f << (4 * g));
                }
                if (row < p.n_rows) {
                    reinterpret_cast<uint32_t*>(p.signs_out + row * 16)[g] = pick_group(seg, g, 0) | (pick_group(seg, g, 1) << 16);
                    if (g == 0) p.rnorm_out[row] = (uint16_t)tq_f32_to_f16_bits(rnorm[rt]);
                }
            }
        }
    }
}

}  // namespace

size_t tq_packed_mfma_lds_bytes(bool proj) { return (size_t)(proj ? 4 : 2) * kD * kStride * sizeof(_Float16); }

int tq_packed_mfma_launch(const void* x, int x_dtype, int64_t x_stride, int64_t n_rows, const float* pit,
                          const float* pist, const float* centroids, const float* boundaries, int bits,
                          uint8_t* idx_out, uint8_t* signs_out, uint16_t* rnorm_out, uint16_t* norm_out,
                          hipStream_t st) {
    PackedParams p = {};
    p.x = x;
    p.x_dtype = x_dtype;
    p.x_stride = x_stride;
    p.n_rows = n_rows;
    const int64_t es = x_dtype == TQ_F32 ? 4 : 2;
    p.x_vec = ((reinterpret_cast<uintptr_t>(x) & 15) == 0 && (x_stride * es) % 16 == 0) ? 1 : 0;
    p.pit = pit;
    p.pist = pist;
    p.centroids = centroids;
    p.boundaries = boundaries;
    p.idx_out = idx_out;
    p.signs_out = signs_out;
    p.rnorm_out = rnorm_out;
    p.norm_out = norm_out;
    const bool proj = pist != nullptr;
    const void* kern = nullptr;
#define TQ_PK_DT(B, PJ, DT) kern = (const void*)packed_compress_mfma_kernel<B, PJ, DT>
#define TQ_PK(B, PJ)                                                \
    if (bits == B && proj == PJ) {                                  \
        if (x_dtype == TQ_BF16) TQ_PK_DT(B, PJ, TQ_BF16);           \
        else if (x_dtype == TQ_F16) TQ_PK_DT(B, PJ, TQ_F16);        \
        else TQ_PK_DT(B, PJ, TQ_F32);                               \
    }
    TQ_PK(1, false) TQ_PK(1, true) TQ_PK(2, false) TQ_PK(2, true)
    TQ_PK(3, false) TQ_PK(3, true) TQ_PK(4, false) TQ_PK(4, true)
#undef TQ_PK
#undef TQ_PK_DT
    if (!kern) return TQ_ERR_BITS;
    const size_t lds = tq_packed_mfma_lds_bytes(proj);
    int dev = 0, max_lds = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return (int)e;
    // the matrices (dynamic LDS) and the kernel's own arrays (static LDS) must fit
    hipFuncAttributes fa{};
    e = hipFuncGetAttributes(&fa, kern);
    if (e != hipSuccess) return (int)e;
    if ((size_t)max_lds < lds + fa.sharedSizeBytes) return TQ_ERR_WORKSPACE;
    {
        // the dynamic-LDS limit is a per-kernel attribute: set once per instance and device
        static std::mutex mu;
        static std::set<std::pair<const void*, int>> done;
        std::lock_guard<std::mutex> lk(mu);
        if (!done.count({kern, dev})) {
            e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return (int)e;
            done.insert({kern, dev});
        }
    }
    const int waves = proj ? packed_wg_waves<true>() : packed_wg_waves<false>();
    const int64_t groups = (n_rows + 16 * kRT - 1) / (16 * kRT);
    int64_t grid = (groups + waves - 1) / waves;
    const int64_t cap = (int64_t)cus * (proj ? 1 : 2);  // resident workgroups (LDS-limited)
    grid = grid < cap ? grid : cap;
    void* args[] = {&p};
    e = hipLaunchKernel(kern, dim3((unsigned)grid), dim3(waves * 64), args, lds, st);
    if (e != hipSuccess) return (int)e;
    e = hipGetLastError();
    return e == hipSuccess ? TQ_OK : (int)e;
}
