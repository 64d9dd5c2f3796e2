// Packed paged prefill / extend attention for gfx950: several query tokens per sequence over
// the packed K/V cache.  The tiled Sq > 1 path of kernels/attention.py:146-196 (_fused_general:
// one online softmax per query row over 16x128 key tiles, fp16 MFMA products with fp32
// accumulation), reading the packed paged cache directly instead of dequantised arrays, with
// the causal limit of a serving extend step (query i of a sequence of length L with n new
// tokens sits at position L - n + i and sees keys 0 .. L - n + i).
//
// Workgroup (256 threads, 4 waves) = (sequence s, KV head kh, block of 128 rows); a row is one
// (new token i, query head of the GQA group) pair, rows ordered token-major, so a workgroup
// serves 128 / G tokens with all G heads of the group and each K/V tile is dequantised once for
// all of them.  A wave owns two 16-row MFMA tiles: every LDS fragment it reads feeds two MFMAs.
// The cache is walked in steps of two 16-token tiles (a tile never spans two blocks).  Per step
// the 256 threads dequantise the next two tiles into the other of two LDS buffers (each two tile
// sub-buffers; 8 dims of one token per thread, for the keys and for the values; mappings in the
// kernel) while the waves compute on this step's:
//   Khat [16 tok][128] fp16 = c[idx] * cscale       row stride 272 B (16 B pad: no bank clash)
//   Shat [16 tok][128] fp16 = +-1                    QJL keys only (sign byte -> LDS table)
//   VhatT [128 dim][16 tok] fp16 = c[vidx] * cscale  transposed: the PV A operand; row stride
//                                                    40 B, so the 4 dim rows a wave writes at
//                                                    once start 16 banks apart
//   kn1, kr2, vn [16] f32 = norm * c1, rnorm * c2, vnorm (c1, c2 below)
// Each wave computes for each of its two 16-row tiles (MFMA layout: lane l, n = l % 16, g = l / 16):
//   S^T [16 tok x 16 rows] = Khat . Q^T     4 x mfma_f32_16x16x32_f16 per tile (B: q row n in registers)
//   T^T = Shat . QP^T                        4 x mfma_f32_16x16x32_f16 per tile (QJL keys)
//   lane (n, g) holds tokens 4g + r of row n in each tile: s = kn1 * S + kr2 * T (log2 units),
//   masked; online softmax per row (column) over the step's 32 keys, the maxima and sums reduced
//   over the lane groups once per step; fp16(p * vnorm) of tokens 4g..4g+3 of both tiles is
//   exactly the B operand (k = 8g + i: tile A token 4g + i, i < 4, tile B token 4g + i - 4) of
//   O^T [128 x 16 rows] += VhatT . P^T        8 x mfma_f32_16x16x32_f16 per step
// Output: lane (n, g) holds dims 16j + 4g + r of row n, divided by the row's denominator.
#include "tq_common.h"

#include <cmath>

namespace {

constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kWhtH = 0.08838834764831845f;  // 1 / sqrt(128)

constexpr int kRT = 2;                           // 16-row MFMA tiles per wave
constexpr int kRowsPerWG = 64 * kRT;
constexpr int kKRow = 272;                       // bytes per token row of Khat / Shat
constexpr int kOffS = 16 * kKRow;                // Shat
constexpr int kVRow = 40;                        // bytes per dim row of VhatT (16 tokens + pad)
constexpr int kOffV = 2 * 16 * kKRow;            // VhatT: 128 rows
constexpr int kOffN = kOffV + 128 * kVRow;       // kn1[16], kr2[16], vn[16]
constexpr int kBuf = kOffN + 3 * 16 * 4;         // one tile buffer
constexpr int kOffTab = 4 * kBuf;                // pair tables: K then V, 256 x 4 bytes each
constexpr int kOffSgn = kOffTab + 2 * 1024;      // sign table: byte b -> 8 fp16 +-1 (16 bytes)
constexpr int kLdsBytes = kOffSgn + 256 * 16;

struct PrefillParams {
    const void* q;
    int64_t q_st, q_sh;
    const void* qp;
    int64_t qp_st, qp_sh;
    int q_dtype, q_vec;
    const int32_t* cu_q;
    int num_seqs, hq, hkv, group, n_rb;
    tq_region kidx, ksig, knorm, krnorm, vidx, vnorm;
    const float* k_cent;
    const float* v_cent;
    int k_lg, v_lg;  // lane-grouped key / value tiles (TQ_TILE_KEYS / TQ_TILE_VALUES)
    float k_cs, v_cs, v_cinv;
    int block_size;
    int64_t num_blocks;
    const int32_t* bt;
    int64_t bt_stride;
    int max_blocks;
    const int32_t* seq_lens;
    float c1;   // sm_scale * log2(e) / k_cs: MSE term in log2 units
    float c2;   // sm_scale * log2(e) * corr_scale: QJL term in log2 units
    int causal;
    int rot_q, rot_qp, rot_out;
    void* out;
    int out_dtype;
    int64_t out_st, out_sh;
};

typedef _Float16 tq_half4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float max_over_groups(float x) {
    auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float y = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum_over_groups(float x) {
    auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Raw packed data one thread dequantises for a tile.
struct Raw {
    uint32_t kw[2], vw[2];   // dwords holding the 8 index fields (funnel-shifted by the byte offset)
    uint32_t sg0;            // sign bits (QJL keys): the dword holding byte pk of the sign row
    uint32_t nrm;            // fp16 norm bits (threads 0-47: K norm, K residual norm, V norm)
    int nv;                  // usable rows of the tile (0: unreadable block)
};

template <int KB, bool KQJL, int VB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_kernel(PrefillParams p) {
    extern __shared__ __attribute__((aligned(16))) uint8_t s_lds[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int n = lane & 15;
    const int g = lane >> 4;

    // row blocks of one (sequence, KV head) in decreasing order: under a causal mask the last
    // rows see the most keys, and dispatching the longest workgroups first leaves short ones
    // for the end of the launch
    const int rb = p.n_rb - 1 - (int)(blockIdx.x % (unsigned)p.n_rb);
    const int skh = (int)(blockIdx.x / (unsigned)p.n_rb);
    const int kh = skh % p.hkv;
    const int s = skh / p.hkv;
    const int q0 = p.cu_q[s];
    const int nq = p.cu_q[s + 1] - q0;
    const int G = p.group;
    if (nq <= 0 || rb * kRowsPerWG >= nq * G) return;  // block-uniform
    int L = p.seq_lens[s];
    const int cap = p.max_blocks * p.block_size;
    L = L < cap ? L : cap;
    L = L > 0 ? L : 0;

    // ---- pair tables: entry e -> half2(c[e & m], c[e >> b]) * cscale ----
    {
        uint32_t* tk = reinterpret_cast<uint32_t*>(s_lds + kOffTab);
        uint32_t* tv = tk + 256;
        if (tid < (1 << (2 * KB)))
            tk[tid] = tq_pack_half2(p.k_cent[tid & ((1 << KB) - 1)] * p.k_cs, p.k_cent[tid >> KB] * p.k_cs);
        if (tid < (1 << (2 * VB)))
            tv[tid] = tq_pack_half2(p.v_cent[tid & ((1 << VB) - 1)] * p.v_cs, p.v_cent[tid >> VB] * p.v_cs);
        if (KQJL) {
            // sign byte b -> halves j = 0..7: bit j set -> +1 (0x3c00), clear -> -1 (0xbc00)
            tq_u32x4 h;
#pragma unroll
            for (int k = 0; k < 4; ++k)
                h[k] = (((tid >> (2 * k)) & 1) ? 0x3c00u : 0xbc00u) | ((((tid >> (2 * k + 1)) & 1) ? 0x3c00u : 0xbc00u) << 16);
            reinterpret_cast<tq_u32x4*>(s_lds + kOffSgn)[tid] = h;
        }
    }

    // ---- this lane's rows: (token i, head gh) of MFMA tile rt, rows 32 wave + 16 rt + n ----
    int iR[kRT], headR[kRT], qposR[kRT];
    bool rvalid[kRT];
#pragma unroll
    for (int rt = 0; rt < kRT; ++rt) {
        const int R = rb * kRowsPerWG + wave * 16 * kRT + 16 * rt + n;
        const int i = R / G;
        const int gh = R - i * G;
        iR[rt] = i;
        rvalid[rt] = i < nq;
        headR[rt] = kh * G + gh;
        qposR[rt] = p.causal ? L - nq + i : L - 1;  // last key position the row sees
    }
    // last key position any row of the workgroup sees (rows are token-major)
    int imax = (rb * kRowsPerWG + kRowsPerWG - 1) / G;
    imax = imax < nq - 1 ? imax : nq - 1;
    int t_end = p.causal ? L - nq + imax + 1 : L;
    t_end = t_end < L ? t_end : L;
    t_end = t_end > 0 ? t_end : 0;
    const int ntiles = (t_end + 15) >> 4;

    // ---- query operands (B of the score products): dims 32cc + 8g + j of row n of tile rt ----
    tq_half8 qop[kRT][4], qpop[kRT][4];
#pragma unroll
    for (int rt = 0; rt < kRT; ++rt) {
        const int i = iR[rt], head = headR[rt];
        const bool rv = rvalid[rt];
        float x[32];
        const int64_t off = (int64_t)(q0 + (rv ? i : 0)) * p.q_st + (int64_t)head * p.q_sh + 8 * g;
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            if (rv && p.q_vec) {
                tq_load8(p.q, off + 32 * cc, p.q_dtype, &x[8 * cc]);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) x[8 * cc + j] = rv ? tq_load1(p.q, off + 32 * cc + j, p.q_dtype) : 0.f;
            }
        }
        // x[8cc + j] is element 32cc + 8g + j: register bits = element bits 0-2 and 5-6
        if (p.rot_q) tq_wht_row_g4(x, kWhtH);
#pragma unroll
        for (int cc = 0; cc < 4; ++cc)
#pragma unroll
            for (int j = 0; j < 8; ++j) qop[rt][cc][j] = (_Float16)x[8 * cc + j];
        if (KQJL) {
            const int64_t offp = (int64_t)(q0 + (rv ? i : 0)) * p.qp_st + (int64_t)head * p.qp_sh + 8 * g;
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                if (rv && p.q_vec) {
                    tq_load8(p.qp, offp + 32 * cc, p.q_dtype, &x[8 * cc]);
                } else {
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        x[8 * cc + j] = rv ? tq_load1(p.qp, offp + 32 * cc + j, p.q_dtype) : 0.f;
                }
            }
            if (p.rot_qp) tq_wht_row_g4(x, kWhtH);
#pragma unroll
            for (int cc = 0; cc < 4; ++cc)
#pragma unroll
                for (int j = 0; j < 8; ++j) qpop[rt][cc][j] = (_Float16)x[8 * cc + j];
        } else {
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) qpop[rt][cc] = tq_half8{};
        }
    }

    // ---- dequantisation of tile ti by this thread: keys and signs of token tk, dims 8pk..8pk+7,
    // values of token tt, dims 8pp..8pp+7.  Keys: each wave takes 4 whole rows (4w..4w+3), so a
    // wave's key loads cover consecutive bytes; values: each wave takes dims 32w..32w+31 of all
    // 16 rows, so its transposed LDS writes hit 4 dim rows 16 banks apart.
    const int tk = 4 * (tid >> 6) + ((tid >> 4) & 3);
    const int pk = tid & 15;
    const int tt = tid & 15;
    const int pp = tid >> 4;
    const int32_t* bt_row = p.bt + (int64_t)s * p.bt_stride;
    // block of tile ti (wave-uniform) and whether it is readable
    auto tile_block = [&](int ti, int& nv) -> int64_t {
        const int t0 = ti * 16;
        int blk = bt_row[t0 / p.block_size];
        nv = L - t0;
        nv = nv < 16 ? nv : 16;
        if (blk < 0 || (int64_t)blk >= p.num_blocks) {
            blk = 0;
            nv = 0;
        }
        return blk;
    };
    // Loop-invariant byte offsets of this thread's data inside a 16-row tile (rows are less than
    // 2^31 / 16 bytes apart: checked on the host), added to the tile's wave-uniform base address.
    // Byte offsets of the thread's index fields (K, V) and of its sign dword in a 16-row
    // sub-tile, for the row-major and the lane-grouped tile layouts.
    uint32_t ok, ov, o_sg;
    if (p.k_lg) {
        const int c = 4 * tk + (pk >> 2);  // chunk: row tk, dim quarter pk / 4
        constexpr int C = 4 * KB + (KQJL ? 4 : 0);
        ok = (uint32_t)(c * C + (pk & 3) * KB);
        o_sg = (uint32_t)(c * C + 4 * KB);  // byte pk & 3 of it: dims 8pk..8pk+7
    } else {
        ok = (uint32_t)(tk * p.kidx.stride_row + KB * pk);
        o_sg = (uint32_t)(tk * p.ksig.stride_row) + 4u * (uint32_t)(pk >> 2);
    }
    if (p.v_lg) {
        // chunk (tt / 4, pp), byte VB (tt & 3): dims 8pp + 2 (tt & 3) and the next, rows 4 (tt / 4)..
        ov = (uint32_t)((16 * (tt >> 2) + pp) * 4 * VB + (tt & 3) * VB);
    } else {
        ov = (uint32_t)(tt * p.vidx.stride_row + VB * pp);
    }
    // the aligned dword holding the first field and the next one; in a row-major row the next
    // one is clamped to the row (a field ending in the row's last dword lies entirely in it), in
    // a lane-grouped tile it is always inside the tile (chunks or the norm region follow)
    auto second = [](uint32_t o, bool lg, uint32_t row_start, int row_dwords) -> uint32_t {
        const uint32_t w0 = o & ~3u;
        if (lg) return w0 + 4u;
        return (w0 + 4u < row_start + 4u * (uint32_t)row_dwords) ? w0 + 4u : w0;
    };
    const uint32_t o_k0 = ok & ~3u, o_k1 = second(ok, p.k_lg, (uint32_t)(tk * p.kidx.stride_row), 4 * KB);
    const uint32_t o_v0 = ov & ~3u, o_v1 = second(ov, p.v_lg, (uint32_t)(tt * p.vidx.stride_row), 4 * VB);
    const uint32_t sh_k = (ok & 3u) * 8u, sh_v = (ov & 3u) * 8u;
    const int ntok = tid & 15;  // token of the norm threads (0-47)
    // (the row strides are selected as values: a per-thread reference into the parameters would
    // make every tile read the region fields with vector loads)
    const int64_t nm_stride = tid < 16 ? p.knorm.stride_row : (tid < 32 ? p.krnorm.stride_row : p.vnorm.stride_row);
    const uint32_t o_nm = (uint32_t)(ntok * nm_stride);
    auto load_raw = [&](int ti, Raw& w) {
        const int64_t blk = tile_block(ti, w.nv);
        const int row0 = (ti * 16) % p.block_size;
        auto base = [&](const tq_region& rg) -> const uint8_t* {  // wave-uniform
            return static_cast<const uint8_t*>(rg.ptr) + blk * rg.stride_block + (int64_t)kh * rg.stride_head +
                   (int64_t)row0 * rg.stride_row;
        };
        auto ld32 = [](const uint8_t* b, uint32_t o) { return *reinterpret_cast<const uint32_t*>(b + (uint64_t)o); };
        const uint8_t* bk = base(p.kidx);
        w.kw[0] = ld32(bk, o_k0);
        w.kw[1] = ld32(bk, o_k1);
        const uint8_t* bv = base(p.vidx);
        w.vw[0] = ld32(bv, o_v0);
        w.vw[1] = ld32(bv, o_v1);
        if (KQJL) {
            w.sg0 = ld32(base(p.ksig), o_sg);
        }
        w.nrm = 0;
        if (tid < 48 && (KQJL || tid < 16 || tid >= 32)) {
            // wave-uniform bases of the three norm regions, one picked per thread
            const uint8_t* nk = base(p.knorm);
            const uint8_t* nr = KQJL ? base(p.krnorm) : nk;
            const uint8_t* nvb = base(p.vnorm);
            const uint8_t* nb = tid < 16 ? nk : (tid < 32 ? nr : nvb);
            w.nrm = *reinterpret_cast<const uint16_t*>(nb + (uint64_t)o_nm);
        }
    };
    auto store_tile = [&](int ti, const Raw& w, int buf) {
        const int nv = w.nv;
        uint8_t* b = s_lds + buf * kBuf;
        const uint8_t* tab = s_lds + kOffTab;
        {
            const uint32_t f = __builtin_amdgcn_alignbit(w.kw[1], w.kw[0], sh_k);
            tq_u32x4 h;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t e = (f >> (2 * KB * k)) & ((1u << (2 * KB)) - 1u);
                h[k] = *reinterpret_cast<const uint32_t*>(tab + 4 * e);
            }
            *reinterpret_cast<tq_u32x4*>(b + tk * kKRow + 16 * pk) = h;
        }
        if (KQJL) {
            // sign of dim 8pk + j: bit j of byte pk & 3 of the dword (natural bit order); the
            // byte's 8 fp16 +-1 come from the sign table
            const uint32_t bitsj = (w.sg0 >> (8 * (pk & 3))) & 0xffu;
            const tq_u32x4 h = *reinterpret_cast<const tq_u32x4*>(s_lds + kOffSgn + 16 * bitsj);
            *reinterpret_cast<tq_u32x4*>(b + kOffS + tk * kKRow + 16 * pk) = h;
        }
        {
            const uint32_t f = __builtin_amdgcn_alignbit(w.vw[1], w.vw[0], sh_v);
            const uint8_t* tv = tab + 1024;
            if (p.v_lg) {
                // values tile layout: the 8 VB bits at byte VB r of chunk (g, pp) (r = tt & 3) are
                // dims 8pp + 2r + jj (jj = 0, 1), four tokens 4g.. each: pairs of tokens go to
                // VhatT as half2 words
                const int g4 = tt & ~3, d0 = 8 * pp + 2 * (tt & 3);
#pragma unroll
                for (int jj = 0; jj < 2; ++jj)
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const uint32_t e = (f >> (4 * VB * jj + 2 * VB * h)) & ((1u << (2 * VB)) - 1u);
                        *reinterpret_cast<uint32_t*>(b + kOffV + (d0 + jj) * kVRow + 2 * (g4 + 2 * h)) =
                            *reinterpret_cast<const uint32_t*>(tv + 4 * e);
                    }
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t e = (f >> (2 * VB * k)) & ((1u << (2 * VB)) - 1u);
                    const uint32_t h2 = *reinterpret_cast<const uint32_t*>(tv + 4 * e);
                    const int d = 8 * pp + 2 * k;
                    *reinterpret_cast<uint16_t*>(b + kOffV + d * kVRow + 2 * tt) = (uint16_t)h2;
                    *reinterpret_cast<uint16_t*>(b + kOffV + (d + 1) * kVRow + 2 * tt) = (uint16_t)(h2 >> 16);
                }
            }
        }
        if (tid < 48) {
            // norms of unusable tokens are zeroed bit-wise (their bits may be anything)
            const int tok = tid & 15;
            const float x = tok < nv ? tq_f16_to_f32(w.nrm) : 0.f;
            const float scale = tid < 16 ? p.c1 : (tid < 32 ? p.c2 : 1.f);
            reinterpret_cast<float*>(b + kOffN)[tid] = x * scale;
        }
    };

    __syncthreads();  // pair tables
    // Steps of 32 keys (tiles 2j, 2j + 1, in the two sub-buffers of buffer j & 1).  The raw data
    // of the next step's two tiles is requested at the start of a step and dequantised into the
    // other buffer at its end.  A tile past the last is staged as an empty one (no loads; zero
    // norms, finite table values), so a step's second tile never holds stale bits.
    Raw rawA, rawB;
    auto load_or_empty = [&](int ti, Raw& w) {
        if (ti < ntiles) {
            load_raw(ti, w);
        } else {
            w.kw[0] = w.kw[1] = w.vw[0] = w.vw[1] = 0u;
            w.sg0 = 0u;
            w.nrm = 0u;
            w.nv = 0;
        }
    };
    const int nsteps = (ntiles + 1) >> 1;
    int nvA = 0, nvB = 0;  // usable rows of the current step's tiles
    if (nsteps > 0) {
        load_or_empty(0, rawA);
        load_or_empty(1, rawB);
        store_tile(0, rawA, 0);
        store_tile(1, rawB, 1);
        nvA = rawA.nv;
        nvB = rawB.nv;
    }
    __syncthreads();

    float m[kRT], lsum[kRT];
    tq_floatx4 acc[kRT][8];
#pragma unroll
    for (int rt = 0; rt < kRT; ++rt) {
        m[rt] = kNegInf;
        lsum[rt] = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[rt][j] = tq_floatx4{0.f, 0.f, 0.f, 0.f};
    }

    for (int js = 0; js < nsteps; ++js) {
        const int cur = 2 * (js & 1);
        const bool more = js + 1 < nsteps;
        if (more) {
            load_or_empty(2 * js + 2, rawA);
            load_or_empty(2 * js + 3, rawB);
        }
        const uint8_t* bA = s_lds + cur * kBuf;
        const uint8_t* bB = bA + kBuf;
        // scores^T of both tiles: tokens 4g + r of row n, tile A then tile B
        float sv[kRT][8];
#pragma unroll
        for (int tt2 = 0; tt2 < 2; ++tt2) {
            const uint8_t* b = tt2 ? bB : bA;
            tq_floatx4 sc[kRT], tj[kRT];
#pragma unroll
            for (int rt = 0; rt < kRT; ++rt) {
                sc[rt] = tq_floatx4{0.f, 0.f, 0.f, 0.f};
                tj[rt] = tq_floatx4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                const tq_half8 a = *reinterpret_cast<const tq_half8*>(b + n * kKRow + 2 * (32 * cc + 8 * g));
#pragma unroll
                for (int rt = 0; rt < kRT; ++rt)
                    sc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qop[rt][cc], sc[rt], 0, 0, 0);
            }
            if (KQJL) {
#pragma unroll
                for (int cc = 0; cc < 4; ++cc) {
                    const tq_half8 a =
                        *reinterpret_cast<const tq_half8*>(b + kOffS + n * kKRow + 2 * (32 * cc + 8 * g));
#pragma unroll
                    for (int rt = 0; rt < kRT; ++rt)
                        tj[rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qpop[rt][cc], tj[rt], 0, 0, 0);
                }
            }
            const tq_floatx4 kn1 = *reinterpret_cast<const tq_floatx4*>(b + kOffN + 16 * g);
            const tq_floatx4 kr2 = *reinterpret_cast<const tq_floatx4*>(b + kOffN + 64 + 16 * g);
            const int nvt = tt2 ? nvB : nvA;
#pragma unroll
            for (int rt = 0; rt < kRT; ++rt) {
                // tokens 4g + r below lim are usable and visible to the row (one compare per
                // token, in the tiles where some lane has one that is not: the diagonal and the
                // last tiles)
                int lim = qposR[rt] - (2 * js + tt2) * 16 + 1 - 4 * g;
                lim = lim < nvt - 4 * g ? lim : nvt - 4 * g;
#pragma unroll
                for (int r = 0; r < 4; ++r) sv[rt][4 * tt2 + r] = __builtin_fmaf(kn1[r], sc[rt][r], kr2[r] * tj[rt][r]);
                if (__builtin_amdgcn_ballot_w64(lim < 4)) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) sv[rt][4 * tt2 + r] = r < lim ? sv[rt][4 * tt2 + r] : kNegInf;
                }
            }
        }
        const tq_floatx4 vnA = *reinterpret_cast<const tq_floatx4*>(bA + kOffN + 128 + 16 * g);
        const tq_floatx4 vnB = *reinterpret_cast<const tq_floatx4*>(bB + kOffN + 128 + 16 * g);
        tq_half8 bop[kRT];
#pragma unroll
        for (int rt = 0; rt < kRT; ++rt) {
            float mt = fmaxf(fmaxf(fmaxf(sv[rt][0], sv[rt][1]), fmaxf(sv[rt][2], sv[rt][3])),
                             fmaxf(fmaxf(sv[rt][4], sv[rt][5]), fmaxf(sv[rt][6], sv[rt][7])));
            mt = max_over_groups(mt);
            // The exponent base m (per row) moves only when some row's max passes it by more
            // than one log2 unit; p = exp2(s - m - 1) <= 1, and acc and lsum carry the same
            // factor, so most steps skip the rescale.
            if (__builtin_amdgcn_ballot_w64(mt > m[rt] + 1.0f)) {
                const float mb = fmaxf(m[rt], mt);
                // 0 while m = -inf; 1 for a row whose max did not move (also a row that has seen
                // no visible token yet: -inf - -inf would be NaN)
                const float alpha = mb == m[rt] ? 1.0f : __builtin_amdgcn_exp2f(m[rt] - mb);
                lsum[rt] *= alpha;
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[rt][j] *= alpha;
                m[rt] = mb;
            }
            const float nb = m[rt] == kNegInf ? 0.f : -m[rt] - 1.0f;
            float pr[8];
#pragma unroll
            for (int r = 0; r < 8; ++r) pr[r] = __builtin_amdgcn_exp2f(sv[rt][r] + nb);  // 0 for masked tokens
            lsum[rt] += ((pr[0] + pr[1]) + (pr[2] + pr[3])) + ((pr[4] + pr[5]) + (pr[6] + pr[7]));
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                bop[rt][r] = (_Float16)(pr[r] * vnA[r]);
                bop[rt][4 + r] = (_Float16)(pr[4 + r] * vnB[r]);
            }
        }
        // O^T += VhatT . P^T over the step's 32 keys: k = 8g + i is token 4g + i of tile A
        // (i < 4) or of tile B (i >= 4), the order of the B operand above
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const tq_half4v va = *reinterpret_cast<const tq_half4v*>(bA + kOffV + (16 * j + n) * kVRow + 8 * g);
            const tq_half4v vb = *reinterpret_cast<const tq_half4v*>(bB + kOffV + (16 * j + n) * kVRow + 8 * g);
            const tq_half8 a = {va[0], va[1], va[2], va[3], vb[0], vb[1], vb[2], vb[3]};
#pragma unroll
            for (int rt = 0; rt < kRT; ++rt)
                acc[rt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bop[rt], acc[rt][j], 0, 0, 0);
        }
        if (more) {
            store_tile(2 * js + 2, rawA, 2 - cur);
            store_tile(2 * js + 3, rawB, 3 - cur);
            nvA = rawA.nv;
            nvB = rawB.nv;
        }
        __syncthreads();
    }

    // ---- normalise, rotate, write ----
#pragma unroll
    for (int rt = 0; rt < kRT; ++rt) {
        const float l = sum_over_groups(lsum[rt]);
        const float inv = l > 0.f ? p.v_cinv / l : 0.f;
        float o[32];
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[4 * j + r] = acc[rt][j][r] * inv;
        // o[4j + r] is dim 16j + 4g + r: register bits = dim bits 0-1 and 4-6
        if (p.rot_out) tq_wht_row_g4(o, kWhtH);
        if (rvalid[rt]) {
            const int64_t ob = (int64_t)(q0 + iR[rt]) * p.out_st + (int64_t)headR[rt] * p.out_sh + 4 * g;
#pragma unroll
            for (int j = 0; j < 8; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) tq_store1(p.out, ob + 16 * j + r, p.out_dtype, o[4 * j + r]);
        }
    }
}

const void* prefill_kernel_ptr(int kb, bool kq, int vb) {
#define TQ_PF(KB, KQ, VB) \
    if (kb == KB && kq == KQ && vb == VB) return (const void*)prefill_kernel<KB, KQ, VB>;
#define TQ_PF_V(KB, KQ) TQ_PF(KB, KQ, 2) TQ_PF(KB, KQ, 3) TQ_PF(KB, KQ, 4)
    TQ_PF_V(2, false) TQ_PF_V(2, true) TQ_PF_V(3, false) TQ_PF_V(3, true) TQ_PF_V(4, false) TQ_PF_V(4, true)
#undef TQ_PF_V
#undef TQ_PF
    return nullptr;
}

bool aligned(const void* ptr, uintptr_t a) { return (reinterpret_cast<uintptr_t>(ptr) & (a - 1)) == 0; }

int check_region(const tq_region& r, int align) {
    if (!r.ptr) return TQ_ERR_INVALID_ARGUMENT;
    if (!aligned(r.ptr, align) || r.stride_block % align || r.stride_head % align || r.stride_row % align)
        return TQ_ERR_INVALID_ARGUMENT;
    return TQ_OK;
}

bool q_vector_ok(const void* q, int dtype, int64_t st, int64_t sh) {
    const uintptr_t a = dtype == TQ_F32 ? 32 : 16;
    return aligned(q, a) && st % 8 == 0 && sh % 8 == 0;
}

}  // namespace

extern "C" int tq_prefill(const void* q, int q_dtype, int64_t q_stride_token, int64_t q_stride_head,
                          const void* q_proj, int64_t qp_stride_token, int64_t qp_stride_head,
                          const int32_t* cu_seqlens_q, int num_seqs, int max_q_len,
                          int num_q_heads, int num_kv_heads, int head_dim,
                          const tq_kv_view* k, const tq_kv_view* v,
                          int block_size, int64_t num_blocks,
                          const int32_t* block_tables, int64_t block_table_stride, int max_blocks_per_seq,
                          const int32_t* seq_lens, float sm_scale, float corr_scale, int flags,
                          void* out, int out_dtype, int64_t out_stride_token, int64_t out_stride_head,
                          tq_stream_t stream) {
    if (head_dim != TQ_HEAD_DIM) return TQ_ERR_HEAD_DIM;
    if (!k || !v) return TQ_ERR_INVALID_ARGUMENT;
    if (num_seqs < 0 || max_q_len < 0 || num_q_heads <= 0 || num_kv_heads <= 0) return TQ_ERR_INVALID_ARGUMENT;
    if (num_q_heads % num_kv_heads) return TQ_ERR_GQA;
    if (k->bits < 2 || k->bits > 4 || v->bits < 2 || v->bits > 4) return TQ_ERR_BITS;
    if (v->qjl) return TQ_ERR_INVALID_ARGUMENT;
    if (block_size <= 0 || block_size % 16) return TQ_ERR_BLOCK_SIZE;
    if (q_dtype != TQ_F32 && q_dtype != TQ_F16 && q_dtype != TQ_BF16) return TQ_ERR_DTYPE;
    if (out_dtype != TQ_F32 && out_dtype != TQ_F16 && out_dtype != TQ_BF16) return TQ_ERR_DTYPE;
    if (flags & ~(TQ_PREFILL_CAUSAL | TQ_PREFILL_ROTATE)) return TQ_ERR_INVALID_ARGUMENT;
    if (k->qjl && k->signs_permuted) return TQ_ERR_INVALID_ARGUMENT;  // paged caches: natural sign order
    if (max_blocks_per_seq < 0 || num_blocks < 1) return TQ_ERR_INVALID_ARGUMENT;  // unreadable entries read block 0
    if (num_seqs == 0 || max_q_len == 0) return TQ_OK;
    if (!q || !cu_seqlens_q || !seq_lens || !block_tables || !out || !k->centroids || !v->centroids)
        return TQ_ERR_INVALID_ARGUMENT;
    if (block_table_stride < max_blocks_per_seq) return TQ_ERR_INVALID_ARGUMENT;
    const bool k_lg = k->layout == TQ_TILE_KEYS, v_lg = v->layout == TQ_TILE_VALUES;
    if ((k->layout != TQ_TILE_ROWS && !k_lg) || (v->layout != TQ_TILE_ROWS && !v_lg)) return TQ_ERR_INVALID_ARGUMENT;
    if (k_lg && k->idx.stride_row != 16 * k->bits + (k->qjl ? 16 : 0))
        return TQ_ERR_INVALID_ARGUMENT;
    if (v_lg && v->idx.stride_row != 16 * v->bits) return TQ_ERR_INVALID_ARGUMENT;
    int rc;
    if ((rc = check_region(k->idx, 4))) return rc;
    if ((rc = check_region(k->norm, 2))) return rc;
    if ((rc = check_region(v->idx, 4))) return rc;
    if ((rc = check_region(v->norm, 2))) return rc;
    if (k->qjl) {
        if (!k_lg && (rc = check_region(k->signs, 4))) return rc;
        if ((rc = check_region(k->rnorm, 2))) return rc;
    }
    // per-thread offsets inside a tile are 32-bit: 16 rows of any region below 2^31 bytes
    const tq_region* regs[6] = {&k->idx, &k->norm, &v->idx, &v->norm, &k->rnorm, k_lg ? &k->idx : &k->signs};
    for (int r = 0; r < (k->qjl ? 6 : 4); ++r)
        if (regs[r]->stride_row < 0 || regs[r]->stride_row >= (1ll << 26)) return TQ_ERR_INVALID_ARGUMENT;
    const int group = num_q_heads / num_kv_heads;
    const int64_t rows = (int64_t)max_q_len * group;
    const int64_t n_rb = (rows + kRowsPerWG - 1) / kRowsPerWG;
    const int64_t grid = n_rb * num_seqs * num_kv_heads;
    if (grid > 0x7fffffff) return TQ_ERR_INVALID_ARGUMENT;

    PrefillParams p = {};
    p.q = q;
    p.q_st = q_stride_token;
    p.q_sh = q_stride_head;
    p.qp = q_proj ? q_proj : q;
    p.qp_st = q_proj ? qp_stride_token : q_stride_token;
    p.qp_sh = q_proj ? qp_stride_head : q_stride_head;
    p.q_dtype = q_dtype;
    p.q_vec = q_vector_ok(p.q, q_dtype, p.q_st, p.q_sh) && q_vector_ok(p.qp, q_dtype, p.qp_st, p.qp_sh);
    p.cu_q = cu_seqlens_q;
    p.num_seqs = num_seqs;
    p.hq = num_q_heads;
    p.hkv = num_kv_heads;
    p.group = group;
    p.n_rb = (int)n_rb;
    p.kidx = k->idx;
    p.ksig = (k->qjl && !k_lg) ? k->signs : k->idx;
    p.knorm = k->norm;
    p.krnorm = k->qjl ? k->rnorm : k->norm;
    p.vidx = v->idx;
    p.vnorm = v->norm;
    p.k_cent = k->centroids;
    p.v_cent = v->centroids;
    p.k_lg = k_lg ? 1 : 0;
    p.v_lg = v_lg ? 1 : 0;
    p.k_cs = k->centroid_scale > 0.f ? k->centroid_scale : 1.f;
    p.v_cs = v->centroid_scale > 0.f ? v->centroid_scale : 1.f;
    p.v_cinv = 1.f / p.v_cs;
    p.block_size = block_size;
    p.num_blocks = num_blocks;
    p.bt = block_tables;
    p.bt_stride = block_table_stride;
    p.max_blocks = max_blocks_per_seq;
    p.seq_lens = seq_lens;
    p.c1 = sm_scale * kLog2e / p.k_cs;
    p.c2 = sm_scale * kLog2e * corr_scale;
    p.causal = (flags & TQ_PREFILL_CAUSAL) ? 1 : 0;
    const int rot = (flags & TQ_PREFILL_ROTATE) ? 1 : 0;
    p.rot_q = rot;
    p.rot_qp = rot && !q_proj;
    p.rot_out = rot;
    p.out = out;
    p.out_dtype = out_dtype;
    p.out_st = out_stride_token;
    p.out_sh = out_stride_head;
    const void* kern = prefill_kernel_ptr(k->bits, k->qjl != 0, v->bits);
    if (!kern) return TQ_ERR_BITS;
    void* args[] = {&p};
    hipError_t le = hipLaunchKernel(kern, dim3((unsigned)grid), dim3(256), args, kLdsBytes, (hipStream_t)stream);
    if (le != hipSuccess) return (int)le;
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TQ_OK : (int)e;
}
