// Packed asymmetric split-K decode attention for gfx950.
//
// Work unit = one wave64 = (sequence, KV head, chunk of tokens_per_chunk tokens), walked in
// tiles of 16 tokens.  A 256-thread workgroup holds 4 units and shares two LDS lookup tables
// that turn a pair of packed indices (2*bits bits) into a half2 of centroids; each table is
// replicated 32x across LDS banks so lanes 0-31 never conflict.
//
// Per tile (all MFMA accumulation in fp32):
//   S^T[token][head]  = K_dq[16 x 128] . Q^T[128 x 16]      4 x mfma_f32_16x16x32_f16
//   QJL^T[token][head]= (+-1)[16 x 128] . (-QP)^T            4 x mfma_f32_16x16x32_f16
//   score = norm * S + corr_scale * rnorm * QJL   (log2 domain: Q pre-scaled by sm_scale*log2 e)
//   online softmax per head; Sparse-V mask from a ballot over the GQA group
//   acc^T[dim][head] += V_dq^T[128 x 16] . (p * vnorm)[16 x 16]  8 x mfma_f32_16x16x16f16
// MFMA output layout (16x16): lane l holds rows 4*(l/16)+r, column l%16, so after the QK
// product lane (head n = l%16, g = l/16) owns tokens 4g..4g+3 of head n, which is exactly the
// B-operand layout of the PV product: no data movement between the two products.
// Each unit writes (m, l, acc[128]) per head; tq_decode_reduce combines chunks:
//   out = sum_c 2^(m_c - M) acc_c / sum_c 2^(m_c - M) l_c      (kernels/attention.py:121-140)
#include "tq_common.h"

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

struct Region {
    const uint8_t* ptr;
    int64_t stride_block, stride_head, stride_seq, stride_row;
};

struct DecodeParams {
    const void* q;
    int64_t q_ss, q_sh;
    const void* qp;
    int64_t qp_ss, qp_sh;
    int q_dtype;
    int num_seqs, hq, hkv, group;
    Region k_idx, k_sig, k_norm, k_rnorm;
    Region v_idx, v_norm;
    const float* k_cent;
    const float* v_cent;
    float k_cscale, v_cscale;  // tables hold fp16(c * cscale) ...
    float k_cinv, v_cinv;      // ... and norms carry 1 / cscale
    int k_perm;
    int block_size;
    int64_t num_blocks;
    const int32_t* bt;
    int64_t bt_stride;
    int max_blocks;
    const int32_t* seq_lens;
    float q_scale;     // sm_scale * log2(e)
    float corr_scale;
    float thresh;      // > 0: Sparse-V on
    int chunk;
    int n_chunks;      // chunks per (seq, head) slot in the workspace
    float* ws_acc;     // [num_seqs][hq][n_chunks][128]
    float* ws_m;       // [num_seqs][hq][n_chunks]  (log2 domain)
    float* ws_l;
    unsigned long long* skip_stats;
};

// Buffer resource over [base, base + 2 GiB): loads at offsets >= kOOB return zero, which is how
// rows past the end of a sequence are masked without branches.
constexpr uint32_t kOOB = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const uint8_t* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), (short)0, 0x7fffffff, 0x00020000);
}

// Half2 dword from two fp16 lanes of two dwords: selects the low (s=0) or high (s=1) halves.
__device__ __forceinline__ uint32_t pick_halves(uint32_t hi_src, uint32_t lo_src, int s) {
    return __builtin_amdgcn_perm(hi_src, lo_src, s ? 0x07060302u : 0x05040100u);
}

__device__ __forceinline__ float f16lo(uint32_t w) { return tq_f16_to_f32(w & 0xffffu); }
__device__ __forceinline__ float f16hi(uint32_t w) { return tq_f16_to_f32(w >> 16); }

// Raw per-lane data of one 16-token tile (see the load plan in decode_kernel).
template <int KB, bool KQJL, int VB>
struct TileRaw {
    uint32_t kw[KB];                      // 32 dims of token n: 32*KB bits
    uint32_t ks;                          // 32 sign bits of token n
    uint32_t kn[2], krn[2], vn[2];        // fp16 norms of tokens 4g..4g+3
    uint32_t vw[4][VB == 3 ? 2 : 1];      // dims 8n..8n+7 of tokens 4g..4g+3
};

struct LaneOffsets {
    uint32_t kidx, ksig;
    uint32_t kn[4], krn[4], vn[4];        // per token 4g+r (u16 loads)
    uint32_t kn8, krn8, vn8;              // 4 consecutive fp16 (b64 load) when rows are 2 bytes apart
    uint32_t vidx[4];
    int vshift;                           // VB == 3: bit offset of the 24-bit field in the 8-byte window
};

struct TileBases {
    const uint8_t *kidx, *ksig, *kn, *krn, *vidx, *vn;
};

template <int KB, bool KQJL, int VB>
__device__ __forceinline__ void load_tile(TileRaw<KB, KQJL, VB>& t, const TileBases& b, const LaneOffsets& o,
                                          int nvalid, int n, int g, bool norm_vec) {
    const bool krow = n < nvalid;
    {
        auto r = make_rsrc(b.kidx);
        const uint32_t off = krow ? o.kidx : kOOB;
        if (KB == 2) {
            tq_u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
            t.kw[0] = v[0]; t.kw[1 % KB] = v[1];
        } else if (KB == 3) {
            typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
            u32x3 v = __builtin_amdgcn_raw_buffer_load_b96(r, off, 0, 0);
            t.kw[0] = v[0]; t.kw[1 % KB] = v[1]; t.kw[2 % KB] = v[2];
        } else {
            tq_u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
            t.kw[0] = v[0]; t.kw[1 % KB] = v[1]; t.kw[2 % KB] = v[2]; t.kw[3 % KB] = v[3];
        }
    }
    if (KQJL) t.ks = __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(b.ksig), krow ? o.ksig : kOOB, 0, 0);
    const bool all4 = 4 * g + 3 < nvalid;
    if (norm_vec && all4) {
        tq_u32x2 a = __builtin_amdgcn_raw_buffer_load_b64(make_rsrc(b.kn), o.kn8, 0, 0);
        t.kn[0] = a[0]; t.kn[1] = a[1];
        tq_u32x2 c = __builtin_amdgcn_raw_buffer_load_b64(make_rsrc(b.vn), o.vn8, 0, 0);
        t.vn[0] = c[0]; t.vn[1] = c[1];
        if (KQJL) {
            tq_u32x2 d = __builtin_amdgcn_raw_buffer_load_b64(make_rsrc(b.krn), o.krn8, 0, 0);
            t.krn[0] = d[0]; t.krn[1] = d[1];
        }
    } else {
        uint32_t kv[4], vv[4], rv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const bool ok = 4 * g + r < nvalid;
            kv[r] = __builtin_amdgcn_raw_buffer_load_b16(make_rsrc(b.kn), ok ? o.kn[r] : kOOB, 0, 0);
            vv[r] = __builtin_amdgcn_raw_buffer_load_b16(make_rsrc(b.vn), ok ? o.vn[r] : kOOB, 0, 0);
            if (KQJL) rv[r] = __builtin_amdgcn_raw_buffer_load_b16(make_rsrc(b.krn), ok ? o.krn[r] : kOOB, 0, 0);
        }
        t.kn[0] = kv[0] | (kv[1] << 16); t.kn[1] = kv[2] | (kv[3] << 16);
        t.vn[0] = vv[0] | (vv[1] << 16); t.vn[1] = vv[2] | (vv[3] << 16);
        if (KQJL) { t.krn[0] = rv[0] | (rv[1] << 16); t.krn[1] = rv[2] | (rv[3] << 16); }
    }
    auto rv = make_rsrc(b.vidx);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint32_t off = (4 * g + r < nvalid) ? o.vidx[r] : kOOB;
        if (VB == 3) {
            tq_u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(rv, off, 0, 0);
            t.vw[r][0] = w[0]; t.vw[r][VB == 3 ? 1 : 0] = w[1];
        } else if (VB == 4) {
            t.vw[r][0] = __builtin_amdgcn_raw_buffer_load_b32(rv, off, 0, 0);
        } else {
            t.vw[r][0] = __builtin_amdgcn_raw_buffer_load_b16(rv, off, 0, 0);
        }
    }
}

// QCOLS: the GQA group fits in 8 heads, so the 16 columns of the QK product carry q (hi part,
// columns 0..7) and q - hi (lo part, columns 8..15); a lane swizzle merges them.
template <int KB, bool KQJL, int VB, bool QCOLS>
__global__ __launch_bounds__(256) void decode_kernel(DecodeParams p) {
    constexpr int KENT = 1 << (2 * KB);
    constexpr int VENT = 1 << (2 * VB);
    __shared__ uint32_t s_ktab[KENT * 32];
    __shared__ uint32_t s_vtab[VENT * 32];

    // Pair tables: entry e -> half2(c[e & (2^b - 1)], c[e >> b]) * cscale, 32 bank replicas.
    for (int i = threadIdx.x; i < KENT * 32; i += 256) {
        int e = i >> 5;
        s_ktab[i] = tq_pack_half2(p.k_cent[e & ((1 << KB) - 1)] * p.k_cscale, p.k_cent[e >> KB] * p.k_cscale);
    }
    for (int i = threadIdx.x; i < VENT * 32; i += 256) {
        int e = i >> 5;
        s_vtab[i] = tq_pack_half2(p.v_cent[e & ((1 << VB) - 1)] * p.v_cscale, p.v_cent[e >> VB] * p.v_cscale);
    }
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int g = lane >> 4;   // lane group: dims 32g.. (K), tokens 4g..4g+3 (scores, V)
    const int n = lane & 15;   // head column (Q/P/out), token row (K loads), dim row (V)
    const uint32_t bank4 = (uint32_t)(lane & 31) << 2;

    const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int c = (int)(unit % p.n_chunks);
    const int64_t sk = unit / p.n_chunks;
    const int kh = (int)(sk % p.hkv);
    const int64_t s = sk / p.hkv;
    if (s >= p.num_seqs) return;

    int L = p.seq_lens[s];
    const int cap = p.max_blocks * p.block_size;
    L = L < cap ? L : cap;
    const int t_begin = c * p.chunk;
    if (t_begin >= L) return;
    const int t_end = (t_begin + p.chunk < L) ? t_begin + p.chunk : L;
    const bool paged = p.bt != nullptr;

    // ---- query operands (B of the QK products), pre-scaled into the log2 domain ----
    const int hq_col = QCOLS ? (n & 7) : n;
    const int head = kh * p.group + hq_col;
    const bool hvalid = n < p.group;
    const bool qload = hq_col < p.group;
    tq_half8 qop[4];
    tq_half8 qlo[QCOLS ? 1 : 4];
    tq_half8 qpop[KQJL ? 4 : 1];
    {
        const int64_t qoff = s * p.q_ss + (int64_t)head * p.q_sh;
        const int64_t qpoff = s * p.qp_ss + (int64_t)head * p.qp_sh;
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float qv = qload ? tq_load1(p.q, qoff + 32 * g + 8 * cc + j, p.q_dtype) * p.q_scale : 0.f;
                const _Float16 qh = (_Float16)qv;
                const _Float16 ql = (_Float16)(qv - (float)qh);
                if (QCOLS) {
                    qop[cc][j] = n < 8 ? qh : ql;
                } else {
                    qop[cc][j] = qh;
                    qlo[cc % (QCOLS ? 1 : 4)][j] = ql;
                }
                if (KQJL) {
                    const int bit = 4 * cc + (j >> 1) + 16 * (j & 1);
                    const int dim = p.k_perm ? 4 * bit + g : 32 * g + bit;
                    const float qpv = hvalid ? -tq_load1(p.qp, qpoff + dim, p.q_dtype) * p.q_scale : 0.f;
                    qpop[cc % (KQJL ? 4 : 1)][j] = (_Float16)qpv;
                }
            }
        }
    }

    // ---- loop-invariant per-lane byte offsets inside a tile ----
    LaneOffsets o;
    o.kidx = (uint32_t)(n * p.k_idx.stride_row + 4 * KB * g);
    o.ksig = KQJL ? (uint32_t)(n * p.k_sig.stride_row + 4 * g) : 0u;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int tok = 4 * g + r;
        o.kn[r] = (uint32_t)(tok * p.k_norm.stride_row);
        o.vn[r] = (uint32_t)(tok * p.v_norm.stride_row);
        o.krn[r] = KQJL ? (uint32_t)(tok * p.k_rnorm.stride_row) : 0u;
        if (VB == 3) {
            const int byte0 = 3 * n;
            int start = (byte0 >> 2) << 2;
            start = start < 40 ? start : 40;      // 8-byte window kept inside the 48-byte row
            o.vidx[r] = (uint32_t)(tok * p.v_idx.stride_row + start);
            o.vshift = 8 * (byte0 - start);
        } else {
            o.vidx[r] = (uint32_t)(tok * p.v_idx.stride_row + VB * n);
            o.vshift = 0;
        }
    }
    o.kn8 = o.kn[0];
    o.vn8 = o.vn[0];
    o.krn8 = o.krn[0];
    // Norm rows 2 bytes apart inside allocated blocks: one 8-byte load per region.
    const bool norm_vec = paged && p.k_norm.stride_row == 2 && p.v_norm.stride_row == 2 &&
                          (!KQJL || p.k_rnorm.stride_row == 2);

    // Per-unit parts of the tile bases (uniform).
    const int64_t seq_off_k = paged ? 0 : s * p.k_idx.stride_seq;
    auto bases_for = [&](int64_t blk, int st) {
        TileBases b;
        const int64_t so = paged ? 0 : s;
        b.kidx = p.k_idx.ptr + blk * p.k_idx.stride_block + kh * p.k_idx.stride_head + so * p.k_idx.stride_seq + st * p.k_idx.stride_row;
        b.kn = p.k_norm.ptr + blk * p.k_norm.stride_block + kh * p.k_norm.stride_head + so * p.k_norm.stride_seq + st * p.k_norm.stride_row;
        b.vidx = p.v_idx.ptr + blk * p.v_idx.stride_block + kh * p.v_idx.stride_head + so * p.v_idx.stride_seq + st * p.v_idx.stride_row;
        b.vn = p.v_norm.ptr + blk * p.v_norm.stride_block + kh * p.v_norm.stride_head + so * p.v_norm.stride_seq + st * p.v_norm.stride_row;
        if (KQJL) {
            b.ksig = p.k_sig.ptr + blk * p.k_sig.stride_block + kh * p.k_sig.stride_head + so * p.k_sig.stride_seq + st * p.k_sig.stride_row;
            b.krn = p.k_rnorm.ptr + blk * p.k_rnorm.stride_block + kh * p.k_rnorm.stride_head + so * p.k_rnorm.stride_seq + st * p.k_rnorm.stride_row;
        } else {
            b.ksig = b.kidx;
            b.krn = b.kn;
        }
        return b;
    };
    (void)seq_off_k;
    // Tile t0 -> (bases, rows valid); a block-table entry outside [0, num_blocks) reads nothing.
    auto locate = [&](int t0, TileBases& b, int& nvalid) {
        const int lb = t0 / p.block_size;
        const int st = t0 - lb * p.block_size;
        int64_t blk = lb;
        nvalid = (t_end - t0 < 16) ? t_end - t0 : 16;
        if (paged) {
            blk = p.bt[s * p.bt_stride + lb];
            if (blk < 0 || blk >= p.num_blocks) {
                blk = 0;
                nvalid = 0;
            }
        }
        b = bases_for(blk, st);
    };

    float m = kNegInf;
    float lsum = 0.f;
    tq_floatx4 acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = tq_floatx4{0.f, 0.f, 0.f, 0.f};
    unsigned long long n_skip = 0, n_tot = 0;
    const bool sparse = p.thresh > 0.f;

    TileRaw<KB, KQJL, VB> cur = {}, nxt = {};
    int cur_valid, nxt_valid = 0;
    {
        TileBases b;
        locate(t_begin, b, cur_valid);
        load_tile<KB, KQJL, VB>(cur, b, o, cur_valid, n, g, norm_vec);
    }

    for (int t0 = t_begin; t0 < t_end; t0 += 16) {
        const bool more = t0 + 16 < t_end;
        if (more) {  // prefetch the next tile while this one is computed
            TileBases b;
            locate(t0 + 16, b, nxt_valid);
            load_tile<KB, KQJL, VB>(nxt, b, o, nxt_valid, n, g, norm_vec);
        }

        // ---------------- QK products ----------------
        tq_floatx4 s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            tq_u32x4 a;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t e = tq_field(cur.kw, 2 * KB * (4 * cc + j), 2 * KB);
                a[j] = s_ktab[(e << 5) | (bank4 >> 2)];
            }
            const tq_half8 ah = __builtin_bit_cast(tq_half8, a);
            s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, qop[cc], s1, 0, 0, 0);
            if (!QCOLS) s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, qlo[cc % (QCOLS ? 1 : 4)], s1, 0, 0, 0);
        }
        tq_floatx4 s2 = {0.f, 0.f, 0.f, 0.f};
        if (KQJL) {
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                tq_u32x4 a;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int pp = 4 * cc + j;
                    a[j] = ((cur.ks << (15 - pp)) & 0x80008000u) | 0x3C003C00u;
                }
                s2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(tq_half8, a), qpop[cc % (KQJL ? 4 : 1)], s2, 0, 0, 0);
            }
        }
        float s1v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) s1v[r] = s1[r];
        if (QCOLS) {
            // column n (hi part) + column n ^ 8 (lo part): swizzle xor 8 inside each 16-lane row.
            // Scalar copies on purpose: shuffling elements of an ext_vector in place miscompiles
            // (the backend reuses one shuffle result for the other elements).
            int sw[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) sw[r] = __builtin_amdgcn_ds_swizzle(__float_as_int(s1v[r]), 0x201f);
#pragma unroll
            for (int r = 0; r < 4; ++r) s1v[r] += __int_as_float(sw[r]);
        }

        // ---------------- online softmax ----------------
        float sc[4], kn[4], vn[4];
        kn[0] = f16lo(cur.kn[0]); kn[1] = f16hi(cur.kn[0]); kn[2] = f16lo(cur.kn[1]); kn[3] = f16hi(cur.kn[1]);
        vn[0] = f16lo(cur.vn[0]); vn[1] = f16hi(cur.vn[0]); vn[2] = f16lo(cur.vn[1]); vn[3] = f16hi(cur.vn[1]);
        float mt = kNegInf;
        bool tv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            tv[r] = 4 * g + r < cur_valid;
            float v = kn[r] * p.k_cinv * s1v[r];
            if (KQJL) {
                const float rn = (r & 1) ? f16hi(cur.krn[r >> 1]) : f16lo(cur.krn[r >> 1]);
                v = __builtin_fmaf(rn * p.corr_scale, s2[r], v);
            }
            sc[r] = tv[r] ? v : kNegInf;
            mt = fmaxf(mt, sc[r]);
        }
        mt = fmaxf(mt, __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, mt), 0x401f)));
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float m_new = fmaxf(m, mt);
        const float mref = m_new == kNegInf ? 0.f : m_new;
        float pr[4];
        float psum = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            pr[r] = __builtin_amdgcn_exp2f(sc[r] - mref);
            psum += pr[r];
        }
        // Rescale only when some head's running max moved (alpha == 1 otherwise).
        if (__ballot(hvalid && m_new > m) != 0) {
            const float alpha = __builtin_amdgcn_exp2f(m - mref);
            lsum *= alpha;
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] *= alpha;
        }
        lsum += psum;
        m = m_new;

        // Sparse-V: token significant when some head of the group has p > thresh.
        bool sig[4] = {true, true, true, true};
        bool any = true;
        if (sparse) {
            uint64_t orall = 0;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint64_t bal = __ballot(hvalid && pr[r] > p.thresh);
                orall |= bal;
                sig[r] = ((bal >> (16 * g)) & 0xffffull) != 0;
            }
            any = orall != 0;
            if (p.skip_stats && n == 0) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    n_tot += tv[r] ? 1 : 0;
                    n_skip += (tv[r] && !sig[r]) ? 1 : 0;
                }
            }
        }

        if (any) {
            float pv[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) pv[r] = (tv[r] && sig[r]) ? pr[r] * (vn[r] * p.v_cinv) : 0.f;
            tq_u32x2 bw = {tq_pack_half2(pv[0], pv[1]), tq_pack_half2(pv[2], pv[3])};
            const tq_half4 bop = __builtin_bit_cast(tq_half4, bw);
            // V dequant: vp[r][q] = half2(dims 8n+2q, 8n+2q+1) of token 4g+r.
            uint32_t vp[4][4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                uint32_t w;
                if (VB == 3) {
                    const uint32_t hi = cur.vw[r][VB == 3 ? 1 : 0], lo = cur.vw[r][0];
                    w = o.vshift >= 32 ? (hi >> (o.vshift - 32)) : __builtin_amdgcn_alignbit(hi, lo, o.vshift);
                } else {
                    w = cur.vw[r][0];
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint32_t e = (w >> (2 * VB * q)) & (VENT - 1);
                    vp[r][q] = s_vtab[(e << 5) | (bank4 >> 2)];
                }
            }
#pragma unroll
            for (int nn = 0; nn < 8; ++nn) {
                const int q = nn >> 1, hs = nn & 1;
                tq_u32x2 aw = {pick_halves(vp[1][q], vp[0][q], hs), pick_halves(vp[3][q], vp[2][q], hs)};
                acc[nn] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(tq_half4, aw), bop, acc[nn], 0, 0, 0);
            }
        }
        if (more) {
            cur = nxt;
            cur_valid = nxt_valid;
        }
    }

    lsum += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, lsum), 0x401f));
    lsum += __shfl_xor(lsum, 32);

    if (hvalid) {
        const int64_t slot = ((s * p.hq + head) * (int64_t)p.n_chunks + c);
        if (g == 0) {
            p.ws_m[slot] = m;
            p.ws_l[slot] = lsum;
        }
        // acc[nn][r] is dim 8*(4g+r)+nn = 32g + 8r + nn.
        float4* dst = reinterpret_cast<float4*>(p.ws_acc + slot * TQ_HEAD_DIM + 32 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            dst[2 * r] = make_float4(acc[0][r], acc[1][r], acc[2][r], acc[3][r]);
            dst[2 * r + 1] = make_float4(acc[4][r], acc[5][r], acc[6][r], acc[7][r]);
        }
    }
    if (sparse && p.skip_stats) {
        unsigned long long a = n_skip, b = n_tot;
        a += __shfl_xor(a, 16);
        a += __shfl_xor(a, 32);
        b += __shfl_xor(b, 16);
        b += __shfl_xor(b, 32);
        if (lane == 0) {
            atomicAdd(p.skip_stats, a);
            atomicAdd(p.skip_stats + 1, b);
        }
    }
}

struct ReduceParams {
    const float* ws_acc;
    const float* ws_m;
    const float* ws_l;
    int num_seqs, hq, n_chunks, chunk, cap;
    const int32_t* seq_lens;
    void* out;
    int out_dtype;
    int64_t out_ss, out_sh;
};

// One wave per (sequence, query head); lane d covers dims 2d, 2d+1.
__global__ __launch_bounds__(64) void decode_reduce_kernel(ReduceParams p) {
    const int64_t sh = blockIdx.x;
    const int64_t s = sh / p.hq;
    const int h = (int)(sh - s * p.hq);
    const int lane = threadIdx.x;
    int L = p.seq_lens[s];
    L = L < p.cap ? L : p.cap;
    int nch = L > 0 ? (L + p.chunk - 1) / p.chunk : 0;
    nch = nch < p.n_chunks ? nch : p.n_chunks;  // tokens past max_seq_len were not processed
    const int64_t base = sh * p.n_chunks;
    float M = kNegInf;
    for (int c = 0; c < nch; ++c) M = fmaxf(M, p.ws_m[base + c]);
    float den = 0.f, a0 = 0.f, a1 = 0.f;
    if (M != kNegInf) {
        for (int c = 0; c < nch; ++c) {
            const float w = __builtin_amdgcn_exp2f(p.ws_m[base + c] - M);
            den = __builtin_fmaf(w, p.ws_l[base + c], den);
            const float2 v = reinterpret_cast<const float2*>(p.ws_acc + (base + c) * TQ_HEAD_DIM)[lane];
            a0 = __builtin_fmaf(w, v.x, a0);
            a1 = __builtin_fmaf(w, v.y, a1);
        }
    }
    const float inv = den > 0.f ? 1.0f / den : 0.f;
    const int64_t o = s * p.out_ss + (int64_t)h * p.out_sh + 2 * lane;
    tq_store1(p.out, o, p.out_dtype, a0 * inv);
    tq_store1(p.out, o + 1, p.out_dtype, a1 * inv);
}

bool aligned(const void* ptr, uintptr_t a) { return (reinterpret_cast<uintptr_t>(ptr) & (a - 1)) == 0; }

int check_region(const tq_region& r, int align) {
    if (!r.ptr) return TQ_ERR_INVALID_ARGUMENT;
    if (!aligned(r.ptr, align) || r.stride_block % align || r.stride_head % align || r.stride_seq % align ||
        r.stride_row % align)
        return TQ_ERR_ALIGNMENT;
    return TQ_OK;
}

Region to_region(const tq_region& r) {
    Region o;
    o.ptr = static_cast<const uint8_t*>(r.ptr);
    o.stride_block = r.stride_block;
    o.stride_head = r.stride_head;
    o.stride_seq = r.stride_seq;
    o.stride_row = r.stride_row;
    return o;
}

int n_chunks_for(int max_seq_len, int chunk) { return max_seq_len <= 0 ? 1 : (max_seq_len + chunk - 1) / chunk; }

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

}  // namespace

extern "C" size_t tq_decode_workspace_bytes(int num_seqs, int num_q_heads, int max_seq_len, int tokens_per_chunk) {
    if (num_seqs <= 0 || num_q_heads <= 0 || tokens_per_chunk <= 0) return 0;
    const size_t slots = (size_t)num_seqs * num_q_heads * n_chunks_for(max_seq_len, tokens_per_chunk);
    return align_up(slots * TQ_HEAD_DIM * sizeof(float), 256) + 2 * align_up(slots * sizeof(float), 256);
}

extern "C" int tq_decode(const void* q, int q_dtype, int64_t q_stride_seq, int64_t q_stride_head,
                         const void* q_proj, int64_t qp_stride_seq, int64_t qp_stride_head,
                         int num_seqs, int num_q_heads, int num_kv_heads, int head_dim,
                         const tq_kv_view* k, const tq_kv_view* v,
                         int block_size, int64_t num_blocks,
                         const int32_t* block_tables, int64_t block_table_stride, int max_blocks_per_seq,
                         const int32_t* seq_lens, int max_seq_len,
                         float sm_scale, float corr_scale, float sparse_threshold,
                         int tokens_per_chunk,
                         void* workspace, size_t workspace_bytes,
                         void* out, int out_dtype, int64_t out_stride_seq, int64_t out_stride_head,
                         unsigned long long* skip_stats,
                         tq_stream_t stream) {
    if (head_dim != TQ_HEAD_DIM) return TQ_ERR_HEAD_DIM;
    if (!k || !v) return TQ_ERR_INVALID_ARGUMENT;
    if (num_seqs < 0 || num_q_heads <= 0 || num_kv_heads <= 0) return TQ_ERR_INVALID_ARGUMENT;
    if (num_q_heads % num_kv_heads) return TQ_ERR_GQA;
    const int group = num_q_heads / num_kv_heads;
    if (group > 16) return TQ_ERR_GQA;
    if (k->bits < 2 || k->bits > 4 || v->bits < 2 || v->bits > 4) return TQ_ERR_BITS;
    if (v->qjl) return TQ_ERR_INVALID_ARGUMENT;
    if (block_size <= 0 || block_size % 16) return TQ_ERR_BLOCK_SIZE;
    if (tokens_per_chunk <= 0 || tokens_per_chunk % 16) return TQ_ERR_CHUNK;
    if (q_dtype != TQ_F32 && q_dtype != TQ_F16 && q_dtype != TQ_BF16) return TQ_ERR_DTYPE;
    if (out_dtype != TQ_F32 && out_dtype != TQ_F16 && out_dtype != TQ_BF16) return TQ_ERR_DTYPE;
    if (max_blocks_per_seq < 0 || num_blocks < 0) return TQ_ERR_INVALID_ARGUMENT;
    if (num_seqs == 0) return TQ_OK;
    if (!q || !seq_lens || !out || !k->centroids || !v->centroids) return TQ_ERR_INVALID_ARGUMENT;
    if (block_tables && block_table_stride < max_blocks_per_seq) return TQ_ERR_INVALID_ARGUMENT;
    int rc;
    if ((rc = check_region(k->idx, 4))) return rc;
    if ((rc = check_region(k->norm, 2))) return rc;
    if ((rc = check_region(v->idx, 4))) return rc;
    if ((rc = check_region(v->norm, 2))) return rc;
    if (k->qjl) {
        if ((rc = check_region(k->signs, 4))) return rc;
        if ((rc = check_region(k->rnorm, 2))) return rc;
    }
    const int n_chunks = n_chunks_for(max_seq_len, tokens_per_chunk);
    const size_t need = tq_decode_workspace_bytes(num_seqs, num_q_heads, max_seq_len, tokens_per_chunk);
    if (!workspace || workspace_bytes < need || !aligned(workspace, 256)) return TQ_ERR_WORKSPACE;

    const size_t slots = (size_t)num_seqs * num_q_heads * n_chunks;
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    float* ws_acc = reinterpret_cast<float*>(ws);
    float* ws_m = reinterpret_cast<float*>(ws + align_up(slots * TQ_HEAD_DIM * sizeof(float), 256));
    float* ws_l = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(ws_m) + align_up(slots * sizeof(float), 256));

    DecodeParams p = {};
    p.q = q;
    p.q_ss = q_stride_seq;
    p.q_sh = q_stride_head;
    p.qp = q_proj ? q_proj : q;
    p.qp_ss = q_proj ? qp_stride_seq : q_stride_seq;
    p.qp_sh = q_proj ? qp_stride_head : q_stride_head;
    p.q_dtype = q_dtype;
    p.num_seqs = num_seqs;
    p.hq = num_q_heads;
    p.hkv = num_kv_heads;
    p.group = group;
    p.k_idx = to_region(k->idx);
    p.k_norm = to_region(k->norm);
    if (k->qjl) {
        p.k_sig = to_region(k->signs);
        p.k_rnorm = to_region(k->rnorm);
    }
    p.v_idx = to_region(v->idx);
    p.v_norm = to_region(v->norm);
    p.k_cent = k->centroids;
    p.v_cent = v->centroids;
    p.k_cscale = k->centroid_scale > 0.f ? k->centroid_scale : 1.f;
    p.v_cscale = v->centroid_scale > 0.f ? v->centroid_scale : 1.f;
    p.k_cinv = 1.f / p.k_cscale;
    p.v_cinv = 1.f / p.v_cscale;
    p.k_perm = k->signs_permuted ? 1 : 0;
    p.block_size = block_size;
    p.num_blocks = block_tables ? num_blocks : (int64_t)1 << 62;
    p.bt = block_tables;
    p.bt_stride = block_table_stride;
    p.max_blocks = max_blocks_per_seq;
    p.seq_lens = seq_lens;
    p.q_scale = sm_scale * kLog2e;
    p.corr_scale = corr_scale;
    p.thresh = sparse_threshold > 0.f ? sparse_threshold : 0.f;
    p.chunk = tokens_per_chunk;
    p.n_chunks = n_chunks;
    p.ws_acc = ws_acc;
    p.ws_m = ws_m;
    p.ws_l = ws_l;
    p.skip_stats = skip_stats;

    const int64_t units = (int64_t)num_seqs * num_kv_heads * n_chunks;
    const int64_t grid = (units + 3) / 4;
    if (grid > 0x7fffffff) return TQ_ERR_INVALID_ARGUMENT;
    hipStream_t st = (hipStream_t)stream;
#define TQ_DEC(KB, KQ, VB)                                                                           \
    do {                                                                                             \
        if (group <= 8)                                                                              \
            hipLaunchKernelGGL((decode_kernel<KB, KQ, VB, true>), dim3((unsigned)grid), dim3(256), 0, st, p); \
        else                                                                                         \
            hipLaunchKernelGGL((decode_kernel<KB, KQ, VB, false>), dim3((unsigned)grid), dim3(256), 0, st, p); \
    } while (0)
    const int key = (k->bits * 10 + v->bits) * 2 + (k->qjl ? 1 : 0);
    switch (key) {
        case 44: TQ_DEC(2, false, 2); break;
        case 45: TQ_DEC(2, true, 2); break;
        case 46: TQ_DEC(2, false, 3); break;
        case 47: TQ_DEC(2, true, 3); break;
        case 48: TQ_DEC(2, false, 4); break;
        case 49: TQ_DEC(2, true, 4); break;
        case 64: TQ_DEC(3, false, 2); break;
        case 65: TQ_DEC(3, true, 2); break;
        case 66: TQ_DEC(3, false, 3); break;
        case 67: TQ_DEC(3, true, 3); break;
        case 68: TQ_DEC(3, false, 4); break;
        case 69: TQ_DEC(3, true, 4); break;
        case 84: TQ_DEC(4, false, 2); break;
        case 85: TQ_DEC(4, true, 2); break;
        case 86: TQ_DEC(4, false, 3); break;
        case 87: TQ_DEC(4, true, 3); break;
        case 88: TQ_DEC(4, false, 4); break;
        case 89: TQ_DEC(4, true, 4); break;
        default: return TQ_ERR_BITS;
    }
#undef TQ_DEC
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;

    ReduceParams rp;
    rp.ws_acc = ws_acc;
    rp.ws_m = ws_m;
    rp.ws_l = ws_l;
    rp.num_seqs = num_seqs;
    rp.hq = num_q_heads;
    rp.n_chunks = n_chunks;
    rp.chunk = tokens_per_chunk;
    rp.cap = max_blocks_per_seq * block_size;
    rp.seq_lens = seq_lens;
    rp.out = out;
    rp.out_dtype = out_dtype;
    rp.out_ss = out_stride_seq;
    rp.out_sh = out_stride_head;
    hipLaunchKernelGGL(decode_reduce_kernel, dim3((unsigned)((int64_t)num_seqs * num_q_heads)), dim3(64), 0, st, rp);
    e = hipGetLastError();
    return e == hipSuccess ? TQ_OK : (int)e;
}
