// Packed asymmetric split-K decode attention for gfx950.
//
// Work unit = one wave64 = (sequence, KV head, chunk of tokens_per_chunk tokens), walked in
// tiles of 16 tokens.  A 256-thread workgroup holds 4 units and shares two LDS lookup tables
// that turn a pair of packed indices (2*bits bits) into a half2 of centroids; each table is
// replicated 32x across LDS banks so lanes 0-31 never conflict.
//
// Per tile (all MFMA accumulation in fp32):
//   S^T[token][head]   = K_dq[16 x 128] . Q^T[128 x 16]       4 x mfma_f32_16x16x32_f16
//   QJL^T[token][head] = (+-1)[16 x 128] . (-QP)^T             4 x mfma_f32_16x16x32_f16
//   score = norm * S + corr_scale * rnorm * QJL   (log2 domain: Q pre-scaled by sm_scale*log2 e)
//   online softmax per head; Sparse-V mask from a ballot over the GQA group
//   acc^T[dim][head] += V_dq^T[128 x 16] . (p * vnorm)[16 x 16]  8 x mfma_f32_16x16x16f16
// MFMA output layout (16x16): lane l holds rows 4*(l/16)+r, column l%16, so after the QK
// product lane (head n = l%16, g = l/16) owns tokens 4g..4g+3 of head n, which is exactly the
// B-operand layout of the PV product: no data movement between the two products.
//
// Memory: every per-token stream is read with buffer loads whose base (the tile's address,
// computed once per tile in scalar registers) is uniform and whose per-lane offsets are loop
// invariant; the next tile is loaded while the current one is computed (two register sets,
// loop unrolled by two).  In a paged cache all rows of a block are allocated, so tiles are read
// whole and rows past the sequence end are masked in the softmax; in a contiguous layout rows
// past the end get an out-of-range offset and read as zero.
//
// Each unit writes (m, l, acc[128]) per head; decode_reduce_kernel combines chunks:
//   out = sum_c 2^(m_c - M) acc_c / sum_c 2^(m_c - M) l_c      (kernels/attention.py:121-140)
#include "tq_common.h"

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();
constexpr uint32_t kOOB = 0x80000000u;  // >= num_records: buffer loads return zero

enum { R_KIDX = 0, R_KSIG, R_KNORM, R_KRNORM, R_VIDX, R_VNORM, R_COUNT };

struct DecodeParams {
    const void* q;
    int64_t q_ss, q_sh;
    const void* qp;
    int64_t qp_ss, qp_sh;
    int q_dtype;
    int q_vec;          // q and qp rows 16-byte aligned: vector loads
    int num_seqs, hq, hkv, group;
    const uint8_t* rptr[R_COUNT];
    int64_t rhead[R_COUNT];
    int64_t rseq[R_COUNT];
    int32_t rrow[R_COUNT];
    int64_t sb_k, sb_v;  // block strides shared by the K regions and by the V regions (paged)
    const float* k_cent;
    const float* v_cent;
    float k_cscale, v_cscale;  // tables hold fp16(c * cscale); the scale is divided back out
    float v_cinv;
    int k_perm;
    int block_size;
    int64_t num_blocks;
    const int32_t* bt;
    int64_t bt_stride;
    int max_blocks;
    const int32_t* seq_lens;
    float q_scale;     // sm_scale * log2(e) / k_cscale  (MSE operand)
    float qp_scale;    // sm_scale * log2(e)             (QJL operand)
    float corr_scale;
    float thresh;      // > 0: Sparse-V on
    int chunk;
    int n_chunks;      // chunks per (seq, head) slot in the workspace
    float* ws_acc;     // [num_seqs][hq][n_chunks][128]
    float* ws_m;       // [num_seqs][hq][n_chunks]  (log2 domain)
    float* ws_l;
    unsigned long long* skip_stats;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const uint8_t* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), (short)0, 0x7fffffff, 0x00020000);
}

// Half2 dword from two fp16 lanes of two dwords: selects the low (s=0) or high (s=1) halves.
__device__ __forceinline__ uint32_t pick_halves(uint32_t hi_src, uint32_t lo_src, int s) {
    return __builtin_amdgcn_perm(hi_src, lo_src, s ? 0x07060302u : 0x05040100u);
}

__device__ __forceinline__ float f16lo(uint32_t w) { return tq_f16_to_f32(w & 0xffffu); }
__device__ __forceinline__ float f16hi(uint32_t w) { return tq_f16_to_f32(w >> 16); }

// Raw per-lane data of one 16-token tile.
template <int KB, bool KQJL, int VB>
struct TileRaw {
    uint32_t kw[KB];                      // dims 32g..32g+31 of token n: 32*KB bits
    uint32_t ks;                          // sign bits of the same dims
    uint32_t kn[2], krn[2], vn[2];        // fp16 norms of tokens 4g..4g+3
    uint32_t vw[4][VB == 3 ? 2 : 1];      // dims 8n..8n+7 of tokens 4g..4g+3
};

struct LaneOff {
    uint32_t kidx, ksig, kn, krn, vn;     // kn/krn/vn: token 4g (next tokens at +row stride)
    uint32_t vidx[4];
    int vshift;                           // VB == 3: bit offset of the 24-bit field in its 8-byte window
};

struct Tile {
    const uint8_t* base[R_COUNT];
    int nvalid;                           // rows of this tile inside the sequence (0: unreadable)
};

// MASKED: rows >= nvalid may lie outside the allocation (contiguous layout, last tile).
template <int KB, bool KQJL, int VB, bool MASKED>
__device__ __forceinline__ void load_tile(TileRaw<KB, KQJL, VB>& t, const Tile& tl, const LaneOff& o,
                                          const int32_t* rrow, int n, int g, bool norm_vec) {
    const bool krow = !MASKED || n < tl.nvalid;
    {
        auto r = make_rsrc(tl.base[R_KIDX]);
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
    if (KQJL) t.ks = __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(tl.base[R_KSIG]), krow ? o.ksig : kOOB, 0, 0);
    if (!MASKED && norm_vec) {
        tq_u32x2 a = __builtin_amdgcn_raw_buffer_load_b64(make_rsrc(tl.base[R_KNORM]), o.kn, 0, 0);
        t.kn[0] = a[0]; t.kn[1] = a[1];
        tq_u32x2 c = __builtin_amdgcn_raw_buffer_load_b64(make_rsrc(tl.base[R_VNORM]), o.vn, 0, 0);
        t.vn[0] = c[0]; t.vn[1] = c[1];
        if (KQJL) {
            tq_u32x2 d = __builtin_amdgcn_raw_buffer_load_b64(make_rsrc(tl.base[R_KRNORM]), o.krn, 0, 0);
            t.krn[0] = d[0]; t.krn[1] = d[1];
        }
    } else {
        uint32_t kv[4], vv[4], rv[4];
        auto rk = make_rsrc(tl.base[R_KNORM]);
        auto rvn = make_rsrc(tl.base[R_VNORM]);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const bool ok = !MASKED || 4 * g + r < tl.nvalid;
            kv[r] = __builtin_amdgcn_raw_buffer_load_b16(rk, ok ? o.kn + r * rrow[R_KNORM] : kOOB, 0, 0);
            vv[r] = __builtin_amdgcn_raw_buffer_load_b16(rvn, ok ? o.vn + r * rrow[R_VNORM] : kOOB, 0, 0);
            if (KQJL)
                rv[r] = __builtin_amdgcn_raw_buffer_load_b16(make_rsrc(tl.base[R_KRNORM]),
                                                             ok ? o.krn + r * rrow[R_KRNORM] : kOOB, 0, 0);
        }
        t.kn[0] = kv[0] | (kv[1] << 16); t.kn[1] = kv[2] | (kv[3] << 16);
        t.vn[0] = vv[0] | (vv[1] << 16); t.vn[1] = vv[2] | (vv[3] << 16);
        if (KQJL) { t.krn[0] = rv[0] | (rv[1] << 16); t.krn[1] = rv[2] | (rv[3] << 16); }
    }
    auto rv = make_rsrc(tl.base[R_VIDX]);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint32_t off = (!MASKED || 4 * g + r < tl.nvalid) ? o.vidx[r] : kOOB;
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

// Online-softmax state of one wave.
struct SoftmaxState {
    float m, lsum;
    tq_floatx4 acc[8];
    unsigned long long n_skip, n_tot;
};

template <int KB, bool KQJL, int VB, bool QCOLS>
__device__ __forceinline__ void compute_tile(const TileRaw<KB, KQJL, VB>& cur, int nvalid, SoftmaxState& st,
                                             const tq_half8 (&qop)[4], const tq_half8 (&qlo)[QCOLS ? 1 : 4],
                                             const tq_half8 (&qpop)[KQJL ? 4 : 1], const uint32_t* s_ktab,
                                             const uint32_t* s_vtab, uint32_t bank, const LaneOff& o, int n, int g,
                                             bool hvalid, const DecodeParams& p, bool sparse, bool count) {
    constexpr int VENT = 1 << (2 * VB);
    // ---------------- QK products ----------------
    tq_floatx4 s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
        tq_u32x4 a;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t e = tq_field(cur.kw, 2 * KB * (4 * cc + j), 2 * KB);
            a[j] = s_ktab[(e << 5) | bank];
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
            s2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(tq_half8, a), qpop[cc % (KQJL ? 4 : 1)], s2,
                                                        0, 0, 0);
        }
    }
    // Scalar copies on purpose: shuffling elements of an ext_vector in place miscompiles (the
    // backend reuses one shuffle result for the other elements).
    float s1v[4], s2v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        s1v[r] = s1[r];
        s2v[r] = s2[r];
    }
    if (QCOLS) {
        // column n (hi part of q) + column n ^ 8 (lo part): swizzle xor 8 inside each 16-lane row
        int sw[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) sw[r] = __builtin_amdgcn_ds_swizzle(__float_as_int(s1v[r]), 0x201f);
#pragma unroll
        for (int r = 0; r < 4; ++r) s1v[r] += __int_as_float(sw[r]);
    }

    // ---------------- online softmax ----------------
    const float kn[4] = {f16lo(cur.kn[0]), f16hi(cur.kn[0]), f16lo(cur.kn[1]), f16hi(cur.kn[1])};
    const float vn[4] = {f16lo(cur.vn[0]), f16hi(cur.vn[0]), f16lo(cur.vn[1]), f16hi(cur.vn[1])};
    float sc[4];
    bool tv[4];
    float mt = kNegInf;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        tv[r] = 4 * g + r < nvalid;
        float v = kn[r] * s1v[r];
        if (KQJL) {
            const float rn = (r & 1) ? f16hi(cur.krn[r >> 1]) : f16lo(cur.krn[r >> 1]);
            v = __builtin_fmaf(rn * p.corr_scale, s2v[r], v);
        }
        sc[r] = tv[r] ? v : kNegInf;
        mt = fmaxf(mt, sc[r]);
    }
    mt = fmaxf(mt, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(mt), 0x401f)));
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    const float m_new = fmaxf(st.m, mt);
    const float mref = m_new == kNegInf ? 0.f : m_new;
    float pr[4];
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        pr[r] = __builtin_amdgcn_exp2f(sc[r] - mref);
        psum += pr[r];
    }
    // Rescale only when some head's running max moved (alpha == 1 otherwise).
    if (__ballot(hvalid && m_new > st.m) != 0) {
        const float alpha = __builtin_amdgcn_exp2f(st.m - mref);
        st.lsum *= alpha;
#pragma unroll
        for (int i = 0; i < 8; ++i) st.acc[i] *= alpha;
    }
    st.lsum += psum;
    st.m = m_new;

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
        if (count && n == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                st.n_tot += tv[r] ? 1 : 0;
                st.n_skip += (tv[r] && !sig[r]) ? 1 : 0;
            }
        }
    }
    if (!any) return;

    // ---------------- PV product ----------------
    float pv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) pv[r] = (tv[r] && sig[r]) ? pr[r] * vn[r] : 0.f;
    tq_u32x2 bw = {tq_pack_half2(pv[0], pv[1]), tq_pack_half2(pv[2], pv[3])};
    const tq_half4 bop = __builtin_bit_cast(tq_half4, bw);
    uint32_t w[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        if (VB == 3) {
            const uint32_t hi = cur.vw[r][VB == 3 ? 1 : 0], lo = cur.vw[r][0];
            w[r] = o.vshift >= 32 ? (hi >> (o.vshift - 32)) : __builtin_amdgcn_alignbit(hi, lo, o.vshift);
        } else {
            w[r] = cur.vw[r][0];
        }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        // dims 8n+2q, 8n+2q+1 of tokens 4g..4g+3
        uint32_t vp[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) vp[r] = s_vtab[(((w[r] >> (2 * VB * q)) & (VENT - 1)) << 5) | bank];
#pragma unroll
        for (int hs = 0; hs < 2; ++hs) {
            tq_u32x2 aw = {pick_halves(vp[1], vp[0], hs), pick_halves(vp[3], vp[2], hs)};
            st.acc[2 * q + hs] =
                __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(tq_half4, aw), bop, st.acc[2 * q + hs], 0, 0, 0);
        }
    }
}

// QCOLS: the GQA group fits in 8 heads, so the 16 columns of the QK product carry q (hi part,
// columns 0..7) and q - hi (lo part, columns 8..15); a lane swizzle merges them.
template <int KB, bool KQJL, int VB, bool QCOLS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 3))) void decode_kernel(DecodeParams p) {
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
    const uint32_t bank = (uint32_t)(lane & 31);

    // The wave index is uniform across the wave; saying so keeps every per-unit value in SGPRs
    // (otherwise buffer descriptors built from it are treated as divergent).
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t unit = (int64_t)blockIdx.x * 4 + wave;
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
        float qv[32], qpv[32];
        const int64_t qoff = s * p.q_ss + (int64_t)head * p.q_sh + 32 * g;
        const int64_t qpoff = s * p.qp_ss + (int64_t)head * p.qp_sh;
        if (qload && p.q_vec) {
#pragma unroll
            for (int i = 0; i < 4; ++i) tq_load8(p.q, qoff + 8 * i, p.q_dtype, &qv[8 * i]);
        } else {
#pragma unroll
            for (int i = 0; i < 32; ++i) qv[i] = qload ? tq_load1(p.q, qoff + i, p.q_dtype) : 0.f;
        }
        if (KQJL) {
            if (hvalid && p.q_vec && !p.k_perm) {
#pragma unroll
                for (int i = 0; i < 4; ++i) tq_load8(p.qp, qpoff + 32 * g + 8 * i, p.q_dtype, &qpv[8 * i]);
            } else {
#pragma unroll
                for (int k = 0; k < 32; ++k) {
                    const int dim = p.k_perm ? 4 * k + g : 32 * g + k;
                    qpv[k] = hvalid ? tq_load1(p.qp, qpoff + dim, p.q_dtype) : 0.f;
                }
            }
        }
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float x = qv[8 * cc + j] * p.q_scale;
                const _Float16 qh = (_Float16)x;
                const _Float16 ql = (_Float16)(x - (float)qh);
                if (QCOLS) {
                    qop[cc][j] = n < 8 ? qh : ql;
                } else {
                    qop[cc][j] = qh;
                    qlo[cc % (QCOLS ? 1 : 4)][j] = ql;
                }
                if (KQJL) {
                    // sign operand slot j of MFMA cc holds bit 4cc + j/2 + 16(j&1) of the lane's 32
                    const int bit = 4 * cc + (j >> 1) + 16 * (j & 1);
                    qpop[cc % (KQJL ? 4 : 1)][j] = (_Float16)(-qpv[bit] * p.qp_scale);
                }
            }
        }
    }

    // ---- loop-invariant per-lane byte offsets inside a tile ----
    LaneOff o;
    o.kidx = (uint32_t)(n * p.rrow[R_KIDX] + 4 * KB * g);
    o.ksig = (uint32_t)(n * p.rrow[R_KSIG] + 4 * g);
    o.kn = (uint32_t)(4 * g * p.rrow[R_KNORM]);
    o.krn = (uint32_t)(4 * g * p.rrow[R_KRNORM]);
    o.vn = (uint32_t)(4 * g * p.rrow[R_VNORM]);
    {
        int start = VB * n;
        o.vshift = 0;
        if (VB == 3) {
            const int byte0 = 3 * n;
            start = (byte0 >> 2) << 2;
            start = start < 40 ? start : 40;  // 8-byte window kept inside the 48-byte row
            o.vshift = 8 * (byte0 - start);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) o.vidx[r] = (uint32_t)((4 * g + r) * p.rrow[R_VIDX] + start);
    }
    // Norm rows 2 bytes apart: one 8-byte load per region.
    const bool norm_vec = p.rrow[R_KNORM] == 2 && p.rrow[R_VNORM] == 2 && (!KQJL || p.rrow[R_KRNORM] == 2);

    // Per-unit part of every region's address.
    const uint8_t* ub[R_COUNT];
#pragma unroll
    for (int r = 0; r < R_COUNT; ++r) ub[r] = p.rptr[r] + kh * p.rhead[r] + (paged ? 0 : s * p.rseq[r]);

    // Block table window: lane i holds entry lb0 + i (refilled every 64 blocks).
    const int nblk_seq = (L + p.block_size - 1) / p.block_size;
    int bt_lb0 = -64;
    int bt_vec = 0;
    auto locate = [&](int t0, Tile& tl) {
        const int lb = t0 / p.block_size;
        const int st = t0 - lb * p.block_size;
        tl.nvalid = (t_end - t0 < 16) ? t_end - t0 : 16;
        int64_t offk = 0, offv = 0;
        if (paged) {
            if (lb - bt_lb0 >= 64) {
                bt_lb0 = lb;
                const int e = lb + lane;
                bt_vec = e < nblk_seq ? p.bt[s * p.bt_stride + e] : 0;
            }
            int64_t blk = __builtin_amdgcn_readlane(bt_vec, lb - bt_lb0);
            if (blk < 0 || blk >= p.num_blocks) {
                blk = 0;
                tl.nvalid = 0;
            }
            offk = blk * p.sb_k;
            offv = blk * p.sb_v;
        }
        const int rowbase = paged ? st : t0;
#pragma unroll
        for (int r = 0; r < R_COUNT; ++r)
            tl.base[r] = ub[r] + (r >= R_VIDX ? offv : offk) + (int64_t)rowbase * p.rrow[r];
    };

    SoftmaxState sm;
    sm.m = kNegInf;
    sm.lsum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) sm.acc[i] = tq_floatx4{0.f, 0.f, 0.f, 0.f};
    sm.n_skip = 0;
    sm.n_tot = 0;
    const bool sparse = p.thresh > 0.f;
    const bool count = sparse && p.skip_stats != nullptr;

    // Loads of the tile at t0: whole tiles in a paged cache (rows allocated), masked rows past the
    // end in a contiguous layout; a tile with an unreadable block entry loads nothing.
    auto fetch = [&](int t0, TileRaw<KB, KQJL, VB>& raw, int& nvalid) {
        Tile tl;
        locate(t0, tl);
        nvalid = tl.nvalid;
        if (tl.nvalid == 0) return;
        if (paged || tl.nvalid == 16)
            load_tile<KB, KQJL, VB, false>(raw, tl, o, p.rrow, n, g, norm_vec);
        else
            load_tile<KB, KQJL, VB, true>(raw, tl, o, p.rrow, n, g, norm_vec);
    };

    TileRaw<KB, KQJL, VB> ra = {}, rb = {};
    int va = 0, vb = 0;
    fetch(t_begin, ra, va);
    for (int t0 = t_begin; t0 < t_end; t0 += 32) {
        if (t0 + 16 < t_end) fetch(t0 + 16, rb, vb);
        compute_tile<KB, KQJL, VB, QCOLS>(ra, va, sm, qop, qlo, qpop, s_ktab, s_vtab, bank, o, n, g, hvalid, p, sparse,
                                          count);
        if (t0 + 16 >= t_end) break;
        if (t0 + 32 < t_end) fetch(t0 + 32, ra, va);
        compute_tile<KB, KQJL, VB, QCOLS>(rb, vb, sm, qop, qlo, qpop, s_ktab, s_vtab, bank, o, n, g, hvalid, p, sparse,
                                          count);
    }

    float lsum = sm.lsum;
    lsum += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(lsum), 0x401f));
    lsum += __shfl_xor(lsum, 32);

    if (hvalid) {
        const int64_t slot = ((s * p.hq + head) * (int64_t)p.n_chunks + c);
        if (g == 0) {
            p.ws_m[slot] = sm.m;
            p.ws_l[slot] = lsum;
        }
        // acc[nn][r] is dim 8*(4g+r)+nn = 32g + 8r + nn; v_cinv undoes the V table scale.
        const float vs = p.v_cinv;
        float4* dst = reinterpret_cast<float4*>(p.ws_acc + slot * TQ_HEAD_DIM + 32 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            dst[2 * r] = make_float4(sm.acc[0][r] * vs, sm.acc[1][r] * vs, sm.acc[2][r] * vs, sm.acc[3][r] * vs);
            dst[2 * r + 1] = make_float4(sm.acc[4][r] * vs, sm.acc[5][r] * vs, sm.acc[6][r] * vs, sm.acc[7][r] * vs);
        }
    }
    if (count) {
        unsigned long long a = sm.n_skip, b = sm.n_tot;
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
    if (r.stride_row <= 0 || r.stride_row > (1 << 20)) return TQ_ERR_INVALID_ARGUMENT;
    return TQ_OK;
}

int n_chunks_for(int max_seq_len, int chunk) { return max_seq_len <= 0 ? 1 : (max_seq_len + chunk - 1) / chunk; }

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

bool q_vector_ok(const void* q, int dtype, int64_t ss, int64_t sh) {
    const int64_t es = dtype == TQ_F32 ? 4 : 2;
    return aligned(q, 16) && (ss * es) % 16 == 0 && (sh * es) % 16 == 0;
}

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
    const tq_region* regs[R_COUNT] = {&k->idx, k->qjl ? &k->signs : &k->idx, &k->norm,
                                      k->qjl ? &k->rnorm : &k->norm, &v->idx, &v->norm};
    int64_t max_row = 0;
    for (int r = 0; r < R_COUNT; ++r) max_row = regs[r]->stride_row > max_row ? regs[r]->stride_row : max_row;
    if (block_tables) {
        // paged: the K regions share one block stride, the V regions another
        for (int r = 1; r < R_VIDX; ++r)
            if (regs[r]->stride_block != regs[R_KIDX]->stride_block) return TQ_ERR_INVALID_ARGUMENT;
        if (regs[R_VNORM]->stride_block != regs[R_VIDX]->stride_block) return TQ_ERR_INVALID_ARGUMENT;
        if ((int64_t)block_size * max_row >= (1ll << 30)) return TQ_ERR_INVALID_ARGUMENT;
    } else {
        // contiguous: token rows follow each other across blocks
        for (int r = 0; r < R_COUNT; ++r)
            if (regs[r]->stride_block != 16 * regs[r]->stride_row) return TQ_ERR_INVALID_ARGUMENT;
        if ((int64_t)(max_blocks_per_seq + 1) * block_size * max_row >= (1ll << 30)) return TQ_ERR_INVALID_ARGUMENT;
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
    p.q_vec = q_vector_ok(p.q, q_dtype, p.q_ss, p.q_sh) && q_vector_ok(p.qp, q_dtype, p.qp_ss, p.qp_sh);
    p.num_seqs = num_seqs;
    p.hq = num_q_heads;
    p.hkv = num_kv_heads;
    p.group = group;
    for (int r = 0; r < R_COUNT; ++r) {
        p.rptr[r] = static_cast<const uint8_t*>(regs[r]->ptr);
        p.rhead[r] = regs[r]->stride_head;
        p.rseq[r] = regs[r]->stride_seq;
        p.rrow[r] = (int32_t)regs[r]->stride_row;
    }
    p.sb_k = regs[R_KIDX]->stride_block;
    p.sb_v = regs[R_VIDX]->stride_block;
    p.k_cent = k->centroids;
    p.v_cent = v->centroids;
    p.k_cscale = k->centroid_scale > 0.f ? k->centroid_scale : 1.f;
    p.v_cscale = v->centroid_scale > 0.f ? v->centroid_scale : 1.f;
    p.v_cinv = 1.f / p.v_cscale;
    p.k_perm = k->signs_permuted ? 1 : 0;
    p.block_size = block_size;
    p.num_blocks = block_tables ? num_blocks : (int64_t)1 << 62;
    p.bt = block_tables;
    p.bt_stride = block_table_stride;
    p.max_blocks = max_blocks_per_seq;
    p.seq_lens = seq_lens;
    p.qp_scale = sm_scale * kLog2e;
    p.q_scale = p.qp_scale / p.k_cscale;
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
