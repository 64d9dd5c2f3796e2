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
// A sequence of one chunk is normalised and written directly.  Otherwise each unit writes
// (m, l, acc[128]) per head to the workspace and decode_reduce_kernel combines the chunks:
//   out = sum_c 2^(m_c - M) acc_c / sum_c 2^(m_c - M) l_c      (kernels/attention.py:121-140)
#include "tq_common.h"
#include "tq_decode_internal.h"

#include <cmath>
#include <cstdlib>
#include <mutex>

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kWhtH = 0.08838834764831845f;  // 1 / sqrt(128): the entries of the normalised H
constexpr float kNegInf = -__builtin_huge_valf();

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
    int share_tab;      // K and V pair tables identical: one LDS table
    int k_perm;
    int block_size;
    int64_t num_blocks;
    const int32_t* bt;
    int64_t bt_stride;
    int max_blocks;
    const int32_t* seq_lens;  // null: every sequence holds uniform_len tokens
    int uniform_len;
    float q_scale;     // sm_scale * log2(e) / k_cscale  (MSE operand)
    float qp_scale;    // sm_scale * log2(e)             (QJL operand)
    float corr_scale;
    float thresh;      // > 0: Sparse-V on
    float log2_thresh;
    int sparse_pair;   // Sparse-V running max per 32-token KV block (two tiles) instead of per tile
    int chunk;
    int n_chunks;      // chunks per (seq, head) slot in the workspace
    float* ws_acc;     // [num_seqs][hq][n_chunks][128]
    float* ws_m;       // [num_seqs][hq][n_chunks]  (log2 domain)
    float* ws_l;
    unsigned long long* skip_stats;
    void* out;
    int out_dtype;
    int64_t out_ss, out_sh;
    int rot_q, rot_qp, rot_out;  // rotate q / q_proj by H on load, the output by H on the write
    float wht_h;                 // 1 / sqrt(128)
    int k_lg, v_lg;              // lane-grouped key / value tiles
    int32_t vstep;               // bytes from value row 4g + r to 4g + r + 1 in the lane's stream
};

// nrec = 0 turns every load through the descriptor into a zero read (unreadable block).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const uint8_t* base, uint32_t nrec) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), (short)0, nrec, 0x00020000);
}

// Scalar operands of buffer loads: a wave-uniform value the compiler may have placed in a
// vector register would otherwise be served by a waterfall loop.
__device__ __forceinline__ int sgpr(int x) { return __builtin_amdgcn_readfirstlane(x); }

typedef __attribute__((address_space(3))) const uint32_t lds_u32;

// Pair-table read.  Tables are placed at LDS addresses that are multiples of their size, so
// (entry << 7) and (table address + 4 * bank) have disjoint bits and OR forms the address.
__device__ __forceinline__ uint32_t lds_read(uint32_t addr) { return *(lds_u32*)(uintptr_t)addr; }

// LDS address of the pair-table entry held in bits [pos, pos + W) of the word array w:
// the field is moved to bit 7 (one shift or funnel shift) and merged with the lane's bank
// address (one and-or).
template <int W, int N>
__device__ __forceinline__ uint32_t pair_addr(const uint32_t (&w)[N], int pos, uint32_t bank_addr) {
    const int wi = pos >> 5, sh = pos & 31;
    uint32_t f;
    if (sh + W <= 32 || wi + 1 >= N)
        f = sh >= 7 ? (w[wi] >> (sh - 7)) : (w[wi] << (7 - sh));
    else
        f = __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh - 7);
    return (f & (((1u << W) - 1u) << 7)) | bank_addr;
}

// Half2 dword from two fp16 lanes of two dwords: selects the low (s=0) or high (s=1) halves.
__device__ __forceinline__ uint32_t pick_halves(uint32_t hi_src, uint32_t lo_src, int s) {
    return __builtin_amdgcn_perm(hi_src, lo_src, s ? 0x07060302u : 0x05040100u);
}

__device__ __forceinline__ float f16lo(uint32_t w) { return tq_f16_to_f32(w & 0xffffu); }
__device__ __forceinline__ float f16hi(uint32_t w) { return tq_f16_to_f32(w >> 16); }

// Raw per-lane data of one 16-token tile.
// NV: norm rows 2 bytes apart, the norms of tokens 4g..4g+3 arrive as two half2 words;
// otherwise one 16-bit load (one word) per token.
template <int KB, bool KQJL, int VB, bool NV>
struct TileRaw {
    uint32_t kw[KB];                      // dims 32g..32g+31 of token n: 32*KB bits
    uint32_t ks;                          // sign bits of the same dims
    uint32_t kn[NV ? 2 : 4], krn[NV ? 2 : 4], vn[NV ? 2 : 4];  // fp16 norms of tokens 4g..4g+3
    uint32_t vw[4][VB == 3 ? 2 : 1];      // dims 8n..8n+7 of tokens 4g..4g+3; values tile layout:
                                          // vw[k][0], k < VB, the words of the lane's chunk
};

template <bool NV>
__device__ __forceinline__ float norm_at(const uint32_t* w, int r) {
    return tq_f16_to_f32(NV ? ((r & 1) ? (w[r >> 1] >> 16) : (w[r >> 1] & 0xffffu)) : (w[r] & 0xffffu));
}

// Loop-invariant per-lane byte offsets inside a tile (norm and V streams: row 4g).
struct LaneOff {
    uint32_t kidx, ksig, kn, krn, vn;     // kn/krn/vn: token 4g
    uint32_t vidx;                        // token 4g
    uint32_t vsel;                        // VB == 3: byte selector of the 3-byte field in its 8-byte window
};

struct Tile {
    const uint8_t* base[R_COUNT];
    uint32_t nrec;                        // buffer record count: 0 for an unreadable block
    int nvalid;                           // rows of this tile inside the sequence (0: unreadable)
};

// Full tiles (MASKED = false): every row is readable; rows 4g+1..4g+3 of the norm and V streams
// are addressed through the scalar offset.  MASKED (contiguous layout, last tile): rows >= nvalid
// may lie outside the allocation, so each region's record count ends at row nvalid and those
// rows read as zero; the row offsets then go into the vector offset, which the range check sees.
template <int KB, bool KQJL, int VB, bool NV, bool MASKED>
__device__ __forceinline__ void load_tile(TileRaw<KB, KQJL, VB, NV>& t, const Tile& tl, const LaneOff& o,
                                          const int32_t* rrow, int32_t vstep, int v_lg) {
    auto nrec = [&](int r) -> uint32_t { return MASKED ? (uint32_t)(tl.nvalid * rrow[r]) : tl.nrec; };
    {
        auto r = make_rsrc(tl.base[R_KIDX], nrec(R_KIDX));
        if (KB == 2) {
            tq_u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, o.kidx, 0, 0);
            t.kw[0] = v[0]; t.kw[1 % KB] = v[1];
        } else if (KB == 3) {
            typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
            u32x3 v = __builtin_amdgcn_raw_buffer_load_b96(r, o.kidx, 0, 0);
            t.kw[0] = v[0]; t.kw[1 % KB] = v[1]; t.kw[2 % KB] = v[2];
        } else {
            tq_u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, o.kidx, 0, 0);
            t.kw[0] = v[0]; t.kw[1 % KB] = v[1]; t.kw[2 % KB] = v[2]; t.kw[3 % KB] = v[3];
        }
    }
    if (KQJL) t.ks = __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(tl.base[R_KSIG], nrec(R_KSIG)), o.ksig, 0, 0);
    if (!MASKED && NV) {
        tq_u32x2 a = __builtin_amdgcn_raw_buffer_load_b64(make_rsrc(tl.base[R_KNORM], tl.nrec), o.kn, 0, 0);
        t.kn[0] = a[0]; t.kn[1] = a[1];
        tq_u32x2 c = __builtin_amdgcn_raw_buffer_load_b64(make_rsrc(tl.base[R_VNORM], tl.nrec), o.vn, 0, 0);
        t.vn[0] = c[0]; t.vn[1] = c[1];
        if (KQJL) {
            tq_u32x2 d = __builtin_amdgcn_raw_buffer_load_b64(make_rsrc(tl.base[R_KRNORM], tl.nrec), o.krn, 0, 0);
            t.krn[0] = d[0]; t.krn[1] = d[1];
        }
    } else {
        uint32_t kv[4], vv[4], rv[4];
        auto rk = make_rsrc(tl.base[R_KNORM], nrec(R_KNORM));
        auto rvn = make_rsrc(tl.base[R_VNORM], nrec(R_VNORM));
        auto rrn = make_rsrc(tl.base[R_KRNORM], nrec(R_KRNORM));
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if (MASKED) {
                kv[r] = __builtin_amdgcn_raw_buffer_load_b16(rk, o.kn + r * rrow[R_KNORM], 0, 0);
                vv[r] = __builtin_amdgcn_raw_buffer_load_b16(rvn, o.vn + r * rrow[R_VNORM], 0, 0);
                if (KQJL) rv[r] = __builtin_amdgcn_raw_buffer_load_b16(rrn, o.krn + r * rrow[R_KRNORM], 0, 0);
            } else {
                kv[r] = __builtin_amdgcn_raw_buffer_load_b16(rk, o.kn, sgpr(r * rrow[R_KNORM]), 0);
                vv[r] = __builtin_amdgcn_raw_buffer_load_b16(rvn, o.vn, sgpr(r * rrow[R_VNORM]), 0);
                if (KQJL) rv[r] = __builtin_amdgcn_raw_buffer_load_b16(rrn, o.krn, sgpr(r * rrow[R_KRNORM]), 0);
            }
        }
        // Kept one word per token unless NV (then combined: only the masked path gets here).
#pragma unroll
        for (int r = 0; r < (NV ? 2 : 4); ++r) {
            t.kn[r] = NV ? (kv[2 * r] | (kv[2 * r + 1] << 16)) : kv[r];
            t.vn[r] = NV ? (vv[2 * r] | (vv[2 * r + 1] << 16)) : vv[r];
            if (KQJL) t.krn[r] = NV ? (rv[2 * r] | (rv[2 * r + 1] << 16)) : rv[r];
        }
    }
    auto rv = make_rsrc(tl.base[R_VIDX], nrec(R_VIDX));
    if (!MASKED && v_lg) {
        // values tile layout: the lane's chunk (4 * VB bytes) in one load
        if (VB == 2) {
            tq_u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(rv, o.vidx, 0, 0);
            t.vw[0][0] = w[0];
            t.vw[1][0] = w[1];
        } else if (VB == 3) {
            typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
            u32x3 w = __builtin_amdgcn_raw_buffer_load_b96(rv, o.vidx, 0, 0);
            t.vw[0][0] = w[0];
            t.vw[1][0] = w[1];
            t.vw[2][0] = w[2];
        } else {
            tq_u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rv, o.vidx, 0, 0);
            t.vw[0][0] = w[0];
            t.vw[1][0] = w[1];
            t.vw[2][0] = w[2];
            t.vw[3][0] = w[3];
        }
        return;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint32_t off = MASKED ? o.vidx + r * vstep : o.vidx;
        if (VB == 3) {
            const int soff = MASKED ? 0 : sgpr(r * vstep);
            tq_u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(rv, off, soff, 0);
            t.vw[r][0] = w[0];
            t.vw[r][VB == 3 ? 1 : 0] = w[1];
            continue;
        }
        const int soff = MASKED ? 0 : sgpr(r * vstep);
        if (VB == 4) {
            t.vw[r][0] = __builtin_amdgcn_raw_buffer_load_b32(rv, off, soff, 0);
        } else {
            t.vw[r][0] = __builtin_amdgcn_raw_buffer_load_b16(rv, off, soff, 0);
        }
    }
}

// Online-softmax state of one wave.
struct SoftmaxState {
    float m, lsum;
    tq_floatx4 acc[8];
    uint32_t n_skip, n_tot;  // wave-uniform (built from ballots)
};

// Max / sum of a value over the four lanes l, l^16, l^32, l^48 (VALU lane swaps, no LDS pipe).
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

// Scores of one tile (log2 units; rows at or past nvalid are -inf) and their max over the
// lane's head column.  kbank: LDS byte address of the lane's bank replica in the K pair table;
// one = 0x3C003C00 (half2 of 1.0) held in a vector register.
template <int KB, bool KQJL, int VB, bool NV, bool QCOLS, bool FULL>
__device__ __forceinline__ float tile_scores(const TileRaw<KB, KQJL, VB, NV>& cur, int nvalid,
                                             const tq_half8 (&qop)[4], const tq_half8 (&qlo)[QCOLS ? 1 : 4],
                                             const tq_half8 (&qpop)[KQJL ? 4 : 1], float qpm, uint32_t kbank,
                                             uint32_t one, int g, float (&sc)[4]) {
    // ---------------- QK products ----------------
    tq_floatx4 s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
        tq_u32x4 a;
#pragma unroll
        for (int j = 0; j < 4; ++j) a[j] = lds_read(pair_addr<2 * KB>(cur.kw, 2 * KB * (4 * cc + j), kbank));
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
                // fp16 sign bits: bit pp of the lane's signs (low half), bit pp + 16 (high half)
                const int pp = 4 * cc + j;
                a[j] = ((cur.ks << (15 - pp)) & 0x80008000u) | one;
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
        // column n (hi part of q) + column n ^ 8 (lo part): rotate each 16-lane row by 8 (DPP)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            s1v[r] += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(s1v[r]), 0x128, 0xf, 0xf, true));
    }

    // score = norm * S (+ rnorm * qpm * QJL: corr_scale and the operand scale 2^-e in qpm)
    float mt = kNegInf;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        float v = norm_at<NV>(cur.kn, r) * s1v[r];
        if (KQJL) v = __builtin_fmaf(norm_at<NV>(cur.krn, r) * qpm, s2v[r], v);
        sc[r] = (FULL || 4 * g + r < nvalid) ? v : kNegInf;
        mt = fmaxf(mt, sc[r]);
    }
    return max_over_groups(mt);
}

// One tile: scores, online softmax, Sparse-V, PV.  FULL: all 16 rows valid (no masking).
// vbank: LDS byte address of the lane's bank replica in the V pair table.  m_blk (> -inf when
// the KV block spans two tiles): the running max through the end of the tile's block, which the
// Sparse-V test then uses instead of the max through this tile.
template <int KB, bool KQJL, int VB, bool NV, bool QCOLS, bool FULL>
__device__ __forceinline__ void compute_tile(const TileRaw<KB, KQJL, VB, NV>& cur, int nvalid, SoftmaxState& st,
                                             const tq_half8 (&qop)[4], const tq_half8 (&qlo)[QCOLS ? 1 : 4],
                                             const tq_half8 (&qpop)[KQJL ? 4 : 1], float qpm, uint32_t kbank, uint32_t vbank,
                                             uint32_t one, const LaneOff& o, int g, uint64_t hmask,
                                             uint64_t gmask, const DecodeParams& p, bool sparse, bool count, float m_blk) {
    // ---------------- online softmax ----------------
    float sc[4];
    const float mt = tile_scores<KB, KQJL, VB, NV, QCOLS, FULL>(cur, nvalid, qop, qlo, qpop, qpm, kbank, one, g, sc);
    const float m_new = fmaxf(st.m, mt);
    const float mref = m_new == kNegInf ? 0.f : m_new;
    float pr[4];
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        pr[r] = __builtin_amdgcn_exp2f(sc[r] - mref);  // 0 for rows past the end
        psum += pr[r];
    }
    // Rescale only when some head's running max moved (alpha == 1 otherwise).
    if (__builtin_amdgcn_ballot_w64(m_new > st.m) & hmask) {
        const float alpha = __builtin_amdgcn_exp2f(st.m - mref);
        st.lsum *= alpha;
#pragma unroll
        for (int i = 0; i < 8; ++i) st.acc[i] *= alpha;
    }
    st.lsum += psum;
    st.m = m_new;

    // P * vnorm; rows past the end may hold any bits in a paged block, so they are zeroed.
    float pv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        pv[r] = norm_at<NV>(cur.vn, r) * pr[r];
        if (!FULL) pv[r] = 4 * g + r < nvalid ? pv[r] : 0.f;
    }
    // Sparse-V: token 4g + r is kept when some head of the group has p > thresh, i.e. when
    // lane group g of the ballot is non-zero (gmask: the 16 lanes of this lane's group).
    if (sparse) {
        uint64_t orall = 0;
        uint32_t nsig = 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const bool pass = p.sparse_pair ? sc[r] > m_blk + p.log2_thresh : pr[r] > p.thresh;
            const uint64_t bal = __builtin_amdgcn_ballot_w64(pass) & hmask;
            orall |= bal;
            const bool keep = (bal & gmask) != 0;
            pv[r] = keep ? pv[r] : 0.f;
            if (count) nsig += (uint32_t)__builtin_popcountll(__builtin_amdgcn_ballot_w64(keep) & 0x0001000100010001ull);
        }
        if (count) {
            const uint32_t nv = FULL ? 16u : (uint32_t)nvalid;
            st.n_tot += nv;
            st.n_skip += nv - nsig;
        }
        if (orall == 0) return;
    }

    // ---------------- PV product ----------------
    tq_u32x2 bw = {tq_pack_half2(pv[0], pv[1]), tq_pack_half2(pv[2], pv[3])};
    const tq_half4 bop = __builtin_bit_cast(tq_half4, bw);
    if (NV && p.v_lg) {
        // values tile layout: field group a of the chunk is dim 8n + a of tokens 4g..4g+3, two
        // pair lookups give the A operand directly
        uint32_t cw[VB];
#pragma unroll
        for (int k = 0; k < VB; ++k) cw[k] = cur.vw[k][0];
#pragma unroll
        for (int a = 0; a < 8; ++a) {
            const tq_u32x2 aw = {lds_read(pair_addr<2 * VB>(cw, 4 * VB * a, vbank)),
                                 lds_read(pair_addr<2 * VB>(cw, 4 * VB * a + 2 * VB, vbank))};
            st.acc[a] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(tq_half4, aw), bop, st.acc[a], 0, 0, 0);
        }
        return;
    }
    uint32_t w[4][1];
#pragma unroll
    for (int r = 0; r < 4; ++r)
        w[r][0] = VB == 3 ? __builtin_amdgcn_perm(cur.vw[r][VB == 3 ? 1 : 0], cur.vw[r][0], o.vsel) : cur.vw[r][0];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        // dims 8n+2q, 8n+2q+1 of tokens 4g..4g+3
        uint32_t vp[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) vp[r] = lds_read(pair_addr<2 * VB>(w[r], 2 * VB * q, vbank));
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
// Tiles in flight per wave (register ring) and waves per SIMD (2 for the 16-column variants
// with QJL keys and 3-bit values, whose registers do not fit 3).
constexpr int kDepth = 2;

template <int KB, bool KQJL, int VB, bool QCOLS>
constexpr int decode_waves() {
    return (!QCOLS && KQJL && VB == 3 && KB >= 3) ? 2 : 3;
}

template <int KB, bool KQJL, int VB, bool QCOLS, bool NV>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(decode_waves<KB, KQJL, VB, QCOLS>(),
                                                                     decode_waves<KB, KQJL, VB, QCOLS>())))
void decode_kernel(DecodeParams p) {
    constexpr int KENT = 1 << (2 * KB);
    constexpr int VENT = 1 << (2 * VB);
    // Dynamic LDS only (no static LDS in this kernel): s_lds sits at LDS address 0.  The larger
    // table goes first, so each table's address is a multiple of its size (see pair_addr).
    // K and V share one table when they use the same codebook (p.share_tab).
    extern __shared__ uint32_t s_lds[];
    uint32_t* s_ktab = (KENT >= VENT || p.share_tab) ? s_lds : s_lds + VENT * 32;
    uint32_t* s_vtab = p.share_tab ? s_lds : (KENT >= VENT ? s_lds + KENT * 32 : s_lds);

    // Pair tables: entry e -> half2(c[e & (2^b - 1)], c[e >> b]) * cscale, 32 bank replicas.
    for (int i = threadIdx.x; i < KENT * 32; i += 256) {
        int e = i >> 5;
        s_ktab[i] = tq_pack_half2(p.k_cent[e & ((1 << KB) - 1)] * p.k_cscale, p.k_cent[e >> KB] * p.k_cscale);
    }
    if (!p.share_tab) {
        for (int i = threadIdx.x; i < VENT * 32; i += 256) {
            int e = i >> 5;
            s_vtab[i] = tq_pack_half2(p.v_cent[e & ((1 << VB) - 1)] * p.v_cscale, p.v_cent[e >> VB] * p.v_cscale);
        }
    }
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int g = lane >> 4;   // lane group: dims 32g.. (K), tokens 4g..4g+3 (scores, V)
    const int n = lane & 15;   // head column (Q/P/out), token row (K loads), dim row (V)
    const uint32_t bank4 = 4u * (uint32_t)(lane & 31);
    const uint32_t kbank = (uint32_t)(uintptr_t)(lds_u32*)s_ktab + bank4;
    const uint32_t vbank = (uint32_t)(uintptr_t)(lds_u32*)s_vtab + bank4;
    uint32_t one;  // half2(1, 1) in a vector register: lets the sign operand build use one and-or
    asm("v_mov_b32 %0, 0x3c003c00" : "=v"(one));

    // The wave index is uniform across the wave; saying so keeps every per-unit value in SGPRs
    // (otherwise buffer descriptors built from it are treated as divergent).
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // Units in (sequence, chunk, KV head) order: the four waves of a workgroup (which holds its
    // CU slot until all four finish) get the same chunk of one sequence, so equal work.
    const int64_t unit = (int64_t)blockIdx.x * 4 + wave;
    const int kh = (int)(unit % p.hkv);
    const int64_t sc = unit / p.hkv;
    const int c = (int)(sc % p.n_chunks);
    const int64_t s = sc / p.n_chunks;
    if (s >= p.num_seqs) return;

    int L = tq_seq_len(p.seq_lens, s, p.uniform_len);
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
    float qpm = 0.f;  // QJL products of this lane's head -> log2 units (undoes the operand scale)
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
        // q x H: elements 32g + i (or, for permuted signs, 4i + g) over lane groups g
        if (p.rot_q) tq_wht_row_g4(qv, p.wht_h);
        if (KQJL && p.rot_qp) tq_wht_row_g4(qpv, p.wht_h);
        // The QJL operand is q_proj * 2^e in fp16, e per head (column) so that the head's largest
        // |q_proj| lands in [2^12, 2^13): a head with a small q_proj stays out of the fp16
        // subnormals.  sm_scale * log2(e) * corr_scale * 2^-e is applied to the fp32 products.
        int qpe = 0;
        if (KQJL) {
            float amax = 0.f;
#pragma unroll
            for (int k = 0; k < 32; ++k) amax = fmaxf(amax, fabsf(qpv[k]));
            amax = max_over_groups(amax);  // lanes (n, g), g = 0..3: the four quarters of head n
            if (amax > 0.f && amax < __builtin_huge_valf()) qpe = 12 - ilogbf(amax);
            qpe = qpe < -100 ? -100 : (qpe > 100 ? 100 : qpe);
            qpm = ldexpf(p.qp_scale * p.corr_scale, -qpe);
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
                    qpop[cc % (KQJL ? 4 : 1)][j] = (_Float16)(-ldexpf(qpv[bit], qpe));
                }
            }
        }
    }

    // ---- loop-invariant per-lane byte offsets inside a tile ----
    LaneOff o;
    // (lane-grouped tiles always have their norm rows 2 bytes apart: NV instances only)
    if (NV && p.k_lg) {
        // chunk (4n + g) of the 16-row sub-tile: index dwords, then the sign dword
        o.kidx = (uint32_t)((4 * n + g) * (4 * KB + (KQJL ? 4 : 0)));
        o.ksig = o.kidx + 4u * KB;
    } else {
        o.kidx = (uint32_t)(n * p.rrow[R_KIDX] + 4 * KB * g);
        o.ksig = (uint32_t)(n * p.rrow[R_KSIG] + 4 * g);
    }
    o.kn = (uint32_t)(4 * g * p.rrow[R_KNORM]);
    o.krn = (uint32_t)(4 * g * p.rrow[R_KRNORM]);
    o.vn = (uint32_t)(4 * g * p.rrow[R_VNORM]);
    if (NV && p.v_lg) {
        // chunk (16g + n) of the 16-row sub-tile, read whole
        o.vidx = (uint32_t)((16 * g + n) * 4 * VB);
        o.vsel = 0;
    } else {
        int start = VB * n;
        o.vsel = 0;
        if (VB == 3) {
            // 8-byte window at a 4-byte boundary, kept inside the 48-byte row; the field starts
            // at byte b (0..5) of it and v_perm picks bytes b..b+2 (selector 0x0c: zero byte)
            const int byte0 = 3 * n;
            start = (byte0 >> 2) << 2;
            start = start < 40 ? start : 40;
            const uint32_t b = (uint32_t)(byte0 - start);
            o.vsel = b | ((b + 1) << 8) | ((b + 2) << 16) | 0x0c000000u;
        }
        o.vidx = (uint32_t)(4 * g * p.rrow[R_VIDX] + start);
    }
    // Per-unit part of every region's address.
    const uint8_t* ub[R_COUNT];
#pragma unroll
    for (int r = 0; r < R_COUNT; ++r) ub[r] = p.rptr[r] + kh * p.rhead[r] + (paged ? 0 : s * p.rseq[r]);

    // Tile at t0: region bases and record count.  live = false (a tile past the end) and an
    // unreadable block entry give nrec = 0, so the loads return zeros: every fetch issues the
    // same loads, which keeps the compiler's outstanding-load counts exact and lets the
    // prefetched tiles stay in flight.  Block-table entries are wave-uniform scalar loads.
    const int nblk_seq = (L + p.block_size - 1) / p.block_size;  // >= 1
    const int32_t* bt_row = paged ? p.bt + s * p.bt_stride : nullptr;
    auto locate = [&](int t0, bool live, Tile& tl) {
        tl.nvalid = live ? ((t_end - t0 < 16) ? t_end - t0 : 16) : 0;
        tl.nrec = live ? 0x7fffffffu : 0u;
        int64_t offk = 0, offv = 0;
        int rowbase = t0;
        if (paged) {
            int lb = t0 / p.block_size;
            lb = lb < nblk_seq ? lb : nblk_seq - 1;
            rowbase = t0 - lb * p.block_size;
            int64_t blk = bt_row[lb];
            if (blk < 0 || blk >= p.num_blocks) {
                blk = 0;
                tl.nvalid = 0;
                tl.nrec = 0;
            }
            offk = blk * p.sb_k;
            offv = blk * p.sb_v;
        }
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
    const uint64_t hmask = __builtin_amdgcn_ballot_w64(hvalid);  // lanes of real heads
    const uint64_t gmask = 0xffffull << (16 * g);                  // this lane's 16-lane group

    auto fetch = [&](int t0, bool live, TileRaw<KB, KQJL, VB, NV>& raw, int& nvalid) {
        Tile tl;
        locate(t0, live, tl);
        nvalid = tl.nvalid;
        load_tile<KB, KQJL, VB, NV, false>(raw, tl, o, p.rrow, p.vstep, NV && p.v_lg);
    };

    // Tiles 0..nfull-1 are complete.  A paged cache allocates whole blocks, so its partial last
    // tile is loaded whole (and prefetched like the others); in a contiguous layout it is loaded
    // with masking after the loop.  The partial tile is computed with row masking.
    // Loads run kDepth - 1 tiles ahead of the compute through a ring of kDepth register tiles;
    // tile T lives in slot T % kDepth.
    constexpr int D = kDepth;
    static_assert(D == 2, "the KV-block max look-ahead reads the next tile from the other ring slot");
    const bool blk2 = sparse && p.sparse_pair;  // (paged: the partial last tile is in the ring)
    float m_blk = kNegInf;
    const int ntiles = (t_end - t_begin + 15) >> 4;
    const int nfull = (t_end - t_begin) >> 4;
    const int nload = paged ? ntiles : nfull;
    TileRaw<KB, KQJL, VB, NV> ring[D];
    int nv[D];
#pragma unroll
    for (int k = 0; k < D - 1; ++k) fetch(t_begin + 16 * k, k < nload, ring[k], nv[k]);
    for (int i = 0; i < nfull; i += D) {
        bool done = false;
#pragma unroll
        for (int k = 0; k < D; ++k) {
            const int t = i + k;
            if (t >= nfull) {
                done = true;
                break;
            }
            const int ahead = t + D - 1;
            fetch(t_begin + 16 * ahead, ahead < nload, ring[(k + D - 1) % D], nv[(k + D - 1) % D]);
            if (blk2 && k == 0) {
                // first tile of a 32-token KV block: the block's max from this tile and the next
                // (already fetched into the other ring slot; a tile past the end scores -inf)
                float sc[4];
                const float ma = tile_scores<KB, KQJL, VB, NV, QCOLS, true>(ring[0], nv[0], qop, qlo, qpop, qpm, kbank,
                                                                            one, g, sc);
                const float mb = tile_scores<KB, KQJL, VB, NV, QCOLS, false>(ring[1 % D], t + 1 < ntiles ? nv[1 % D] : 0,
                                                                             qop, qlo, qpop, qpm, kbank, one, g, sc);
                m_blk = fmaxf(sm.m, fmaxf(nv[0] ? ma : kNegInf, mb));
            }
            if (nv[k])
                compute_tile<KB, KQJL, VB, NV, QCOLS, true>(ring[k], nv[k], sm, qop, qlo, qpop, qpm, kbank, vbank, one, o,
                                                            g, hmask, gmask, p, sparse, count, m_blk);
        }
        if (done) break;
    }
    if (nfull < ntiles) {
        TileRaw<KB, KQJL, VB, NV> tr;
        int tv;
        if (paged) {
            const int slot = nfull % D;
            tr = ring[0];
            tv = nv[0];
#pragma unroll
            for (int k = 1; k < D; ++k)
                if (slot == k) {
                    tr = ring[k];
                    tv = nv[k];
                }
        } else {
            Tile tl;
            locate(t_begin + 16 * nfull, true, tl);
            tv = tl.nvalid;
            load_tile<KB, KQJL, VB, NV, true>(tr, tl, o, p.rrow, p.vstep, NV && p.v_lg);
        }
        if (blk2 && (nfull & 1) == 0) {
            // a partial tile that starts a KV block ends it too
            float sc[4];
            m_blk = fmaxf(sm.m, tile_scores<KB, KQJL, VB, NV, QCOLS, false>(tr, tv, qop, qlo, qpop, qpm, kbank, one, g, sc));
        }
        if (tv)
            compute_tile<KB, KQJL, VB, NV, QCOLS, false>(tr, tv, sm, qop, qlo, qpop, qpm, kbank, vbank, one, o, g, hmask,
                                                         gmask, p, sparse, count, m_blk);
    }

    const float lsum = sum_over_groups(sm.lsum);
    if (count && lane == 0) {
        atomicAdd(p.skip_stats, (unsigned long long)sm.n_skip);
        atomicAdd(p.skip_stats + 1, (unsigned long long)sm.n_tot);
    }
    // acc[nn][r] is dim 8*(4g+r)+nn = 32g + 8r + nn; v_cinv undoes the V table scale.
    const float vs = p.v_cinv;
    int nch = (L + p.chunk - 1) / p.chunk;
    nch = nch < p.n_chunks ? nch : p.n_chunks;  // tokens past max_seq_len are not processed

    // the only chunk: normalise and write the output directly (a rotated output is written by
    // decode_reduce_kernel, which takes single chunks too)
    if (nch == 1 && !p.rot_out) {
        if (hvalid) {
            const float inv = lsum > 0.f ? vs / lsum : 0.f;
            const int64_t ob = s * p.out_ss + (int64_t)head * p.out_sh + 32 * g;
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int nn = 0; nn < 8; ++nn) tq_store1(p.out, ob + 8 * r + nn, p.out_dtype, sm.acc[nn][r] * inv);
        }
        return;
    }

    // Partial results of this chunk: (m, l, acc) per head.
    if (hvalid) {
        const int64_t slot = ((s * p.hq + head) * (int64_t)p.n_chunks + c);
        if (g == 0) {
            p.ws_m[slot] = sm.m;
            p.ws_l[slot] = lsum;
        }
        float4* dst = reinterpret_cast<float4*>(p.ws_acc + slot * TQ_HEAD_DIM + 32 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            dst[2 * r] = make_float4(sm.acc[0][r] * vs, sm.acc[1][r] * vs, sm.acc[2][r] * vs, sm.acc[3][r] * vs);
            dst[2 * r + 1] = make_float4(sm.acc[4][r] * vs, sm.acc[5][r] * vs, sm.acc[6][r] * vs, sm.acc[7][r] * vs);
        }
    }
}

struct ReduceParams {
    const float* ws_acc;
    const float* ws_m;
    const float* ws_l;
    int num_seqs, hq, n_chunks, chunk, cap;
    const int32_t* seq_lens;  // null: every sequence holds uniform_len tokens
    int uniform_len;
    void* out;
    int out_dtype;
    int64_t out_ss, out_sh;
    int rot_out;  // write out x H
    float wht_h;
    // balanced schedule: partial rows [slot][group][128] located through the decode kernel's plan
    int balanced, n_workers, hkv, group, len_cap;
    const int64_t* plan;
};

// Split-K merge, W waves per (sequence, query head):
//   out = sum_c 2^(m_c - M) acc_c / sum_c 2^(m_c - M) l_c      (kernels/attention.py:128-140)
// The chunk maxima and denominators are read one lane per chunk and reduced across the wave;
// the rows acc_c are summed in chunk order with lane d covering dims 2d, 2d+1, sixteen chunks
// (rows, maxima, denominators) requested together.  With W > 1 (many chunks per sequence) wave w
// takes batches w, w + W, ... and wave 0 combines the W partial merges through LDS, so the
// batches' load rounds overlap.  Sequences of one chunk were written by the decode kernel
// (unless the output is rotated: then every sequence is written here); empty ones are written
// as zero here.
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
    return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, 64);
    return x;
}

template <int W>
__global__ __launch_bounds__(64 * W) void decode_reduce_kernel(ReduceParams p) {
    const int64_t sh = blockIdx.x;
    const int64_t s = sh / p.hq;
    const int h = (int)(sh - s * p.hq);
    const int lane = threadIdx.x & 63;
    const int wave = W == 1 ? 0 : __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    int nch;
    int64_t base, stride;  // partial row of the first piece, rows between pieces
    if (!p.balanced) {
        int L = tq_seq_len(p.seq_lens, s, p.uniform_len);
        L = L < p.cap ? L : p.cap;
        nch = L > 0 ? (L + p.chunk - 1) / p.chunk : 0;
        nch = nch < p.n_chunks ? nch : p.n_chunks;  // tokens past max_seq_len were not processed
        if (nch == 1 && !p.rot_out) return;
        base = sh * p.n_chunks;
        stride = 1;
    } else {
        // the workers w0..w1 that hold segment (s, kh): partial slots w0 + g .. w1 + g
        const int kh = h / p.group;
        const int np = tq_bal_pairs(tq_seq_len(p.seq_lens, s, p.uniform_len), p.len_cap);
        nch = 0;
        base = 0;
        stride = p.group;
        if (np > 0) {
            const int64_t P = p.plan[0] * p.hkv;
            const int64_t R = P < p.n_workers ? P : (int64_t)p.n_workers;
            const int64_t x0 = p.plan[1 + s] * p.hkv + (int64_t)kh * np;
            const int64_t w0 = tq_bal_worker(x0, P, R);
            const int64_t w1 = tq_bal_worker(x0 + np - 1, P, R);
            if (w0 == w1 && !p.rot_out) return;  // written by the decode kernel
            nch = (int)(w1 - w0 + 1);
            base = (w0 + s * p.hkv + kh) * p.group + (h - kh * p.group);
        }
    }
    // Batches of 16 chunks: the batch's rows, maxima and denominators are all requested before
    // any of them is used (the rows do not depend on the maxima), so a batch costs one load
    // round.  Per batch the running max M rescales what was summed so far.
    float M = kNegInf, den = 0.f, a0 = 0.f, a1 = 0.f;
    const float2* rows = reinterpret_cast<const float2*>(p.ws_acc + base * TQ_HEAD_DIM) + lane;
    for (int c0 = 16 * wave; c0 < nch; c0 += 16 * W) {
        const int nb = nch - c0 < 16 ? nch - c0 : 16;
        const bool mine = lane < nb;
        const float mc = mine ? p.ws_m[base + (int64_t)(c0 + lane) * stride] : kNegInf;
        const float lc = mine ? p.ws_l[base + (int64_t)(c0 + lane) * stride] : 0.f;
        float2 v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j)
            v[j] = j < nb ? rows[(int64_t)(c0 + j) * stride * (TQ_HEAD_DIM / 2)] : make_float2(0.f, 0.f);
        const float Mb = wave_max(mc);
        const float Mn = fmaxf(M, Mb);
        if (Mn == kNegInf) continue;  // every chunk so far empty
        const float alpha = M == kNegInf ? 0.f : __builtin_amdgcn_exp2f(M - Mn);
        den *= alpha;
        a0 *= alpha;
        a1 *= alpha;
        M = Mn;
        const float w = mine ? __builtin_amdgcn_exp2f(mc - M) : 0.f;
        den += wave_sum(w * lc);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), j));
            a0 = __builtin_fmaf(wj, v[j].x, a0);
            a1 = __builtin_fmaf(wj, v[j].y, a1);
        }
    }
    if (W > 1) {
        __shared__ float s_m[W], s_den[W];
        __shared__ float2 s_acc[W][64];
        if (lane == 0) {
            s_m[wave] = M;
            s_den[wave] = den;
        }
        s_acc[wave][lane] = make_float2(a0, a1);
        __syncthreads();
        if (wave != 0) return;
        float Mt = kNegInf;
#pragma unroll
        for (int w = 0; w < W; ++w) Mt = fmaxf(Mt, s_m[w]);
        den = 0.f;
        a0 = 0.f;
        a1 = 0.f;
        if (Mt != kNegInf) {
#pragma unroll
            for (int w = 0; w < W; ++w) {
                const float f = s_m[w] == kNegInf ? 0.f : __builtin_amdgcn_exp2f(s_m[w] - Mt);
                den = __builtin_fmaf(f, s_den[w], den);
                a0 = __builtin_fmaf(f, s_acc[w][lane].x, a0);
                a1 = __builtin_fmaf(f, s_acc[w][lane].y, a1);
            }
        }
    }
    float inv = den > 0.f ? 1.0f / den : 0.f;
    if (p.rot_out) {
        // element 2 lane + e: bit 0 in registers, bits 1-6 over the lanes
        const float b0 = a0 + a1, b1 = a0 - a1;
        a0 = b0;
        a1 = b1;
#pragma unroll
        for (int m = 1; m < 64; m <<= 1) {
            a0 = tq_wht_lane(a0, m);
            a1 = tq_wht_lane(a1, m);
        }
        inv *= p.wht_h;
    }
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

size_t lds_bytes(int kb, int vb, int share) {
    return ((size_t)1 << (2 * kb)) * 32 * 4 + (share ? 0 : ((size_t)1 << (2 * vb)) * 32 * 4);
}

// The decode_kernel instance for a configuration (nullptr: unsupported bit widths).
const void* decode_kernel_ptr(int kb, bool kq, int vb, bool qcols, bool nv) {
#define TQ_KP(KB, KQ, VB)                                                                          \
    if (kb == KB && kq == KQ && vb == VB)                                                          \
        return qcols ? (nv ? (const void*)decode_kernel<KB, KQ, VB, true, true>                    \
                           : (const void*)decode_kernel<KB, KQ, VB, true, false>)                  \
                     : (nv ? (const void*)decode_kernel<KB, KQ, VB, false, true>                   \
                           : (const void*)decode_kernel<KB, KQ, VB, false, false>);
#define TQ_KP_V(KB, KQ) TQ_KP(KB, KQ, 2) TQ_KP(KB, KQ, 3) TQ_KP(KB, KQ, 4)
    TQ_KP_V(2, false) TQ_KP_V(2, true) TQ_KP_V(3, false) TQ_KP_V(3, true) TQ_KP_V(4, false) TQ_KP_V(4, true)
#undef TQ_KP_V
#undef TQ_KP
    return nullptr;
}

bool q_vector_ok(const void* q, int dtype, int64_t ss, int64_t sh) {
    const int64_t es = dtype == TQ_F32 ? 4 : 2;
    return aligned(q, 16) && (ss * es) % 16 == 0 && (sh * es) % 16 == 0;
}

int launch_reduce(float* ws_acc, float* ws_m, float* ws_l, int num_seqs, int num_q_heads, int n_chunks, int chunk,
                  int cap, const int32_t* seq_lens, int uniform_len, void* out, int out_dtype, int64_t out_ss,
                  int64_t out_sh, int rot_out, hipStream_t st, const FastDecodeParams* bal = nullptr) {
    ReduceParams rp = {};
    if (bal) {
        rp.balanced = 1;
        rp.n_workers = bal->n_workers;
        rp.hkv = bal->hkv;
        rp.group = bal->group;
        rp.len_cap = bal->len_cap;
        rp.plan = bal->plan;
    }
    rp.rot_out = rot_out;
    rp.wht_h = kWhtH;
    rp.ws_acc = ws_acc;
    rp.ws_m = ws_m;
    rp.ws_l = ws_l;
    rp.num_seqs = num_seqs;
    rp.hq = num_q_heads;
    rp.n_chunks = n_chunks;
    rp.chunk = chunk;
    rp.cap = cap;
    rp.seq_lens = seq_lens;
    rp.uniform_len = uniform_len;
    rp.out = out;
    rp.out_dtype = out_dtype;
    rp.out_ss = out_ss;
    rp.out_sh = out_sh;
    // one wave per batch of 16 chunks, up to sixteen, so a sequence's batches load in one round
    // (2, 4, 8 or 16 waves per (sequence, query head) beyond 16, 32, 64 or 128 chunks)
    const unsigned nsh = (unsigned)((int64_t)num_seqs * num_q_heads);
    if (!bal && n_chunks > 128)
        hipLaunchKernelGGL(decode_reduce_kernel<16>, dim3(nsh), dim3(1024), 0, st, rp);
    else if (!bal && n_chunks > 64)
        hipLaunchKernelGGL(decode_reduce_kernel<8>, dim3(nsh), dim3(512), 0, st, rp);
    else if (!bal && n_chunks > 32)
        hipLaunchKernelGGL(decode_reduce_kernel<4>, dim3(nsh), dim3(256), 0, st, rp);
    else if (!bal && n_chunks > 16)
        hipLaunchKernelGGL(decode_reduce_kernel<2>, dim3(nsh), dim3(128), 0, st, rp);
    else
        hipLaunchKernelGGL(decode_reduce_kernel<1>, dim3(nsh), dim3(64), 0, st, rp);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TQ_OK : (int)e;
}

// The fast kernel reads this library's tile layout: per cache one block stride and one head
// stride for all regions, rows of 16*bits index bytes, 16 sign bytes and 2-byte norms, the
// other regions after the index region of the same tile.  *addr: TQ_ADDR_BIG when some tile
// lies 2 GiB or more from its head's base (64-bit per-tile addressing), else TQ_ADDR_STREAM when
// the two caches together are larger than the last-level cache, else TQ_ADDR_CACHED.
bool fast_path_ok(const tq_kv_view* k, const tq_kv_view* v, int group, int block_size, int64_t num_blocks,
                  const int32_t* block_tables, int* addr) {
    // num_blocks >= 1: unreadable table entries are redirected to block 0 and masked
    if (!block_tables || num_blocks < 1 || group > 8 || k->signs_permuted) return false;
    if (block_size & (block_size - 1)) return false;  // 16 << tile_shift
    auto same = [](const tq_region& a, const tq_region& b) {
        return a.stride_block == b.stride_block && a.stride_head == b.stride_head;
    };
    auto delta_ok = [](const tq_region& base, const tq_region& r, int64_t rows_bytes) {
        const int64_t d = static_cast<const uint8_t*>(r.ptr) - static_cast<const uint8_t*>(base.ptr);
        return d >= 0 && d + rows_bytes < (1ll << 30);
    };
    const int64_t bs = block_size;
    if (k->layout != TQ_TILE_KEYS || v->layout != TQ_TILE_VALUES) return false;
    if (k->idx.stride_row != 16 * k->bits + (k->qjl ? 16 : 0) || k->norm.stride_row != 2 || !same(k->idx, k->norm))
        return false;
    if (!delta_ok(k->idx, k->norm, 2 * bs)) return false;
    if (k->qjl) {
        if (k->rnorm.stride_row != 2 || !same(k->idx, k->rnorm)) return false;
        if (!delta_ok(k->idx, k->rnorm, 2 * bs)) return false;
    }
    if (v->idx.stride_row != 16 * v->bits || v->norm.stride_row != 2 || !same(v->idx, v->norm)) return false;
    if (!delta_ok(v->idx, v->norm, 2 * bs)) return false;
    auto stride_ok = [&](const tq_region& r) { return r.stride_block > 0 && r.stride_block < (1ll << 30); };
    if (!stride_ok(k->idx) || !stride_ok(v->idx)) return false;
    auto small = [&](const tq_region& r) { return num_blocks * r.stride_block < (1ll << 31) - (1ll << 16); };
    const int64_t extent = num_blocks * (k->idx.stride_block + v->idx.stride_block);
    *addr = !(small(k->idx) && small(v->idx)) ? TQ_ADDR_BIG : extent > kTqStreamBytes ? TQ_ADDR_STREAM : TQ_ADDR_CACHED;
    return true;
}

// decode_contig_kernel reads the reference's row-major per-sequence arrays: no block tables, 2-bit
// keys with QJL and 2-bit values, rows following each other (16-row block strides) of 32 index
// bytes, 16 sign bytes and 2-byte norms, aligned for its 8-byte loads, whole 16-row tiles up to
// max_seq_len (the rows each sequence holds), GQA groups of at most 8, no Sparse-V, no rotation.
bool contig_path_ok(const tq_kv_view* k, const tq_kv_view* v, int group, const int32_t* block_tables,
                    int block_size, int max_seq_len, int max_blocks_per_seq, float sparse_threshold, int rotate) {
    if (block_tables || block_size != 16 || group > 8 || sparse_threshold > 0.f || rotate) return false;
    if (k->bits != 2 || !k->qjl || v->bits != 2) return false;
    if (k->layout != TQ_TILE_ROWS || v->layout != TQ_TILE_ROWS) return false;
    if (max_seq_len <= 0 || max_seq_len % 16 || max_seq_len > 16 * (int64_t)max_blocks_per_seq) return false;
    auto rows = [&](const tq_region& r, int64_t row, uint64_t align) {
        return r.ptr && r.stride_row == row && r.stride_block == 16 * row && (uintptr_t)r.ptr % align == 0 &&
               (uint64_t)r.stride_seq % align == 0 && (uint64_t)r.stride_head % align == 0 &&
               (int64_t)max_seq_len * row < (1ll << 31);  // 32-bit row offsets
    };
    return rows(k->idx, 32, 8) && rows(k->signs, 16, 4) && rows(k->norm, 2, 8) && rows(k->rnorm, 2, 8) &&
           rows(v->idx, 32, 8) && rows(v->norm, 2, 8);
}

}  // namespace

// Balanced schedule: partial rows for up to 16 resident waves per CU of the largest gfx950
// (256 CUs) at 8 query heads per group, plus one per (sequence, query head).
constexpr int kTqMaxCus = 256;
size_t bal_rows(int num_seqs, int num_q_heads) {
    return (size_t)kTqBalRowsPerCu * kTqMaxCus + (size_t)num_seqs * num_q_heads;
}
size_t bal_plan_bytes(int num_seqs) { return align_up((size_t)(num_seqs + 1) * sizeof(int64_t), 256); }

// Fixed chunks for the general kernel under tokens_per_chunk = 0: as many per sequence as the
// balanced workspace holds (at most one more than its extra rows per (sequence, query head)).
int general_chunk(int num_seqs, int num_q_heads, int max_seq_len, bool pair) {
    const int64_t tiles = max_seq_len > 0 ? (max_seq_len + 15) / 16 : 1;
    int64_t n = 1 + (int64_t)kTqBalRowsPerCu * kTqMaxCus / ((int64_t)num_seqs * num_q_heads);
    n = n < tiles ? n : tiles;
    int64_t c = 16 * ((tiles + n - 1) / n);
    if (pair && c % 32) c += 16;
    return (int)c;
}

// Resident waves of the fast kernel on the current device (one launch's workers), cached per
// (device, kernel, LDS bytes).
int resident_waves(const void* kern, int wg_waves, size_t lds, int* waves) {
    struct Entry {
        int dev;
        const void* kern;
        size_t lds;
        int waves;
    };
    static Entry cache[64];
    static int n_cache = 0;
    static std::mutex mu;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    std::lock_guard<std::mutex> lock(mu);
    for (int i = 0; i < n_cache; ++i)
        if (cache[i].dev == dev && cache[i].kern == kern && cache[i].lds == lds) {
            *waves = cache[i].waves;
            return TQ_OK;
        }
    const int arc = tq_decode_fast_lds_attr(kern);
    if (arc) return arc;
    int blocks = 0, cus = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kern, 64 * wg_waves, lds);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return (int)e;
    *waves = blocks * wg_waves * cus;
    if (*waves < wg_waves) *waves = wg_waves;
    if (n_cache < 64) cache[n_cache++] = Entry{dev, kern, lds, *waves};
    return TQ_OK;
}

extern "C" size_t tq_decode_workspace_bytes(int num_seqs, int num_q_heads, int max_seq_len, int tokens_per_chunk) {
    if (num_seqs <= 0 || num_q_heads <= 0 || tokens_per_chunk < 0) return 0;
    if (tokens_per_chunk == 0) {
        const size_t rows = bal_rows(num_seqs, num_q_heads);
        return bal_plan_bytes(num_seqs) + align_up(rows * TQ_HEAD_DIM * sizeof(float), 256) +
               2 * align_up(rows * sizeof(float), 256);
    }
    const size_t slots = (size_t)num_seqs * num_q_heads * n_chunks_for(max_seq_len, tokens_per_chunk);
    // acc, m, l per (sequence, query head, chunk)
    return align_up(slots * TQ_HEAD_DIM * sizeof(float), 256) + 2 * align_up(slots * sizeof(float), 256);
}

extern "C" int tq_decode_concurrent_units(int k_bits, int k_qjl, int v_bits, int num_q_heads, int num_kv_heads,
                                          int norm_row_bytes, int share_codebook, int* units) {
    if (!units) return TQ_ERR_INVALID_ARGUMENT;
    if (k_bits < 2 || k_bits > 4 || v_bits < 2 || v_bits > 4) return TQ_ERR_BITS;
    if (num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads) return TQ_ERR_GQA;
    const int group = num_q_heads / num_kv_heads;
    if (group > 16) return TQ_ERR_GQA;
    const void* kern = decode_kernel_ptr(k_bits, k_qjl != 0, v_bits, group <= 8, norm_row_bytes == 2);
    if (!kern) return TQ_ERR_BITS;
    const int share = (share_codebook && k_bits == v_bits) ? 1 : 0;
    size_t lds = lds_bytes(k_bits, v_bits, share);
    if (norm_row_bytes == 2 && group <= 8) {
        // the paged fast path (library tile layout): workgroups of tq_decode_fast_wg_waves waves
        FastLdsLayout lay;
        tq_decode_fast_lds_layout(k_bits, k_qjl != 0, v_bits, share != 0, &lay);
        return resident_waves(tq_decode_fast_kernel_ptr(k_bits, k_qjl != 0, v_bits),
                              tq_decode_fast_wg_waves(k_bits, k_qjl != 0, v_bits, lay.total), lay.total, units);
    }
    int blocks = 0, dev = 0, cus = 0;
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kern, 256, lds);
    if (e == hipSuccess) e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return (int)e;
    *units = blocks * 4 * cus;  // 4 units (waves) per 256-thread workgroup
    return TQ_OK;
}

extern "C" int tq_decode_workgroup_waves(int k_bits, int k_qjl, int v_bits, int num_q_heads, int num_kv_heads,
                                         int norm_row_bytes, int share_codebook, int* waves) {
    if (!waves) return TQ_ERR_INVALID_ARGUMENT;
    if (k_bits < 2 || k_bits > 4 || v_bits < 2 || v_bits > 4) return TQ_ERR_BITS;
    if (num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads) return TQ_ERR_GQA;
    const int group = num_q_heads / num_kv_heads;
    if (group > 16) return TQ_ERR_GQA;
    *waves = 4;  // decode_kernel: 256-thread workgroups
    if (norm_row_bytes == 2 && group <= 8) {
        const int share = (share_codebook && k_bits == v_bits) ? 1 : 0;
        FastLdsLayout lay;
        tq_decode_fast_lds_layout(k_bits, k_qjl != 0, v_bits, share != 0, &lay);
        *waves = tq_decode_fast_wg_waves(k_bits, k_qjl != 0, v_bits, lay.total);
    }
    return TQ_OK;
}

// rotate: q (and q_proj when it is q) enter as q x H, the output leaves as out x H.
// Shared by tq_decode, tq_decode_rotated and the fixed-scratch variant (tq_decode_internal.h).
int tq_decode_impl(int rotate, const void* q, int q_dtype, int64_t q_stride_seq, int64_t q_stride_head,
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
    if (tokens_per_chunk < 0 || tokens_per_chunk % 16) return TQ_ERR_CHUNK;  // 0: balanced
    if (q_dtype != TQ_F32 && q_dtype != TQ_F16 && q_dtype != TQ_BF16) return TQ_ERR_DTYPE;
    if (out_dtype != TQ_F32 && out_dtype != TQ_F16 && out_dtype != TQ_BF16) return TQ_ERR_DTYPE;
    if (max_blocks_per_seq < 0 || num_blocks < 0) return TQ_ERR_INVALID_ARGUMENT;
    if (num_seqs == 0) return TQ_OK;
    if (!q || !out || !k->centroids || !v->centroids) return TQ_ERR_INVALID_ARGUMENT;
    if (!seq_lens && max_seq_len <= 0) return TQ_ERR_INVALID_ARGUMENT;  // null lengths: max_seq_len each
    if (block_tables && block_table_stride < max_blocks_per_seq) return TQ_ERR_INVALID_ARGUMENT;
    // lane-grouped tiles: keys as TQ_TILE_KEYS, values as TQ_TILE_VALUES, paged, natural sign
    // order, the payload region's row stride = payload bytes per token
    const bool k_lg = k->layout == TQ_TILE_KEYS, v_lg = v->layout == TQ_TILE_VALUES;
    if ((k->layout != TQ_TILE_ROWS && !k_lg) || (v->layout != TQ_TILE_ROWS && !v_lg)) return TQ_ERR_INVALID_ARGUMENT;
    if (k_lg && (!block_tables || k->signs_permuted || k->idx.stride_row != 16 * k->bits + (k->qjl ? 16 : 0)))
        return TQ_ERR_INVALID_ARGUMENT;
    if (v_lg && (!block_tables || v->idx.stride_row != 16 * v->bits)) return TQ_ERR_INVALID_ARGUMENT;
    // the kernels read lane-grouped tiles only with every norm stream at 2 bytes per row
    if ((k_lg || v_lg) && (k->norm.stride_row != 2 || v->norm.stride_row != 2 || (k->qjl && k->rnorm.stride_row != 2)))
        return TQ_ERR_INVALID_ARGUMENT;
    int rc;
    if ((rc = check_region(k->idx, 4))) return rc;
    if ((rc = check_region(k->norm, 2))) return rc;
    if ((rc = check_region(v->idx, 4))) return rc;
    if ((rc = check_region(v->norm, 2))) return rc;
    if (k->qjl) {
        if (!k_lg && (rc = check_region(k->signs, 4))) return rc;
        if ((rc = check_region(k->rnorm, 2))) return rc;
    }
    const tq_region* regs[R_COUNT] = {&k->idx, (k->qjl && !k_lg) ? &k->signs : &k->idx, &k->norm,
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
    // Sparse-V over KV blocks of 32 tokens or more: the running max the skip test uses is updated
    // once per 32-token block (once per KV block for block_size 32, kernels/sparse_v.py:70-123),
    // so chunks start on such a block (tokens_per_chunk rounded up to a multiple of 32; the
    // workspace this needs is never larger).
    const bool sparse_pair = sparse_threshold > 0.f && block_size >= 32 && block_tables;
    const size_t need = tq_decode_workspace_bytes(num_seqs, num_q_heads, max_seq_len, tokens_per_chunk);
    if (!workspace || workspace_bytes < need || !aligned(workspace, 256)) return TQ_ERR_WORKSPACE;
    int addr = TQ_ADDR_CACHED;
    const bool fast = fast_path_ok(k, v, group, block_size, num_blocks, block_tables, &addr);
    const float k_cscale = k->centroid_scale > 0.f ? k->centroid_scale : 1.f;
    const float v_cscale = v->centroid_scale > 0.f ? v->centroid_scale : 1.f;
    const bool share = k->centroids == v->centroids && k->bits == v->bits && k_cscale == v_cscale;
    const bool contig = !fast && contig_path_ok(k, v, group, block_tables, block_size, max_seq_len, max_blocks_per_seq,
                                                sparse_threshold, rotate);
    if (contig && tokens_per_chunk == 0) {
        // one round of the resident waves, at least 6 tiles per unit (a unit's start-up is worth
        // several tiles; 6 measured faster than 8 at BH 8 x 32768), and no more units than the
        // workspace of tokens_per_chunk = 0 holds
        FastLdsLayout lay;
        tq_decode_fast_lds_layout(2, true, 2, share, &lay);
        int waves = 0;
        const int orc = resident_waves(tq_decode_fast_kernel_ptr(2, true, 2, 0, TQ_ADDR_CONTIG),
                                       tq_decode_fast_wg_waves(2, true, 2, lay.total), lay.total, &waves);
        if (orc) return orc;
        const int64_t tiles = (int64_t)num_seqs * num_kv_heads * (max_seq_len / 16);
        int64_t per = (tiles + waves - 1) / (waves > 0 ? waves : 1);
        per = per < 6 ? 6 : per;
        int64_t chunk = 16 * per;
        const int64_t fit = general_chunk(num_seqs, num_q_heads, max_seq_len, false);
        chunk = chunk > fit ? chunk : fit;
        tokens_per_chunk = (int)(chunk < max_seq_len ? chunk : max_seq_len);
    }
    // tokens_per_chunk = 0: the balanced schedule on the fast kernel; fixed chunks that fit the
    // same workspace on the general one
    // (the kernel keeps pair positions in 32 bits: at most num_seqs * num_kv_heads * ceil(len / 32))
    const int bal_cap = max_blocks_per_seq * block_size;
    const int bal_len = max_seq_len > 0 && max_seq_len < bal_cap ? max_seq_len : bal_cap;
    const bool balanced = tokens_per_chunk == 0 && fast &&
                          (int64_t)num_seqs * num_kv_heads * ((bal_len + 31) / 32) < (1ll << 31);
    if (tokens_per_chunk == 0 && !fast)
        tokens_per_chunk = general_chunk(num_seqs, num_q_heads, max_seq_len, sparse_pair);
    if (!balanced && sparse_pair && tokens_per_chunk % 32) tokens_per_chunk += 16;
    const int n_chunks = balanced ? 1 : n_chunks_for(max_seq_len, tokens_per_chunk);

    const size_t slots = (size_t)num_seqs * num_q_heads * n_chunks;
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    if (fast || contig) {
        FastDecodeParams f = {};
        f.addr = contig ? TQ_ADDR_CONTIG : addr;
        if (contig) {
            const tq_region* cr[6] = {&k->idx, &k->signs, &k->norm, &k->rnorm, &v->idx, &v->norm};
            for (int a = 0; a < 6; ++a) {
                f.contig[a].ptr = static_cast<const uint8_t*>(cr[a]->ptr);
                f.contig[a].stride_seq = cr[a]->stride_seq;
                f.contig[a].stride_head = cr[a]->stride_head;
            }
            f.contig_perm = k->signs_permuted ? 1 : 0;
        }
        f.q = q;
        f.q_ss = q_stride_seq;
        f.q_sh = q_stride_head;
        f.qp = q_proj ? q_proj : q;
        f.qp_ss = q_proj ? qp_stride_seq : q_stride_seq;
        f.qp_sh = q_proj ? qp_stride_head : q_stride_head;
        f.q_dtype = q_dtype;
        f.q_vec = q_vector_ok(f.q, q_dtype, f.q_ss, f.q_sh) && q_vector_ok(f.qp, q_dtype, f.qp_ss, f.qp_sh);
        f.num_seqs = num_seqs;
        f.hq = num_q_heads;
        f.hkv = num_kv_heads;
        f.group = group;
        const uint8_t* kb = static_cast<const uint8_t*>(k->idx.ptr);
        f.kbase = kb;
        f.k_sh = k->idx.stride_head;
        f.k_sb = (uint32_t)k->idx.stride_block;
        f.d_kn = (uint32_t)(static_cast<const uint8_t*>(k->norm.ptr) - kb);
        if (k->qjl) f.d_krn = (uint32_t)(static_cast<const uint8_t*>(k->rnorm.ptr) - kb);
        const uint8_t* vb = static_cast<const uint8_t*>(v->idx.ptr);
        f.vbase = vb;
        f.v_sh = v->idx.stride_head;
        f.v_sb = (uint32_t)v->idx.stride_block;
        f.d_vn = (uint32_t)(static_cast<const uint8_t*>(v->norm.ptr) - vb);
        f.k_cent = k->centroids;
        f.v_cent = v->centroids;
        f.k_cscale = k_cscale;
        f.v_cscale = v_cscale;
        f.v_cinv = 1.f / v_cscale;
        FastLdsLayout lay;
        tq_decode_fast_lds_layout(k->bits, k->qjl != 0, v->bits, share, &lay);
        const size_t lds_total = lay.total;
        f.lds_sign = lay.sign;
        f.lds_k = lay.k;
        f.lds_v = lay.v;
        f.lds_scratch = lay.scratch;
        f.rep_s = lay.rep_s;
        f.rep_k = lay.rep_k;
        f.rep_v = lay.rep_v;
        const int wpg = tq_decode_fast_wg_waves(k->bits, k->qjl != 0, v->bits, lds_total);
        f.block_size = block_size;
        int tsh = 0;
        while ((16 << tsh) < block_size) ++tsh;
        f.tile_shift = tsh;
        f.num_blocks = num_blocks;
        f.bt = block_tables;
        f.bt_stride = block_table_stride;
        f.max_blocks = contig ? max_seq_len / 16 : max_blocks_per_seq;  // contiguous: whole tiles up to max_seq_len
        f.seq_lens = seq_lens;
        f.uniform_len = max_seq_len;
        f.c_exp = sm_scale * kLog2e / k_cscale;
        f.sparse = sparse_threshold > 0.f ? 1 : 0;
        f.sparse_pair = sparse_pair ? 1 : 0;
        f.thr_log = f.sparse ? std::log2(sparse_threshold) / f.c_exp : 0.f;
        f.qp_mul = corr_scale * k_cscale;
        f.chunk = tokens_per_chunk;
        f.n_chunks = n_chunks;
        f.skip_stats = skip_stats;
        int64_t grid;
        if (balanced) {
            const size_t rows = bal_rows(num_seqs, num_q_heads);
            int waves = 0;
            // the plain instance, as tq_decode_concurrent_units counts it (the statistics and
            // 64-bit instances share its register budget and LDS)
            const int orc = resident_waves(tq_decode_fast_kernel_ptr(k->bits, k->qjl != 0, v->bits), wpg, lds_total, &waves);
            if (orc) return orc;
            // partial slots stay below workers + num_seqs * num_kv_heads
            const int64_t wmax = (int64_t)(rows / group) - (int64_t)num_seqs * num_kv_heads;
            f.balanced = 1;
            f.n_workers = (int)(waves < wmax ? waves : wmax);
            f.len_cap = bal_len;
            f.plan = reinterpret_cast<int64_t*>(ws);
            uint8_t* wsr = ws + bal_plan_bytes(num_seqs);
            f.ws_acc = reinterpret_cast<float*>(wsr);
            f.ws_m = reinterpret_cast<float*>(wsr + align_up(rows * TQ_HEAD_DIM * sizeof(float), 256));
            f.ws_l = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(f.ws_m) + align_up(rows * sizeof(float), 256));
            grid = (f.n_workers + wpg - 1) / wpg;
        } else {
            f.ws_acc = reinterpret_cast<float*>(ws);
            f.ws_m = reinterpret_cast<float*>(ws + align_up(slots * TQ_HEAD_DIM * sizeof(float), 256));
            f.ws_l = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(f.ws_m) + align_up(slots * sizeof(float), 256));
            grid = ((int64_t)num_seqs * num_kv_heads * n_chunks + wpg - 1) / wpg;
        }
        f.out = out;
        f.out_dtype = out_dtype;
        f.out_ss = out_stride_seq;
        f.out_sh = out_stride_head;
        f.rot_q = rotate;
        f.rot_qp = rotate && !q_proj;
        f.rot_out = rotate;
        f.wht_h = kWhtH;
        if (grid * wpg > 0x7fffffffll) return TQ_ERR_INVALID_ARGUMENT;  // unit indices stay below 2^31
        int frc = tq_decode_fast_launch(f, k->bits, k->qjl != 0, v->bits, grid, lds_total, (hipStream_t)stream);
        if (frc) return frc;
        return launch_reduce(f.ws_acc, f.ws_m, f.ws_l, num_seqs, num_q_heads, n_chunks, tokens_per_chunk,
                             max_blocks_per_seq * block_size, seq_lens, max_seq_len, out, out_dtype, out_stride_seq,
                             out_stride_head, rotate, (hipStream_t)stream, balanced ? &f : nullptr);
    }
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
    p.share_tab = (k->centroids == v->centroids && k->bits == v->bits && p.k_cscale == p.v_cscale) ? 1 : 0;
    p.k_perm = k->signs_permuted ? 1 : 0;
    p.block_size = block_size;
    p.num_blocks = block_tables ? num_blocks : (int64_t)1 << 62;
    p.bt = block_tables;
    p.bt_stride = block_table_stride;
    p.max_blocks = max_blocks_per_seq;
    p.seq_lens = seq_lens;
    p.uniform_len = max_seq_len;
    p.qp_scale = sm_scale * kLog2e;
    p.q_scale = p.qp_scale / p.k_cscale;
    p.corr_scale = corr_scale;
    p.thresh = sparse_threshold > 0.f ? sparse_threshold : 0.f;
    p.log2_thresh = sparse_threshold > 0.f ? std::log2(sparse_threshold) : 0.f;
    p.sparse_pair = sparse_pair ? 1 : 0;
    p.chunk = tokens_per_chunk;
    p.n_chunks = n_chunks;
    p.ws_acc = ws_acc;
    p.ws_m = ws_m;
    p.ws_l = ws_l;
    p.skip_stats = skip_stats;
    p.out = out;
    p.out_dtype = out_dtype;
    p.out_ss = out_stride_seq;
    p.out_sh = out_stride_head;
    p.rot_q = rotate;
    p.rot_qp = rotate && !q_proj;
    p.rot_out = rotate;
    p.wht_h = kWhtH;
    p.k_lg = k_lg ? 1 : 0;
    p.v_lg = v_lg ? 1 : 0;
    p.vstep = v_lg ? v->bits : (int32_t)v->idx.stride_row;

    const int64_t units = (int64_t)num_seqs * num_kv_heads * n_chunks;
    const int64_t grid = (units + 3) / 4;
    if (grid > 0x7fffffff) return TQ_ERR_INVALID_ARGUMENT;
    hipStream_t st = (hipStream_t)stream;
    // Norm rows 2 bytes apart: one 8-byte load per norm stream per tile.
    const bool nv = p.rrow[R_KNORM] == 2 && p.rrow[R_VNORM] == 2 && (!k->qjl || p.rrow[R_KRNORM] == 2);
    const void* kern = decode_kernel_ptr(k->bits, k->qjl != 0, v->bits, group <= 8, nv);
    if (!kern) return TQ_ERR_BITS;
    void* args[] = {&p};
    hipError_t le = hipLaunchKernel(kern, dim3((unsigned)grid), dim3(256), args,
                                    lds_bytes(k->bits, v->bits, p.share_tab), st);
    if (le != hipSuccess) return (int)le;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;

    return launch_reduce(ws_acc, ws_m, ws_l, num_seqs, num_q_heads, n_chunks, tokens_per_chunk,
                         max_blocks_per_seq * block_size, seq_lens, max_seq_len, out, out_dtype, out_stride_seq, out_stride_head,
                         rotate, st);
}

extern "C" size_t tq_packed_attention_workspace_bytes(int bh, int sk, int tokens_per_chunk) {
    if (bh <= 0 || sk <= 0 || tokens_per_chunk < 0) return 0;
    return tq_decode_workspace_bytes(bh, 1, sk, tokens_per_chunk);
}

extern "C" int tq_packed_attention(const void* q, const void* q_proj, int q_dtype, const uint8_t* k_idx,
                                   const uint8_t* k_signs, int signs_permuted, const uint16_t* k_rnorm,
                                   const uint16_t* k_norm, const uint8_t* v_idx, const uint16_t* v_norm,
                                   const float* centroids, float centroid_scale, float corr_scale, int bh, int sk,
                                   int tokens_per_chunk, void* workspace, size_t workspace_bytes, void* out,
                                   int out_dtype, tq_stream_t stream) {
    if (bh < 0 || sk < 0) return TQ_ERR_INVALID_ARGUMENT;
    if (bh == 0) return TQ_OK;
    if (sk == 0 || !q || !q_proj || !k_idx || !k_signs || !k_rnorm || !k_norm || !v_idx || !v_norm || !centroids)
        return TQ_ERR_INVALID_ARGUMENT;
    // every head is a sequence of sk rows of its own (one query head per KV head), its rows
    // following each other: 16-row tiles addressed by stride, no block table
    const int64_t nblk = ((int64_t)sk + 15) / 16;
    if (nblk > 0x7fffffff) return TQ_ERR_INVALID_ARGUMENT;
    auto region = [&](const void* ptr, int64_t row) {
        return tq_region{ptr, 16 * row, 0, (int64_t)sk * row, row};
    };
    tq_kv_view k = {};
    k.idx = region(k_idx, 32);
    k.signs = region(k_signs, 16);
    k.norm = region(k_norm, 2);
    k.rnorm = region(k_rnorm, 2);
    k.centroids = centroids;
    k.bits = 2;
    k.qjl = 1;
    k.signs_permuted = signs_permuted ? 1 : 0;
    k.centroid_scale = centroid_scale;
    k.layout = TQ_TILE_ROWS;
    tq_kv_view v = {};
    v.idx = region(v_idx, 32);
    v.norm = region(v_norm, 2);
    v.centroids = centroids;
    v.bits = 2;
    v.centroid_scale = centroid_scale;
    v.layout = TQ_TILE_ROWS;
    return tq_decode_impl(0, q, q_dtype, TQ_HEAD_DIM, TQ_HEAD_DIM, q_proj, TQ_HEAD_DIM, TQ_HEAD_DIM, bh, 1, 1,
                          TQ_HEAD_DIM, &k, &v, 16, nblk, nullptr, 0, (int)nblk, nullptr, sk, 1.0f, corr_scale, 0.0f,
                          tokens_per_chunk, workspace, workspace_bytes, out, out_dtype, TQ_HEAD_DIM, TQ_HEAD_DIM,
                          nullptr, stream);
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
    return tq_decode_impl(0, q, q_dtype, q_stride_seq, q_stride_head, q_proj, qp_stride_seq, qp_stride_head, num_seqs, num_q_heads,
                       num_kv_heads, head_dim, k, v, block_size, num_blocks, block_tables, block_table_stride,
                       max_blocks_per_seq, seq_lens, max_seq_len, sm_scale, corr_scale, sparse_threshold,
                       tokens_per_chunk, workspace, workspace_bytes, out, out_dtype, out_stride_seq, out_stride_head,
                       skip_stats, stream);
}

extern "C" int tq_decode_rotated(const void* q, int q_dtype, int64_t q_stride_seq, int64_t q_stride_head,
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
    return tq_decode_impl(1, q, q_dtype, q_stride_seq, q_stride_head, q_proj, qp_stride_seq, qp_stride_head, num_seqs, num_q_heads,
                       num_kv_heads, head_dim, k, v, block_size, num_blocks, block_tables, block_table_stride,
                       max_blocks_per_seq, seq_lens, max_seq_len, sm_scale, corr_scale, sparse_threshold,
                       tokens_per_chunk, workspace, workspace_bytes, out, out_dtype, out_stride_seq, out_stride_head,
                       skip_stats, stream);
}
