// Packed asymmetric split-K decode attention for gfx950: the paged fast path.
//
// Used by tq_decode when the caches are in this library's tile layout (one tile of 16-token
// rows per (physical block, KV head), see tq_compress_paged) and the GQA group has at most 8
// query heads.  Other layouts go through decode_kernel (tq_decode.hip).
//
// Work unit = one wave64 = (sequence, KV head, chunk of tokens_per_chunk tokens), walked in
// pairs of 16-token tiles (A, B).  Per pair (fp32 accumulation throughout):
//   S_X^T[token][col] = K_X[16 x 128] . Q^T[128 x 16]         4 x mfma_f32_16x16x32_f16 per tile
//       K_X: a pair of packed indices -> half2 of centroids through an LDS table;
//       column col of Q holds query head col & 7, so both halves of the output hold all heads.
//   QJL_X^T = (+-1)[16 x 128] . QP^T                           3 x mfma_scale_f32_16x16x128_f8f6f4
//       sign bits -> fp4 +-1 through a byte-indexed LDS table (one dword per 8 signs); q_proj
//       as three fp6 (e2m3) parts with per-lane E8M0 block scales: the error of each element is
//       at most 2^-14 of the largest magnitude of its 32-element block (fp16 q_proj, the
//       reference's operand, carries 2^-11 of each element).  fp4 x fp6 runs at the fp4 rate:
//       three of these cost less matrix time than two fp4 x fp8 products.
//   Lanes with col < 8 keep tile A's scores and lanes with col >= 8 tile B's, so after the
//   merge one wave holds 32 tokens x 8 heads of scores (4 per lane): the online softmax, the
//   Sparse-V test and the conversions run once per pair.
//   acc^T[dim][col] += V^T[128 x 32] . P^T[32 x 16]           8 x mfma_f32_16x16x32_f16 per pair
//       k-slots 0-3 of lane group g are tile A's tokens 4g..4g+3, slots 4-7 tile B's; column
//       col < 8 takes tile A's p from its own lane and tile B's from lane col + 8 (DPP row
//       rotate), so columns 0-7 accumulate both tiles and columns 8-15 are ignored.  The values
//       tile stores each dim's four tokens side by side, so one table lookup per tile and dim
//       is the A operand (no lane-local transposes).
// MFMA output layout (16x16): lane l holds rows 4(l/16)+r, column l%16 - after the QK product
// lane (col, g) owns tokens 4g..4g+3, the B-operand layout of the PV product.
//
// Scores stay in "raw" units (q . k * centroid_scale, no softmax scale): q enters the MFMA as
// fp16 without scaling (exact for bf16/fp16 queries) and the softmax scale is applied in the
// exponent: p = exp2(c * (s - m)), c = sm_scale * log2(e) / centroid_scale.
//
// Memory: the caches are in the lane-grouped tile layouts (TQ_TILE_KEYS / TQ_TILE_VALUES):
// per 16-row sub-tile a lane reads its key data (index dwords + sign dword) with one load and
// its value data (4 rows x 8 dims) with one load.  The K and V buffer descriptors are loop
// invariant (base = cache + head offset) and a tile is addressed by scalar offsets (block *
// block_stride + region offset) when the cache spans less than 2 GiB; the norm streams are then
// read once per pair (lanes of tile A and tile B differ in their vector offset).  A larger cache
// (the BIG instances, picked on the host) gets one descriptor per tile from a 64-bit base and
// reads each tile's norms with the lanes of that tile.
// Block-table entries arrive four tiles at a time in lanes 0-3 of one vector load, a loop
// iteration ahead, and are read with v_readlane.  Tile loads run one pair ahead.
//
// Sparse-V (kernels/sparse_v.py:108-149): for tile X, m_X = running max through tile X; token t
// is dropped from PV when no head of the group has exp2(c (s - m_X)) > threshold, tested as
// s > m_X + log2(threshold)/c with a ballot; dropped tokens stay in the denominator.
#include <mutex>
#include <set>
#include <type_traits>
#include <utility>

#include "tq_common.h"
#include "tq_decode_internal.h"

namespace {

constexpr float kNegInf = -__builtin_huge_valf();

typedef int tq_i32x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) const uint32_t lds_u32;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const uint8_t* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), (short)0, 0x7fffffff, 0x00020000);
}

__device__ __forceinline__ uint32_t lds_read(uint32_t addr) { return *(lds_u32*)(uintptr_t)addr; }

// LDS address of the 3-bit quad table entry held in bits [pos, pos + 12) of the word array w:
// the field is moved to bit 3 (entries of 8 bytes; one shift or funnel shift) and masked, and the
// table base merged in (folded away for the K table at address 0).
template <int N>
__device__ __forceinline__ uint32_t quad3_addr(const uint32_t (&w)[N], int pos, uint32_t base) {
    const int wi = pos >> 5, sh = pos & 31;
    uint32_t f;
    if (sh + 12 <= 32 || wi + 1 >= N)
        f = sh >= 3 ? (w[wi] >> (sh - 3)) : (w[wi] << (3 - sh));
    else
        f = __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh - 3);
    return (f & 0x7ff8u) | base;
}

__device__ __forceinline__ tq_u32x2 lds_read2(uint32_t addr) {
    typedef __attribute__((address_space(3))) const tq_u32x2 lds_u32x2;
    return *(lds_u32x2*)(uintptr_t)addr;
}

// Index fields are looked up in LDS tables: 2- and 3-bit fields four at a time (a 4B-bit field
// -> 4 fp16 centroids, an 8-byte entry), 4-bit fields in pairs (a byte -> half2, 4 bytes), and
// sign bytes -> 8 fp4 values +-1 (4 bytes).
// Row tables (2-bit quads, 4-bit pairs, the sign table) are indexed by one byte of a word:
// entry e, replica r at base + 256 e + es r (es: entry bytes), base = 64 KB x region + column
// (0, or 128 when two tables share the rows of a region).  A lookup address is one byte permute
// of the word and the lane's word lw = base + es (lane & (replicas - 1)): byte 0 column and
// replica, byte 1 the field, byte 2 the region.  Each lane reads its own replica: a full row
// (256 bytes) holds 32 quad or 64 pair / sign replicas, one per bank (pair) of the LDS.
// 3-bit quad tables: 4096 entries of 8 bytes at 32 KB-aligned offsets (a K table at 0), not
// replicated (quad3_addr).
template <int B>
constexpr bool quad_table() {
    return B == 3 || B == 2;
}
// Entry bytes of a row table.
template <int B>
constexpr uint32_t row_entry_bytes() {
    return B == 2 ? 8u : 4u;
}
__device__ __forceinline__ uint32_t row_addr(uint32_t w, int k, uint32_t lw) {
    // bytes: lw.0 (column + replica), w.k (the field), lw.2 (region), 0
    return __builtin_amdgcn_perm(lw, w, 0x0c060004u | ((uint32_t)k << 8));
}
// The row-table address of the byte at bit pos (a multiple of 8) of the word array w.
template <int N>
__device__ __forceinline__ uint32_t row_addr_at(const uint32_t (&w)[N], int pos, uint32_t lw) {
    return row_addr(w[pos >> 5], (pos & 31) >> 3, lw);
}

__device__ __forceinline__ float half_at(const uint32_t (&w)[2], int r) {
    const uint32_t b = (r & 1) ? (w[r >> 1] >> 16) : (w[r >> 1] & 0xffffu);
    return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}

// Each quad of lanes (4 consecutive bits) of m set when any of its bits is (s_wqm_b64).
__device__ __forceinline__ uint64_t quad_any(uint64_t m) {
    uint64_t q;
    asm("s_wqm_b64 %0, %1" : "=s"(q) : "s"(m) : "scc");
    return q;
}

// Value of lane l ^ 8 within its row of 16 lanes (DPP row_ror:8).
__device__ __forceinline__ uint32_t row_swap8(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x128, 0xf, 0xf, false);
}
__device__ __forceinline__ float row_swap8f(float x) { return __uint_as_float(row_swap8(__float_as_uint(x))); }

// inclusive prefix sum over the 64 lanes (once per wave and 64 sequences: cross-lane moves)
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t t = (uint32_t)__shfl_up((int)v, d, 64);
        if (lane >= d) v += t;
    }
    return v;
}

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

// half2 of (vn.lo * p0, vn.hi * p1) for a word vn of two fp16 norms, each product rounded once
// to nearest: v_fma_mixlo_f16 writes the low half, v_fma_mixhi_f16 the high half keeping the low
// (two instructions; the compiler forms each half alone and then shifts and ors them).
__device__ __forceinline__ uint32_t scale_to_half2(uint32_t vn, float p0, float p1) {
    uint32_t u;
    asm("v_fma_mixlo_f16 %0, %1, %2, 0 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixhi_f16 %0, %1, %3, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
        : "=&v"(u)
        : "v"(vn), "v"(p0), "v"(p1));
    return u;
}

// Raw data of one pair of tiles.  K part: loaded one pair ahead; V part: loaded at the start
// of its own pair (it is first needed after the QK products and the softmax).
template <int KB, bool KQJL>
struct KRaw {
    uint32_t kwA[KB], kwB[KB];  // dims 32g..32g+31 of token n, tiles A and B
    uint32_t ksA, ksB;          // sign bits of the same dims
    uint32_t kn[2], krn[2];     // fp16 norms of tokens 4g..4g+3 of the lane's tile
};
template <int VB>
struct VRaw {
    uint32_t vwA[VB], vwB[VB];  // chunk 16g + n of the values tile: field 4j + r = dim 8n + j of
                                // token 4g + r (VB bits each)
    uint32_t vn[2];             // fp16 norms of tokens 4g..4g+3 of the lane's tile
};
// Wave-uniform description of a pair.
struct PairInfo {
    uint32_t vbA, vbB;          // scalar byte offsets of the tiles' blocks in the V cache (BIG:
                                // the block numbers)
    uint32_t r0A, r0B;          // first row of each tile inside its block
    int nvA, nvB;               // valid rows (0: past the end or unreadable block)
};

struct Softmax {
    float m;        // Sparse-V: running max per head (raw score units), equal in lanes col and col ^ 8
    float mref;     // exponent base of lsum and acc: p = exp2(c s + nb), nb = -c mref - 1
    float nb;
    float lsum;     // this lane's tokens
    tq_floatx4 acc[8];
    uint32_t n_tot, n_kept;  // wave-uniform
};

// Per-lane constants of the compute step.
struct LaneCtx {
    tq_half8 qop[4];            // q (fp16), MFMA chunk cc: dims 32g + 8cc + j
    tq_i32x8 qp6[3];            // q_proj * corr * cscale * 2^b as three fp6 parts (6 dwords each)
    // E8M0 scales of the parts in bytes 0-2 (2^-b, 2^-(b+5), 2^-(b+10)) for tile A's products in
    // qscA and tile B's in qscB, with byte value 0 (2^-127) in the other tile's columns (lanes)
    int qscA, qscB;
    uint32_t klw, vlw, slw;     // lane words of the K, V and sign row tables (row_addr)
    uint32_t vquad;             // 3-bit V quad table base (a 3-bit K quad table is at address 0)
    uint64_t hmask;             // lanes of real heads
    float gap;                  // 1 / c_exp: one log2 unit of p in raw score units
    bool lo8;                   // column < 8: tile A
};

template <int KB>
__device__ __forceinline__ tq_floatx4 qk_tile(const uint32_t (&kw)[KB], const LaneCtx& c) {
    tq_floatx4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
        tq_u32x4 a;
        if (quad_table<KB>()) {
            // dims 8cc..8cc+7 of the lane's 32: two quads (a 3-bit K quad table sits at LDS
            // address 0, so its address is the field times 8)
            const tq_u32x2 lo = lds_read2(KB == 3 ? quad3_addr(kw, 24 * cc, 0u) : row_addr_at(kw, 16 * cc, c.klw));
            const tq_u32x2 hi = lds_read2(KB == 3 ? quad3_addr(kw, 24 * cc + 12, 0u) : row_addr_at(kw, 16 * cc + 8, c.klw));
            a[0] = lo[0];
            a[1] = lo[1];
            a[2] = hi[0];
            a[3] = hi[1];
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) a[j] = lds_read(row_addr(kw[cc], j, c.klw));
        }
        s = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(tq_half8, a), c.qop[cc], s, 0, 0, 0);
    }
    return s;
}

// QJL products of one tile accumulated onto t with B scales sc (a tile's own columns carry the
// real scales; the other tile's columns 2^-127, so that two tiles chained on one accumulator
// leave each column holding its own tile's term, plus at most 128 * 7.5 * 2^-127 < 6e-36).
__device__ __forceinline__ tq_floatx4 qjl_tile(uint32_t ks, tq_floatx4 t, int sc, const LaneCtx& c) {
    tq_i32x8 a;
#pragma unroll
    for (int b = 0; b < 4; ++b) a[b] = (int)lds_read(row_addr(ks, b, c.slw));
#pragma unroll
    for (int b = 4; b < 8; ++b) a[b] = 0;  // fp4 operand: only the first four dwords are read
    // A: fp4 (format 4), B: fp6 e2m3 (format 2); the B scale is byte 0, 1, 2 of sc
    t = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, c.qp6[0], t, 4, 2, 0, 127, 0, sc);
    t = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, c.qp6[1], t, 4, 2, 0, 127, 1, sc);
    t = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, c.qp6[2], t, 4, 2, 0, 127, 2, sc);
    return t;
}

// Lanes (col, g) whose tile row 4g + r is valid: tile A in columns 0-7, tile B in 8-15.
__device__ __forceinline__ uint64_t row_mask(int nvA, int nvB, int r) {
    auto groups = [](int nv, int r) -> uint64_t {
        int ng = (nv - r + 3) >> 2;  // lane groups g with 4g + r < nv
        ng = ng < 0 ? 0 : ng;
        return ng >= 4 ? ~0ull : ((1ull << (16 * ng)) - 1ull);
    };
    return (groups(nvA, r) & 0x00ff00ff00ff00ffull) | (groups(nvB, r) & 0xff00ff00ff00ff00ull);
}

// One pair of tiles.
template <int KB, bool KQJL, int VB, int SPV>
__device__ __forceinline__ void compute_pair(const KRaw<KB, KQJL>& kr, const VRaw<VB>& vr, const PairInfo& pi,
                                             Softmax& st, const LaneCtx& c, const FastDecodeParams& p) {
    // ---------------- scores ----------------
    const tq_floatx4 sA = qk_tile<KB>(kr.kwA, c);
    const tq_floatx4 sB = qk_tile<KB>(kr.kwB, c);
    // QJL: tile B's products accumulate onto tile A's; columns < 8 end with tile A's term and
    // columns >= 8 with tile B's (the scales zero the other tile's columns), so no selects
    tq_floatx4 t = {0.f, 0.f, 0.f, 0.f};
    if (KQJL) {
        t = qjl_tile(kr.ksA, t, c.qscA, c);
        t = qjl_tile(kr.ksB, t, c.qscB, c);
    }
    // Rows past the end may hold any bits in a paged block: masked out of the scores, and their
    // value norms zeroed (bit-wise, before any arithmetic), in partial pairs only.
    uint32_t vn[2] = {vr.vn[0], vr.vn[1]};
    float sc[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        // Scalar copies: shuffling ext_vector elements in place has miscompiled before.
        const float s1 = c.lo8 ? sA[r] : sB[r];
        if (KQJL) {
            const float s2 = t[r];
            sc[r] = __builtin_fmaf(half_at(kr.kn, r), s1, __builtin_fmaf(half_at(kr.krn, r), s2, 0.0f));
        } else {
            sc[r] = half_at(kr.kn, r) * s1;
        }
    }
    if (pi.nvA != 16 || pi.nvB != 16) {
        uint64_t rm[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            rm[r] = row_mask(pi.nvA, pi.nvB, r);
            sc[r] = __builtin_amdgcn_inverse_ballot_w64(rm[r]) ? sc[r] : kNegInf;
        }
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const uint32_t lo = __builtin_amdgcn_inverse_ballot_w64(rm[2 * k]) ? 0x0000ffffu : 0u;
            const uint32_t hi = __builtin_amdgcn_inverse_ballot_w64(rm[2 * k + 1]) ? 0xffff0000u : 0u;
            vn[k] &= lo | hi;
        }
    }

    // ---------------- online softmax ----------------
    // The exponent base mref moves only when some head's max passes it by more than one log2
    // unit (gap = 1 / c), and p is taken at half scale, exp2(c (s - mref) - 1) <= 1: p * norm
    // stays within fp16 as with the exact running max, while most pairs skip the rescale of
    // acc and lsum.  The Sparse-V test keeps the exact running max (st.m).
    float mt = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
    mt = max_over_groups(mt);                 // this tile's max for the lane's head
    const float other = row_swap8f(mt);       // the other tile's max for the same head
    const float m_pair = fmaxf(mt, other);
    const float cexp = p.c_exp;
    float m_old = 0.f, m_new = 0.f;
    if (SPV) {
        m_old = st.m;
        m_new = fmaxf(m_old, m_pair);
        st.m = m_new;
    }
    if (__builtin_amdgcn_ballot_w64(m_pair > st.mref + c.gap) & c.hmask) {
        const float mb = fmaxf(st.mref, m_pair);
        const float alpha = __builtin_amdgcn_exp2f(cexp * (st.mref - mb));  // 0 while mref = -inf
        st.lsum *= alpha;
#pragma unroll
        for (int i = 0; i < 8; ++i) st.acc[i] *= alpha;
        st.mref = mb;
        st.nb = __builtin_fmaf(-cexp, mb, -1.0f);
    }
    float pr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) pr[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[r], cexp, st.nb));  // 0 for masked rows
    st.lsum += (pr[0] + pr[1]) + (pr[2] + pr[3]);

    // ---------------- Sparse-V ----------------
    // The skip test uses the running max through the token's KV block: through its own tile for
    // 16-token blocks, through the pair (a 32-token block) otherwise.
    if (SPV) {
        const float m_skip = (c.lo8 && !p.sparse_pair) ? fmaxf(m_old, mt) : m_new;
        const float thr = m_skip + p.thr_log;
        uint32_t kept = 0;
        uint64_t any = 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint64_t bal = __builtin_amdgcn_ballot_w64(sc[r] > thr) & c.hmask;
            any |= bal;
            // lanes of the 8-lane groups (one token of one tile, the group's heads) with a passing
            // head, on the scalar unit: each quad of lanes OR-spread (s_wqm), then each pair of quads
            const uint64_t q = quad_any(bal);
            const uint64_t lo = (q | (q >> 4)) & 0x0f0f0f0f0f0f0f0full;
            const uint64_t keepm = lo | (lo << 4);
            pr[r] = __builtin_amdgcn_inverse_ballot_w64(keepm) ? pr[r] : 0.f;
            if (SPV == 2) kept += (uint32_t)__builtin_popcountll(keepm & 0x0101010101010101ull);
        }
        if (SPV == 2) {
            st.n_tot += (uint32_t)(pi.nvA + pi.nvB);
            st.n_kept += kept;
        }
        if (!any) return;  // every token of the pair dropped: no PV products
    }

    // ---------------- PV ----------------
    const uint32_t p01 = scale_to_half2(vn[0], pr[0], pr[1]);
    const uint32_t p23 = scale_to_half2(vn[1], pr[2], pr[3]);
    const tq_u32x4 bw = {p01, p23, row_swap8(p01), row_swap8(p23)};
    const tq_half8 bop = __builtin_bit_cast(tq_half8, bw);
    // acc[a] (dim 8n + a): field group a of the lane's chunk is that dim's four tokens, so the
    // lookups are the A operand as they come: k-slots 0-3 tile A's tokens, 4-7 tile B's.
    auto vlook = [&](int a) -> tq_u32x4 {
        tq_u32x4 aw;
        if (quad_table<VB>()) {
            // one quad per tile
            const uint32_t fa = VB == 3 ? quad3_addr(vr.vwA, 12 * a, c.vquad) : row_addr_at(vr.vwA, 8 * a, c.vlw);
            const uint32_t fb = VB == 3 ? quad3_addr(vr.vwB, 12 * a, c.vquad) : row_addr_at(vr.vwB, 8 * a, c.vlw);
            const tq_u32x2 xa = lds_read2(fa);
            const tq_u32x2 xb = lds_read2(fb);
            aw = tq_u32x4{xa[0], xa[1], xb[0], xb[1]};
        } else {
            // two pairs per tile: tokens 0, 1 and 2, 3
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                aw[h] = lds_read(row_addr_at(vr.vwA, 16 * a + 8 * h, c.vlw));
                aw[2 + h] = lds_read(row_addr_at(vr.vwB, 16 * a + 8 * h, c.vlw));
            }
        }
        return aw;
    };
    // Software pipeline: the lookups of dim group a + 2 are issued before the product of group
    // a, so a wave has two groups of LDS reads in flight behind each MFMA (the schedule below
    // pins that order; left to itself the scheduler waited for every pair of reads).
    tq_u32x4 w0 = vlook(0), w1 = vlook(1);
#pragma unroll
    for (int a = 0; a < 8; ++a) {
        tq_u32x4 w2 = w1;
        if (a + 2 < 8) w2 = vlook(a + 2);
        st.acc[a] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(tq_half8, w0), bop, st.acc[a], 0, 0, 0);
        w0 = w1;
        w1 = w2;
    }
    constexpr int kReads = quad_table<VB>() ? 2 : 4;  // LDS reads per dim group
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * kReads, 0);  // DS reads: groups 0 and 1
#pragma unroll
    for (int a = 0; a < 6; ++a) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);       // MFMA of group a
        __builtin_amdgcn_sched_group_barrier(0x100, kReads, 0);  // DS reads of group a + 2
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
}

// Waves per SIMD (register budget 512 / waves): QJL keys need the fp8 q_proj operands.
template <int KB, bool KQJL, int VB>
constexpr int fast_waves() {
    return KQJL ? 3 : 4;
}
// Most waves per workgroup (the launch bound): a compute unit's resident waves in one workgroup.
// The host launches fewer per workgroup when the tables leave room for several workgroups per
// compute unit (tq_decode_fast_wg_waves).
template <int KB, bool KQJL, int VB>
constexpr int fast_wg_waves() {
    return 4 * fast_waves<KB, KQJL, VB>();
}

// Fixed chunks: work unit u is (sequence s, chunk ci, KV head kh), sequence-major (u = (s *
// n_chunks + ci) * hkv + kh): consecutive workgroups, which the dispatcher deals round-robin to
// the XCDs, take neighbouring chunks of one sequence, so every XCD gets a share of each
// sequence.  Returns whether the unit holds tokens.
__device__ __forceinline__ bool chunk_unit(int u, const FastDecodeParams& p, int cap, int& s, int& ci, int& kh,
                                           int& L) {
    kh = u % p.hkv;
    const int t = u / p.hkv;
    ci = t % p.n_chunks;
    s = t / p.n_chunks;
    if (s >= p.num_seqs) return false;
    L = tq_seq_len(p.seq_lens, s, p.uniform_len);
    L = L < cap ? L : cap;
    return ci * p.chunk < L;
}
// Whether any unit of this workgroup's waves holds tokens (else the workgroup returns before
// building its tables): lane w of each wave tests wave w's unit, all lengths in one load round.
// Unit indices stay below 2^31 (checked on the host).
__device__ __forceinline__ bool chunk_group_busy(const FastDecodeParams& p, int cap, int wpg) {
    const int lane = (int)(threadIdx.x & 63);
    bool busy = false;
    if (lane < wpg) {
        int s, ci, kh, L;
        busy = chunk_unit((int)blockIdx.x * wpg + lane, p, cap, s, ci, kh, L);
    }
    return __builtin_amdgcn_ballot_w64(busy) != 0;
}

// LDS tables, built by the whole workgroup before any tile is read (part of each wave's
// start-up): the fp4 sign table (QJL) and the K and V tables at the offsets and with the
// replica counts chosen by the host (tq_decode_fast_lds_layout).  The scaled fp16 centroids are
// first staged in the 512-byte scratch area (K in dwords 0-63, V in 64-127: 3-bit: the 64 pairs
// of fields as half2; 2-bit: the 16 pairs; 4-bit: the 16 values), then every entry is read from
// there.  Row tables are written with 16-byte stores, consecutive threads along a row (a wave
// writes 1 KB of consecutive bytes).  Ends with a workgroup barrier.
// Thread tid's dword of the staging area (K in dwords 0-63, V's own table in 64-127; 0 where
// unused), loaded at kernel entry so that its round trip overlaps the first length reads.
template <int KB, int VB>
__device__ __forceinline__ uint32_t stage_value(const FastDecodeParams& p, int tid) {
    auto val = [&](auto bits_c, const float* cent, float cs, int x) -> uint32_t {
        constexpr int bits = decltype(bits_c)::value;
        if (bits == 3) return tq_pack_half2(cent[x & 7] * cs, cent[x >> 3] * cs);
        if (x >= 16) return 0u;
        return bits == 2 ? tq_pack_half2(cent[x & 3] * cs, cent[x >> 2] * cs) : tq_pack_half2(cent[x] * cs, 0.f);
    };
    if (tid < 64) return val(std::integral_constant<int, KB>{}, p.k_cent, p.k_cscale, tid);
    if (tid < 128 && p.lds_v != p.lds_k) return val(std::integral_constant<int, VB>{}, p.v_cent, p.v_cscale, tid - 64);
    return 0u;
}

template <int KB, bool KQJL, int VB>
__device__ __forceinline__ void build_tables(const FastDecodeParams& p, uint32_t* s_lds, int tid, uint32_t staged) {
    const int NT = (int)__builtin_amdgcn_workgroup_size_x();
    uint8_t* lds8 = reinterpret_cast<uint8_t*>(s_lds);
    uint32_t* st = s_lds + p.lds_scratch / 4;
    const bool vown = p.lds_v != p.lds_k;
    if (tid < 128) st[tid] = staged;
    // row table at base with es-byte entries, rep + 1 replicas; value(e): 16 bytes of entry e
    auto fill_row = [&](uint32_t base, uint32_t es, uint32_t rep, auto value) {
        const int S = (int)(es * (rep + 1) / 16);  // 16-byte stores per row: 8 or 16
        const int sh = S == 16 ? 4 : 3;
        for (int i = tid; i < 256 * S; i += NT) {
            const int e = i >> sh;
            *reinterpret_cast<tq_u32x4*>(lds8 + base + 256 * e + 16 * (i & (S - 1))) = value(e);
        }
    };
    if (KQJL) {
        // sign byte e -> 8 fp4 values: bit j set +1 (0x2), clear -1 (0xA), in nibble j
        fill_row(p.lds_sign, 4u, p.rep_s, [&](int e) {
            uint32_t x = (uint32_t)e;  // bit j -> bit 4j
            x = (x | (x << 12)) & 0x000f000fu;
            x = (x | (x << 6)) & 0x03030303u;
            x = (x | (x << 3)) & 0x11111111u;
            const uint32_t w = 0xaaaaaaaau ^ (x << 3);
            return tq_u32x4{w, w, w, w};
        });
    }
    __syncthreads();
    auto fill_codes = [&](auto bits_c, uint32_t base, uint32_t rep, const uint32_t* sv) {
        constexpr int bits = decltype(bits_c)::value;
        if constexpr (bits == 2) {
            // 4 x fp16 c[(e >> 2j) & 3], j = 0..3
            fill_row(base, 8u, rep, [&](int e) {
                const uint32_t lo = sv[e & 15], hi = sv[e >> 4];
                return tq_u32x4{lo, hi, lo, hi};
            });
        } else if constexpr (bits == 4) {
            // half2(c[e & 15], c[e >> 4])
            fill_row(base, 4u, rep, [&](int e) {
                const uint32_t w = (sv[e & 15] & 0xffffu) | (sv[e >> 4] << 16);
                return tq_u32x4{w, w, w, w};
            });
        } else {
            // 4096 entries of 8 bytes: 4 x fp16 c[(e >> 3j) & 7], from the pairs of fields
            tq_u32x2* t = reinterpret_cast<tq_u32x2*>(lds8 + base);
            for (int e = tid; e < 4096; e += NT) t[e] = tq_u32x2{sv[e & 63], sv[e >> 6]};
        }
    };
    fill_codes(std::integral_constant<int, KB>{}, p.lds_k, p.rep_k, st);
    if (vown) fill_codes(std::integral_constant<int, VB>{}, p.lds_v, p.rep_v, st + 64);
    __syncthreads();
}

// The lane's row-table words and 3-bit V table base, and its tile half (column < 8: tile A).
template <int KB, int VB>
__device__ __forceinline__ void init_lane_tables(LaneCtx& c, const FastDecodeParams& p, int lane) {
    c.lo8 = (lane & 15) < 8;
    c.klw = p.lds_k + row_entry_bytes<KB>() * ((uint32_t)lane & p.rep_k);
    c.vlw = p.lds_v + row_entry_bytes<VB>() * ((uint32_t)lane & p.rep_v);
    c.slw = p.lds_sign + 4u * ((uint32_t)lane & p.rep_s);
    // 3-bit V quad table: address 0 when it is the K quad table, else its base from a VGPR (a
    // VALU op takes one scalar operand, and the field mask is one)
    c.vquad = p.lds_v;
    if (VB == 3 && !(KB == 3 && p.lds_v == 0)) asm volatile("v_mov_b32 %0, %1" : "=v"(c.vquad) : "s"(c.vquad));
}

// Query operands from the lane's 32 loaded elements of q (qv) and of q_proj (x): q as fp16
// (rotated by H first when asked), q_proj * corr * cscale as three fp6 e2m3 parts with E8M0
// scales (QJL keys).
template <bool KQJL>
__device__ __forceinline__ void make_q_operands(LaneCtx& c, const FastDecodeParams& p, float (&qv)[32], float (&x)[32]) {
    if (p.rot_q) tq_wht_row_g4(qv, p.wht_h);  // q x H: elements 32g + i
#pragma unroll
    for (int cc = 0; cc < 4; ++cc)
#pragma unroll
        for (int j = 0; j < 8; ++j) c.qop[cc][j] = (_Float16)qv[8 * cc + j];
    if constexpr (KQJL) {
        if (p.rot_qp) tq_wht_row_g4(x, p.wht_h);  // q_proj x H: elements 32g + i
        // One E8M0 scale per lane: its 32 elements are one 32-wide scale block of the instruction.
        float amax = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            x[i] *= p.qp_mul;
            amax = fmaxf(amax, fabsf(x[i]));
        }
        // 2^b brings the block's largest magnitude into [2, 4) (e2m3 holds magnitudes up to 7.5)
        int b = 0;
        if (amax > 0.f && amax < __builtin_huge_valf()) b = 1 - ilogbf(amax);
        b = b < -117 ? -117 : (b > 117 ? 117 : b);
        const int qsc = (127 - b) | ((122 - b) << 8) | ((117 - b) << 16);
        c.qscA = c.lo8 ? qsc : 0;
        c.qscB = c.lo8 ? 0 : qsc;
        // x 2^b = hi + mid / 32 + lo / 1024 + e: each part rounded to nearest even (the
        // conversion divides by its scale argument), the residuals before it exact in fp32; the
        // last part is at most 4 in magnitude, so |e| <= 2^-3 / 1024 = 2^-13 next to a block
        // maximum of at least 2.
        typedef float f32x16 __attribute__((ext_vector_type(16)));
        typedef int i32x6 __attribute__((ext_vector_type(6)));
        float r[32];
#pragma unroll
        for (int i = 0; i < 32; ++i) r[i] = ldexpf(x[i], b);
#pragma unroll
        for (int part = 0; part < 3; ++part) {
            // packed element 2i comes from the first vector's element i, 2i + 1 from the second's
            f32x16 ev, od;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                ev[i] = r[2 * i];
                od[i] = r[2 * i + 1];
            }
            const float sc = part == 0 ? 1.0f : 0.03125f;  // code = RNE(value / sc)
            const i32x6 code = __builtin_amdgcn_cvt_scalef32_2xpk16_fp6_f32(ev, od, sc);
#pragma unroll
            for (int j = 0; j < 6; ++j) c.qp6[part][j] = code[j];
            c.qp6[part][6] = 0;
            c.qp6[part][7] = 0;
            if (part < 2) {
                const auto dq = __builtin_amdgcn_cvt_scalef32_pk32_f32_fp6(code, 1.0f);
#pragma unroll
                for (int i = 0; i < 32; ++i) r[i] = part == 0 ? r[i] - dq[i] : __builtin_fmaf(r[i], 32.f, -dq[i]);
            }
        }
    } else {
        c.qscA = c.qscB = 127;
    }
}

// SPV: Sparse-V off (0), on (1), on with skip statistics (2); separate instances keep the test
// and the counting off the paths that do not use them.
// ADDR: how K / V tiles are addressed and cached.
//   TQ_ADDR_CACHED: 32-bit offsets from one descriptor per head; loads allocate in the caches
//       (K + V fit the 256 MB last-level cache, so repeated decodes of them can hit there);
//   TQ_ADDR_STREAM: the same addressing with non-temporal (streaming) loads, for caches larger
//       than the last-level cache, where every byte is read once per decode;
//   TQ_ADDR_BIG: a cache spanning 2 GiB or more: tiles addressed from 64-bit per-tile bases,
//       streaming loads.
template <int KB, bool KQJL, int VB, int SPV, int ADDR>
__global__ __launch_bounds__((64 * fast_wg_waves<KB, KQJL, VB>()))
__attribute__((amdgpu_waves_per_eu(fast_waves<KB, KQJL, VB>(), fast_waves<KB, KQJL, VB>())))
void decode_fast_kernel(FastDecodeParams p) {
    constexpr bool BIG = ADDR == TQ_ADDR_BIG;
    constexpr int AUX = ADDR == TQ_ADDR_CACHED ? 0 : 2;  // buffer-load cache policy: 2 = non-temporal
    extern __shared__ uint32_t s_lds[];
    const int tid = threadIdx.x;
    const uint32_t staged = stage_value<KB, VB>(p, tid);
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wpg = (int)(__builtin_amdgcn_workgroup_size_x() >> 6);  // waves per workgroup
    const int wv = (int)blockIdx.x * wpg + wave;  // this wave's unit (chunks) or worker (balanced)
    const int cap = p.max_blocks * p.block_size;

    // ---- this wave's work, settled before the tables are built: idle workgroups skip them ----
    // Balanced schedule: the pair range [bal_pos, bal_end) of worker wv and the sequence bal_s
    // (bal_np pairs per KV head, bal_q pairs per KV head before it) that holds its first pair.
    int bal_pos = 0, bal_end = 0, bal_q = 0;  // below 2^31 pairs (checked on the host)
    int bal_s = 0, bal_np = 0;
    if (p.balanced) {
        // the first 64 sequences' pairs and prefix sums are kept for the second pass
        const uint32_t np0 = lane < p.num_seqs ? (uint32_t)tq_bal_pairs(tq_seq_len(p.seq_lens, lane, p.uniform_len), p.len_cap) : 0u;
        const uint32_t incl0 = wave_incl_scan_u32(np0);
        int64_t tot = (int64_t)__builtin_amdgcn_readlane(incl0, 63);
        for (int b = 64; b < p.num_seqs; b += 64) {
            const int sl = b + lane;
            const uint32_t np = sl < p.num_seqs ? (uint32_t)tq_bal_pairs(tq_seq_len(p.seq_lens, sl, p.uniform_len), p.len_cap) : 0u;
            tot += (int64_t)__builtin_amdgcn_readlane(wave_incl_scan_u32(np), 63);
        }
        const int64_t P = tot * p.hkv;
        const int64_t R = P < p.n_workers ? P : (int64_t)p.n_workers;
        const bool planner = wv == 0;  // writes the plan the merge reads
        if (wv < R) {
            bal_pos = (int)tq_bal_begin(wv, P, R);
            bal_end = (int)tq_bal_begin(wv + 1, P, R);
        }
        if (planner || wv < R) {
            int64_t carry = 0;
            bool found = wv >= R;
            for (int b = 0; b < p.num_seqs; b += 64) {
                const int sl = b + lane;
                uint32_t np = np0, incl = incl0;
                if (b > 0) {
                    np = sl < p.num_seqs ? (uint32_t)tq_bal_pairs(tq_seq_len(p.seq_lens, sl, p.uniform_len), p.len_cap) : 0u;
                    incl = wave_incl_scan_u32(np);
                }
                if (planner && sl < p.num_seqs) p.plan[1 + sl] = carry + (int64_t)(incl - np);
                if (!found) {
                    const uint64_t m =
                        __builtin_amdgcn_ballot_w64(sl < p.num_seqs && (carry + (int64_t)incl) * p.hkv > bal_pos);
                    if (m) {
                        const int l = __builtin_ctzll(m);
                        bal_s = b + l;
                        bal_np = (int)__builtin_amdgcn_readlane(np, l);
                        bal_q = (int)(carry + (int64_t)__builtin_amdgcn_readlane(incl, l)) - bal_np;
                        found = true;
                    }
                }
                carry += (int64_t)__builtin_amdgcn_readlane(incl, 63);
                if (found && !planner) break;
            }
            if (planner && lane == 0) p.plan[0] = tot;
        }
        if ((int64_t)blockIdx.x * wpg >= R) return;  // the whole workgroup idle
    } else if (!chunk_group_busy(p, cap, wpg)) {
        return;
    }
    build_tables<KB, KQJL, VB>(p, s_lds, tid, staged);

    const int g = lane >> 4;
    const int n = lane & 15;
    const int hcol = n & 7;
    LaneCtx c;
    init_lane_tables<KB, VB>(c, p, lane);

    // ---- loop-invariant lane offsets inside a tile ----
    // lane-grouped tiles: the lane's key chunk (row n, dims 32g..) and value chunk (rows
    // 4g..4g+3, dims 8n..8n+7) inside a 16-row sub-tile
    const uint32_t o_kch = (uint32_t)((4 * n + g) * (4 * KB + (KQJL ? 4 : 0)));
    const uint32_t o_vch = (uint32_t)((16 * g + n) * 4 * VB);
    const uint32_t o_norm = (uint32_t)(8 * g);  // tokens 4g..4g+3, 2 bytes each
    const uint64_t hi8 = 0xff00ff00ff00ff00ull;

    // Balanced schedule: the KV head and the pair offset of bal_pos inside its segment.
    int kh_b = 0;
    int pp = 0;
    if (p.balanced && bal_pos < bal_end) {
        const int off = bal_pos - bal_q * p.hkv;
        kh_b = off / bal_np;
        pp = off - kh_b * bal_np;
    }
    unsigned long long cnt_tot = 0, cnt_kept = 0;

    // ---- pieces: one (sequence, KV head, token range) per pass ----
    // Fixed chunks: the wave's one unit (chunk_unit).  Balanced: the segments the worker's pair
    // range crosses.
    for (;;) {
    int s;
    int kh, L, t_begin, t_end;
    bool direct;           // the piece is the whole sequence: write the output here
    int prow_base;         // partial row of the group's first head
    int prow_step;         // rows between the group's heads
    int take = 0;          // balanced: pairs of this piece
    if (!p.balanced) {
        int ci;
        if (!chunk_unit(wv, p, cap, s, ci, kh, L)) break;
        t_begin = ci * p.chunk;
        t_end = (t_begin + p.chunk < L) ? t_begin + p.chunk : L;
        int nch = (L + p.chunk - 1) / p.chunk;
        nch = nch < p.n_chunks ? nch : p.n_chunks;
        // (a rotated output is written by decode_reduce_kernel, which takes single chunks too)
        direct = nch == 1 && !p.rot_out;
        prow_base = (s * p.hq + kh * p.group) * p.n_chunks + ci;
        prow_step = p.n_chunks;
    } else {
        if (bal_pos >= bal_end) break;
        s = bal_s;
        kh = kh_b;
        L = tq_seq_len(p.seq_lens, s, p.uniform_len);
        L = L < p.len_cap ? L : p.len_cap;
        take = bal_np - pp;
        take = take < bal_end - bal_pos ? take : bal_end - bal_pos;
        t_begin = 32 * pp;
        t_end = 32 * (pp + take);
        t_end = t_end < L ? t_end : L;
        direct = pp == 0 && take == bal_np && !p.rot_out;
        prow_base = (wv + s * p.hkv + kh) * p.group;
        prow_step = 1;
    }

    // One descriptor per head (tiles at 32-bit scalar offsets from it), or, for a cache spanning
    // 2 GiB or more (BIG), one per tile from a 64-bit base.
    const uint8_t* kunit = p.kbase + (int64_t)kh * p.k_sh;
    const uint8_t* vunit = p.vbase + (int64_t)kh * p.v_sh;
    const auto rk = rsrc(kunit);
    const auto rv = rsrc(vunit);

    // ---- tile walk ----
    const int nblk_seq = (L + p.block_size - 1) / p.block_size;  // >= 1
    const int32_t* bt_row = p.bt + s * p.bt_stride;
    const int tile0 = t_begin >> 4;                               // absolute tile index of the chunk start
    const int tmask = (1 << p.tile_shift) - 1;
    // Block numbers (clamped into the sequence's blocks) of tiles t .. t + 3 of the chunk in
    // lanes 0-3 of one vector load, issued a loop iteration (two pairs) ahead of their use and
    // read with v_readlane.  (Scalar loads of them would share the LDS reads' counter, so the
    // pipelined lookups would wait for them.)
    auto bt_quad = [&](int t) -> int {
        int lb = (tile0 + t + (lane & 3)) >> p.tile_shift;
        lb = lb < nblk_seq ? lb : nblk_seq - 1;
        return bt_row[lb];
    };
    const uint32_t nblocks32 = p.num_blocks < 0x7fffffff ? (uint32_t)p.num_blocks : 0x7fffffffu;

    // Norm rows of tiles A (lanes col < 8) and B (col >= 8) in one load: the scalar offset
    // addresses the nearer tile, lanes of the farther one add the distance.
    struct NormAddr {
        uint32_t vo, so;
    };
    auto norm_addr = [&](uint32_t oA, uint32_t oB) -> NormAddr {
        const uint32_t lo = oA < oB ? oA : oB;
        const uint32_t d = (oA < oB ? oB : oA) - lo;
        const uint64_t up = oB > oA ? hi8 : ~hi8;
        return NormAddr{o_norm + (__builtin_amdgcn_inverse_ballot_w64(up) ? d : 0u), lo};
    };

    // K part of pair pi, whose tiles' block numbers are b0, b1; fills the V offsets of pi.
    auto fetch_k = [&](int pi, int b0, int b1, KRaw<KB, KQJL>& kr, PairInfo& info) {
        int blk[2] = {b0, b1};
        uint32_t kb[2], r0[2];
        int nv[2];
#pragma unroll
        for (int x = 0; x < 2; ++x) {
            const int i = 2 * pi + x;
            const int t0 = t_begin + 16 * i;
            int nvr = t_end - t0;
            nvr &= ~(nvr >> 31);  // max(., 0)
            nvr = nvr < 16 ? nvr : 16;
            int bk = blk[x];
            if ((uint32_t)bk >= nblocks32) {  // unreadable entry (negative or past the cache): read block 0, mask it
                bk = 0;
                nvr = 0;
            }
            blk[x] = bk;
            nv[x] = nvr;
            r0[x] = (uint32_t)(((tile0 + i) & tmask) << 4);
            kb[x] = BIG ? 0u : (uint32_t)bk * p.k_sb;
        }
        info.nvA = nv[0];
        info.nvB = nv[1];
        // BIG: the block numbers themselves
        info.vbA = BIG ? (uint32_t)blk[0] : (uint32_t)blk[0] * p.v_sb;
        info.vbB = BIG ? (uint32_t)blk[1] : (uint32_t)blk[1] * p.v_sb;
        info.r0A = r0[0];
        info.r0B = r0[1];
        // One load per tile: chunk (4n + g) of the 16-row sub-tile holds the lane's index
        // dwords and, with QJL, the sign dword after them (4 * (KB + QJL) bytes).
        auto load_k = [&](uint32_t (&kw)[KB], uint32_t& ks, __amdgpu_buffer_rsrc_t rk, uint32_t soff) {
            constexpr int C = 4 * KB + (KQJL ? 4 : 0);
            uint32_t d[5];
            if (C == 8) {
                tq_u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rk, o_kch, soff, AUX);
                d[0] = v[0]; d[1] = v[1];
            } else if (C == 12) {
                typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
                u32x3 v = __builtin_amdgcn_raw_buffer_load_b96(rk, o_kch, soff, AUX);
                d[0] = v[0]; d[1] = v[1]; d[2] = v[2];
            } else {
                tq_u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rk, o_kch, soff, AUX);
                d[0] = v[0]; d[1] = v[1]; d[2] = v[2]; d[3] = v[3];
                if (C == 20) d[4] = __builtin_amdgcn_raw_buffer_load_b32(rk, o_kch + 16u, soff, AUX);
            }
#pragma unroll
            for (int j = 0; j < KB; ++j) kw[j] = d[j];
            ks = KQJL ? d[KB] : 0u;
        };
        constexpr uint32_t P = 16 * KB + (KQJL ? 16 : 0);  // payload bytes per row
        if (BIG) {
            const auto rkA = rsrc(kunit + (int64_t)blk[0] * p.k_sb);
            const auto rkB = rsrc(kunit + (int64_t)blk[1] * p.k_sb);
            load_k(kr.kwA, kr.ksA, rkA, r0[0] * P);
            load_k(kr.kwB, kr.ksB, rkB, r0[1] * P);
            // lanes with col < 8 read tile A's norms, the others tile B's
            tq_u32x2 a, bb = {0u, 0u};
            if (c.lo8) {
                a = __builtin_amdgcn_raw_buffer_load_b64(rkA, o_norm, 2u * r0[0] + p.d_kn, AUX);
                if (KQJL) bb = __builtin_amdgcn_raw_buffer_load_b64(rkA, o_norm, 2u * r0[0] + p.d_krn, AUX);
            } else {
                a = __builtin_amdgcn_raw_buffer_load_b64(rkB, o_norm, 2u * r0[1] + p.d_kn, AUX);
                if (KQJL) bb = __builtin_amdgcn_raw_buffer_load_b64(rkB, o_norm, 2u * r0[1] + p.d_krn, AUX);
            }
            kr.kn[0] = a[0];
            kr.kn[1] = a[1];
            kr.krn[0] = bb[0];
            kr.krn[1] = bb[1];
            return;
        }
        load_k(kr.kwA, kr.ksA, rk, kb[0] + r0[0] * P);
        load_k(kr.kwB, kr.ksB, rk, kb[1] + r0[1] * P);
        const NormAddr na = norm_addr(kb[0] + 2u * r0[0], kb[1] + 2u * r0[1]);
        tq_u32x2 a = __builtin_amdgcn_raw_buffer_load_b64(rk, na.vo, na.so + p.d_kn, AUX);
        kr.kn[0] = a[0];
        kr.kn[1] = a[1];
        if (KQJL) {
            tq_u32x2 bb = __builtin_amdgcn_raw_buffer_load_b64(rk, na.vo, na.so + p.d_krn, AUX);
            kr.krn[0] = bb[0];
            kr.krn[1] = bb[1];
        }
    };
    auto load_v = [&](const PairInfo& info, VRaw<VB>& vr) {
        // One load per tile: chunk (16g + n) of the 16-row sub-tile, 4 * VB bytes (dims 8n..8n+7
        // of rows 4g..4g+3, dimension-major).
        auto load1 = [&](uint32_t (&vw)[VB], __amdgpu_buffer_rsrc_t rv, uint32_t soff) {
            if (VB == 2) {
                tq_u32x2 a = __builtin_amdgcn_raw_buffer_load_b64(rv, o_vch, soff, AUX);
                vw[0] = a[0]; vw[1 % VB] = a[1];
            } else if (VB == 3) {
                typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
                u32x3 a = __builtin_amdgcn_raw_buffer_load_b96(rv, o_vch, soff, AUX);
                vw[0] = a[0]; vw[1 % VB] = a[1]; vw[2 % VB] = a[2];
            } else {
                tq_u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rv, o_vch, soff, AUX);
                vw[0] = a[0]; vw[1 % VB] = a[1]; vw[2 % VB] = a[2]; vw[3 % VB] = a[3];
            }
        };
        if (BIG) {
            const auto rvA = rsrc(vunit + (int64_t)info.vbA * p.v_sb);
            const auto rvB = rsrc(vunit + (int64_t)info.vbB * p.v_sb);
            load1(vr.vwA, rvA, info.r0A * (uint32_t)(16 * VB));
            load1(vr.vwB, rvB, info.r0B * (uint32_t)(16 * VB));
            tq_u32x2 a;
            if (c.lo8) a = __builtin_amdgcn_raw_buffer_load_b64(rvA, o_norm, 2u * info.r0A + p.d_vn, AUX);
            else a = __builtin_amdgcn_raw_buffer_load_b64(rvB, o_norm, 2u * info.r0B + p.d_vn, AUX);
            vr.vn[0] = a[0];
            vr.vn[1] = a[1];
            return;
        }
        load1(vr.vwA, rv, info.vbA + info.r0A * (uint32_t)(16 * VB));
        load1(vr.vwB, rv, info.vbB + info.r0B * (uint32_t)(16 * VB));
        // norm of row j of a tile at row0 of its block: d_vn + 2 (row0 + j)
        const NormAddr na = norm_addr(info.vbA + 2u * info.r0A, info.vbB + 2u * info.r0B);
        tq_u32x2 a = __builtin_amdgcn_raw_buffer_load_b64(rv, na.vo, na.so + p.d_vn, AUX);
        vr.vn[0] = a[0];
        vr.vn[1] = a[1];
    };

    // ---- query operands: loads (converted once the first pair's loads are issued, so the
    // block-table, query and first K/V round trips overlap) ----
    const int head = kh * p.group + hcol;
    const bool hvalid = hcol < p.group;
    c.hmask = __builtin_amdgcn_ballot_w64(hvalid);
    c.gap = 1.0f / p.c_exp;
    float qv[32];
    {
        const int64_t qoff = s * p.q_ss + (int64_t)head * p.q_sh + 32 * g;
        if (hvalid && p.q_vec) {
#pragma unroll
            for (int i = 0; i < 4; ++i) tq_load8(p.q, qoff + 8 * i, p.q_dtype, &qv[8 * i]);
        } else {
#pragma unroll
            for (int i = 0; i < 32; ++i) qv[i] = hvalid ? tq_load1(p.q, qoff + i, p.q_dtype) : 0.f;
        }
    }
    // fp6 operand element m of lane group g is dim 32 g + m (the pairing of an fp4 A operand
    // with an fp6 B operand in the 16x16x128 MFMA, measured), the dims of the lane's key chunk.
    float x[32];
    if constexpr (KQJL) {
        const int64_t off = s * p.qp_ss + (int64_t)head * p.qp_sh + 32 * g;
        if (hvalid && p.q_vec) {
#pragma unroll
            for (int i = 0; i < 4; ++i) tq_load8(p.qp, off + 8 * i, p.q_dtype, &x[8 * i]);
        } else {
#pragma unroll
            for (int i = 0; i < 32; ++i) x[i] = hvalid ? tq_load1(p.qp, off + i, p.q_dtype) : 0.f;
        }
    }
    // All data of a pair is loaded one pair ahead (two register sets).  Pairs past the end read
    // block data that is never used (every fetch issues the same loads, which keeps the
    // compiler's outstanding-load counts exact).
    KRaw<KB, KQJL> kr[2];
    PairInfo info[2];
    VRaw<VB> vr[2];
    const int bt0 = bt_quad(0);  // tiles 0-3: pair 0
    // tiles 2-5: pairs 1 and 2, the first loop iteration (issued before pair 0's loads, as in
    // the loop, where it precedes two pairs' loads)
    int btw = bt_quad(2);
    fetch_k(0, __builtin_amdgcn_readlane(bt0, 0), __builtin_amdgcn_readlane(bt0, 1), kr[0], info[0]);
    load_v(info[0], vr[0]);
    // ---- query operands: conversion ----
    make_q_operands<KQJL>(c, p, qv, x);

    Softmax st;
    st.m = kNegInf;
    st.mref = kNegInf;
    st.nb = 0.f;
    st.lsum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) st.acc[i] = tq_floatx4{0.f, 0.f, 0.f, 0.f};
    st.n_tot = 0;
    st.n_kept = 0;

    const int ntiles = (t_end - t_begin + 15) >> 4;
    const int npairs = (ntiles + 1) >> 1;
    for (int i = 0; i < npairs; i += 2) {
        const int btc = btw;
        btw = bt_quad(2 * i + 6);  // the next iteration's pairs i + 3, i + 4
        fetch_k(i + 1, __builtin_amdgcn_readlane(btc, 0), __builtin_amdgcn_readlane(btc, 1), kr[1], info[1]);
        load_v(info[1], vr[1]);
        compute_pair<KB, KQJL, VB, SPV>(kr[0], vr[0], info[0], st, c, p);
        if (i + 1 >= npairs) break;
        fetch_k(i + 2, __builtin_amdgcn_readlane(btc, 2), __builtin_amdgcn_readlane(btc, 3), kr[0], info[0]);
        load_v(info[0], vr[0]);
        compute_pair<KB, KQJL, VB, SPV>(kr[1], vr[1], info[1], st, c, p);
    }

    // ---- combine the lane groups and the two tile halves ----
    float lsum = sum_over_groups(st.lsum);
    lsum += row_swap8f(lsum);
    if (SPV == 2) {
        cnt_tot += (unsigned long long)st.n_tot;
        cnt_kept += (unsigned long long)st.n_kept;
    }
    const bool writer = c.lo8 && hvalid;
    // acc[nn][r] is dim 8 * (4g + r) + nn of head col; v_cinv undoes the V table scale.
    const float vs = p.v_cinv;
    if (direct) {
        if (writer) {
            const float inv = lsum > 0.f ? vs / lsum : 0.f;
            const int64_t ob = s * p.out_ss + (int64_t)head * p.out_sh + 32 * g;
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int nn = 0; nn < 8; ++nn) tq_store1(p.out, ob + 8 * r + nn, p.out_dtype, st.acc[nn][r] * inv);
        }
    } else if (writer) {
        const int64_t slot = prow_base + (int64_t)hcol * prow_step;
        if (g == 0) {
            p.ws_m[slot] = st.mref == kNegInf ? kNegInf : st.mref * p.c_exp;  // log2 units for the merge
            p.ws_l[slot] = lsum;
        }
        float4* dst = reinterpret_cast<float4*>(p.ws_acc + slot * TQ_HEAD_DIM + 32 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            dst[2 * r] = make_float4(st.acc[0][r] * vs, st.acc[1][r] * vs, st.acc[2][r] * vs, st.acc[3][r] * vs);
            dst[2 * r + 1] = make_float4(st.acc[4][r] * vs, st.acc[5][r] * vs, st.acc[6][r] * vs, st.acc[7][r] * vs);
        }
    }
    if (!p.balanced) break;
    // next piece: the rest of the segment, the next KV head, or the next non-empty sequence
    bal_pos += take;
    pp += take;
    if (pp == bal_np) {
        pp = 0;
        if (++kh_b == p.hkv) {
            kh_b = 0;
            while (bal_pos < bal_end) {
                bal_q += bal_np;
                if (++bal_s >= p.num_seqs) {
                    bal_pos = bal_end;  // unreachable with the lengths the range was cut from
                    break;
                }
                bal_np = tq_bal_pairs(tq_seq_len(p.seq_lens, bal_s, p.uniform_len), p.len_cap);
                if (bal_np > 0) break;
            }
        }
    }
    }  // pieces
    if (SPV == 2 && lane == 0 && cnt_tot) {
        atomicAdd(p.skip_stats, cnt_tot - cnt_kept);
        atomicAdd(p.skip_stats + 1, cnt_tot);
    }
}

// ---- row-major per-sequence arrays (the layout of the reference's packed_attention) ----

// Byte a of a value chunk built by rows_to_dim_major2 holds dim 8n + kContigDim[a].
constexpr int kContigDim[8] = {0, 4, 2, 6, 1, 5, 3, 7};

// The lane's 2-bit value chunk (dims 8n..8n+7 of rows 4g..4g+3) from the four 16-bit row slices
// h[r] (dim j at bits 2j): each byte of the result holds the four rows of one dim (row r at
// bits 2r), the form the 2-bit V quad table reads; dims in the order kContigDim.  18 bit
// operations per tile instead of a layout change in memory.
__device__ __forceinline__ void rows_to_dim_major2(const uint32_t (&h)[4], uint32_t (&w)[2]) {
    const uint32_t A = h[0] | (h[2] << 16);  // rows 0 | 2
    const uint32_t B = h[1] | (h[3] << 16);  // rows 1 | 3
    // nibble k of x: dim 2(k & 3) of rows (0, 1) for k < 4, rows (2, 3) for k >= 4; y: dim 2(k & 3) + 1
    const uint32_t x = (A & 0x33333333u) | ((B << 2) & 0xccccccccu);
    const uint32_t y = ((A >> 2) & 0x33333333u) | (B & 0xccccccccu);
    // nibbles k and k + 4 side by side: bytes 0, 1 of px = dims 0, 4 (of x's parity), of qx = 2, 6
    const uint32_t px = (x & 0x0f0f0f0fu) | ((x >> 12) & 0xf0f0f0f0u);
    const uint32_t qx = ((x >> 4) & 0x0f0f0f0fu) | ((x >> 16) & 0xf0f0f0f0u);
    const uint32_t py = (y & 0x0f0f0f0fu) | ((y >> 12) & 0xf0f0f0f0u);
    const uint32_t qy = ((y >> 4) & 0x0f0f0f0fu) | ((y >> 16) & 0xf0f0f0f0u);
    w[0] = (px & 0xffffu) | (qx << 16);  // dims 0, 4, 2, 6
    w[1] = (py & 0xffffu) | (qy << 16);  // dims 1, 5, 3, 7
}

// Decode over the row-major per-sequence arrays of the reference's packed_attention
// (kernels/packed_attention.py:75-196, arrays as in :290-344): K indices (16 * KB bytes per
// row), K sign rows (16 bytes, natural or stride-4 permuted bit order), fp16 K norms and
// residual norms, V indices (16 * VB bytes), fp16 V norms, without block tables.  2-bit K with
// QJL, 2-bit V, fixed chunks, no Sparse-V and no rotation (tq_decode sends other requests to
// decode_kernel).  One wave per (sequence, KV head, chunk), pairs of 16-token tiles through
// compute_pair as in decode_fast_kernel; only the loads differ: lane (n, g) reads bytes
// 4KB*g.. of key row n (the dims 32g..32g+31 the keys tile layout gives it) and bytes 4g..4g+3
// of sign row n, whose 32 signs are dims 32g + m (natural) or 4m + g (permuted: q_proj is taken
// in that order); its value chunk comes from four 16-bit slices of rows 4g..4g+3
// (rows_to_dim_major2).  Rows past a sequence's last tile are never read (the arrays hold
// max_blocks * 16 rows per sequence; tiles past the end re-read the last one, masked).
template <int KB, bool KQJL, int VB>
__global__ __launch_bounds__((64 * fast_wg_waves<KB, KQJL, VB>()))
__attribute__((amdgpu_waves_per_eu(fast_waves<KB, KQJL, VB>(), fast_waves<KB, KQJL, VB>())))
void decode_contig_kernel(FastDecodeParams p) {
    static_assert(KB == 2 && KQJL && VB == 2, "row-major decode: 2-bit keys with QJL, 2-bit values");
    extern __shared__ uint32_t s_lds[];
    const int tid = threadIdx.x;
    const uint32_t staged = stage_value<KB, VB>(p, tid);
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wpg = (int)(__builtin_amdgcn_workgroup_size_x() >> 6);  // waves per workgroup
    const int wv = (int)blockIdx.x * wpg + wave;  // this wave's unit
    const int cap = p.max_blocks * 16;          // rows per sequence in the arrays
    if (!chunk_group_busy(p, cap, wpg)) return;
    build_tables<KB, KQJL, VB>(p, s_lds, tid, staged);
    const int g = lane >> 4;
    const int n = lane & 15;
    const int hcol = n & 7;
    LaneCtx c;
    init_lane_tables<KB, VB>(c, p, lane);

    int s, ci, kh, L;
    if (!chunk_unit(wv, p, cap, s, ci, kh, L)) return;
    const int t_begin = ci * p.chunk;
    const int t_end = t_begin + p.chunk < L ? t_begin + p.chunk : L;
    int nch = (L + p.chunk - 1) / p.chunk;
    nch = nch < p.n_chunks ? nch : p.n_chunks;
    const bool direct = nch == 1;
    const int prow_base = (s * p.hq + kh * p.group) * p.n_chunks + ci;

    const uint8_t* base[6];
#pragma unroll
    for (int a = 0; a < 6; ++a)
        base[a] = p.contig[a].ptr + (int64_t)s * p.contig[a].stride_seq + (int64_t)kh * p.contig[a].stride_head;
    const int ntl = (L + 15) >> 4;  // tiles holding the sequence's rows (>= 1)
    const int tile0 = t_begin >> 4;
    constexpr uint32_t KROW = 16 * KB, VROW = 16 * VB;
    const uint32_t o_ki = (uint32_t)(n * KROW + 4 * KB * g);    // key row n, dims 32g..
    const uint32_t o_ks = (uint32_t)(n * 16 + 4 * g);           // sign row n, bytes 4g..
    const uint32_t o_v = (uint32_t)(4 * g * VROW + VB * n);     // value row 4g, dims 8n..
    const uint32_t o_n = (uint32_t)(8 * g);                     // norms of rows 4g..4g+3

    struct VRows {
        uint32_t hA[4], hB[4];  // 16-bit slices of rows 4g..4g+3, tiles A and B
        uint32_t vn[2];
    };
    auto ld2 = [](const uint8_t* b, uint32_t off) { return *reinterpret_cast<const tq_u32x2*>(b + off); };
    auto ld1 = [](const uint8_t* b, uint32_t off) { return *reinterpret_cast<const uint32_t*>(b + off); };
    auto ldh = [](const uint8_t* b, uint32_t off) { return (uint32_t)*reinterpret_cast<const uint16_t*>(b + off); };
    auto fetch = [&](int pi, KRaw<KB, KQJL>& kr, VRows& vw, PairInfo& info) {
        int nv[2];
        uint32_t ti[2];
#pragma unroll
        for (int x = 0; x < 2; ++x) {
            const int i = 2 * pi + x;
            int nvr = t_end - (t_begin + 16 * i);
            nvr &= ~(nvr >> 31);  // max(., 0)
            nv[x] = nvr < 16 ? nvr : 16;
            const int t = tile0 + i;
            ti[x] = (uint32_t)(t < ntl ? t : ntl - 1);  // past the end: the last tile again (masked)
        }
        info.nvA = nv[0];
        info.nvB = nv[1];
        const tq_u32x2 a = ld2(base[0], ti[0] * (16 * KROW) + o_ki);
        const tq_u32x2 b = ld2(base[0], ti[1] * (16 * KROW) + o_ki);
        kr.kwA[0] = a[0];
        kr.kwA[1] = a[1];
        kr.kwB[0] = b[0];
        kr.kwB[1] = b[1];
        kr.ksA = ld1(base[1], ti[0] * 256u + o_ks);
        kr.ksB = ld1(base[1], ti[1] * 256u + o_ks);
        // lanes with col < 8 read tile A's norms, the others tile B's
        const uint32_t no = (c.lo8 ? ti[0] : ti[1]) * 32u + o_n;
        const tq_u32x2 kn = ld2(base[2], no), krn = ld2(base[3], no), vn = ld2(base[5], no);
        kr.kn[0] = kn[0];
        kr.kn[1] = kn[1];
        kr.krn[0] = krn[0];
        kr.krn[1] = krn[1];
        vw.vn[0] = vn[0];
        vw.vn[1] = vn[1];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            vw.hA[r] = ldh(base[4], ti[0] * (16 * VROW) + o_v + r * VROW);
            vw.hB[r] = ldh(base[4], ti[1] * (16 * VROW) + o_v + r * VROW);
        }
    };

    // ---- query operands ----
    const int head = kh * p.group + hcol;
    const bool hvalid = hcol < p.group;
    c.hmask = __builtin_amdgcn_ballot_w64(hvalid);
    c.gap = 1.0f / p.c_exp;
    float qv[32], x[32];
    {
        const int64_t qoff = s * p.q_ss + (int64_t)head * p.q_sh + 32 * g;
        if (hvalid && p.q_vec) {
#pragma unroll
            for (int i = 0; i < 4; ++i) tq_load8(p.q, qoff + 8 * i, p.q_dtype, &qv[8 * i]);
        } else {
#pragma unroll
            for (int i = 0; i < 32; ++i) qv[i] = hvalid ? tq_load1(p.q, qoff + i, p.q_dtype) : 0.f;
        }
        // element m of lane group g pairs with sign bit 32g + m of the row: dim 32g + m, or 4m + g
        // in the permuted order
        const int64_t poff = s * p.qp_ss + (int64_t)head * p.qp_sh;
        if (p.contig_perm) {
#pragma unroll
            for (int m = 0; m < 32; ++m) x[m] = hvalid ? tq_load1(p.qp, poff + 4 * m + g, p.q_dtype) : 0.f;
        } else if (hvalid && p.q_vec) {
#pragma unroll
            for (int i = 0; i < 4; ++i) tq_load8(p.qp, poff + 32 * g + 8 * i, p.q_dtype, &x[8 * i]);
        } else {
#pragma unroll
            for (int m = 0; m < 32; ++m) x[m] = hvalid ? tq_load1(p.qp, poff + 32 * g + m, p.q_dtype) : 0.f;
        }
    }
    KRaw<KB, KQJL> kr[2];
    VRows vw[2];
    PairInfo info[2];
    fetch(0, kr[0], vw[0], info[0]);
    make_q_operands<KQJL>(c, p, qv, x);

    Softmax st;
    st.m = kNegInf;
    st.mref = kNegInf;
    st.nb = 0.f;
    st.lsum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) st.acc[i] = tq_floatx4{0.f, 0.f, 0.f, 0.f};
    st.n_tot = 0;
    st.n_kept = 0;
    auto compute = [&](const KRaw<KB, KQJL>& k, const VRows& v, const PairInfo& pi) {
        VRaw<VB> vr;
        rows_to_dim_major2(v.hA, vr.vwA);
        rows_to_dim_major2(v.hB, vr.vwB);
        vr.vn[0] = v.vn[0];
        vr.vn[1] = v.vn[1];
        compute_pair<KB, KQJL, VB, 0>(k, vr, pi, st, c, p);
    };
    const int ntiles = (t_end - t_begin + 15) >> 4;
    const int npairs = (ntiles + 1) >> 1;
    for (int i = 0; i < npairs; i += 2) {
        fetch(i + 1, kr[1], vw[1], info[1]);
        compute(kr[0], vw[0], info[0]);
        if (i + 1 >= npairs) break;
        fetch(i + 2, kr[0], vw[0], info[0]);
        compute(kr[1], vw[1], info[1]);
    }

    // ---- combine the lane groups and the two tile halves; acc[a][r] is dim 8(4g + r) + kContigDim[a] ----
    float lsum = sum_over_groups(st.lsum);
    lsum += row_swap8f(lsum);
    if (!(c.lo8 && hvalid)) return;
    const float vs = p.v_cinv;
    if (direct) {
        const float inv = lsum > 0.f ? vs / lsum : 0.f;
        const int64_t ob = s * p.out_ss + (int64_t)head * p.out_sh + 32 * g;
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int a = 0; a < 8; ++a) tq_store1(p.out, ob + 8 * r + kContigDim[a], p.out_dtype, st.acc[a][r] * inv);
    } else {
        const int64_t slot = prow_base + (int64_t)hcol * p.n_chunks;
        if (g == 0) {
            p.ws_m[slot] = st.mref == kNegInf ? kNegInf : st.mref * p.c_exp;  // log2 units for the merge
            p.ws_l[slot] = lsum;
        }
        float4* dst = reinterpret_cast<float4*>(p.ws_acc + slot * TQ_HEAD_DIM + 32 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            dst[2 * r] = make_float4(st.acc[0][r] * vs, st.acc[4][r] * vs, st.acc[2][r] * vs, st.acc[6][r] * vs);
            dst[2 * r + 1] = make_float4(st.acc[1][r] * vs, st.acc[5][r] * vs, st.acc[3][r] * vs, st.acc[7][r] * vs);
        }
    }
}

}  // namespace

const void* tq_decode_fast_kernel_ptr(int kb, bool kq, int vb, int spv, int addr) {
    if (addr == TQ_ADDR_CONTIG)
        return (kb == 2 && kq && vb == 2 && spv == 0) ? (const void*)decode_contig_kernel<2, true, 2> : nullptr;
#define TQ_FP_A(KB, KQ, VB, A)                                                                         \
    if (addr == A)                                                                                     \
        return spv == 2 ? (const void*)decode_fast_kernel<KB, KQ, VB, 2, A>                            \
               : spv == 1 ? (const void*)decode_fast_kernel<KB, KQ, VB, 1, A>                          \
                          : (const void*)decode_fast_kernel<KB, KQ, VB, 0, A>;
#define TQ_FP(KB, KQ, VB)                                                                              \
    if (kb == KB && kq == KQ && vb == VB) {                                                            \
        TQ_FP_A(KB, KQ, VB, TQ_ADDR_CACHED) TQ_FP_A(KB, KQ, VB, TQ_ADDR_STREAM) TQ_FP_A(KB, KQ, VB, TQ_ADDR_BIG) \
        return nullptr;                                                                                \
    }
#define TQ_FP_V(KB, KQ) TQ_FP(KB, KQ, 2) TQ_FP(KB, KQ, 3) TQ_FP(KB, KQ, 4)
    TQ_FP_V(2, false) TQ_FP_V(2, true) TQ_FP_V(3, false) TQ_FP_V(3, true) TQ_FP_V(4, false) TQ_FP_V(4, true)
#undef TQ_FP_V
#undef TQ_FP
#undef TQ_FP_A
    return nullptr;
}

void tq_decode_fast_lds_layout(int kb, bool kq, int vb, bool share, FastLdsLayout* l) {
    *l = FastLdsLayout{};
    // 3-bit quad tables in [0, 64 KB): K at 0, then V's own
    uint32_t end3 = 0;
    if (kb == 3) end3 = 32768;
    if (vb == 3 && !share) {
        l->v = end3;
        end3 += 32768;
    }
    // row tables in 64 KB regions after them: a full row each when there are enough regions
    // (2 without 3-bit tables, 1 with: 128 KB in all), else the first two share a region's
    // rows in 128-byte halves
    struct Row {
        uint32_t* off;
        uint32_t* rep;
        uint32_t es;
    } rt[3];
    int n = 0;
    if (kb != 3) rt[n++] = {&l->k, &l->rep_k, kb == 2 ? 8u : 4u};
    if (vb != 3 && !share) rt[n++] = {&l->v, &l->rep_v, vb == 2 ? 8u : 4u};
    if (kq) rt[n++] = {&l->sign, &l->rep_s, 4u};
    const int regions = end3 ? 1 : 2;
    const int halves = n > regions ? 2 : 0;
    uint32_t reg = end3 ? 65536u : 0u;
    for (int i = 0; i < n; ++i) {
        if (i < halves) {
            *rt[i].off = reg + 128u * (uint32_t)(i & 1);
            *rt[i].rep = 128u / rt[i].es - 1u;
            if (i & 1) reg += 65536u;
        } else {
            *rt[i].off = reg;
            *rt[i].rep = 256u / rt[i].es - 1u;
            reg += 65536u;
        }
    }
    if (share) {
        l->v = l->k;
        l->rep_v = l->rep_k;
    }
    // 512 bytes of scratch (pairs of 3-bit fields while a quad table is built): the hole
    // between one 3-bit table and the row regions, else at the end
    const uint32_t end = n ? reg : end3;
    l->scratch = (end3 == 32768 && n) ? 32768u : end;
    l->total = (size_t)(end > l->scratch + 512 ? end : l->scratch + 512);
}

int tq_decode_fast_lds_attr(const void* kern) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    static std::mutex mu;
    static std::set<std::pair<const void*, int>> done;
    std::lock_guard<std::mutex> lk(mu);
    if (done.count({kern, dev})) return TQ_OK;
    e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kTqFastLdsMax);
    if (e != hipSuccess) return (int)e;
    done.insert({kern, dev});
    return TQ_OK;
}

int tq_decode_fast_wg_waves(int kb, bool kq, int vb, size_t lds_bytes) {
    (void)kb;
    (void)vb;
    const int cu_waves = kq ? fast_wg_waves<2, true, 2>() : fast_wg_waves<2, false, 2>();
    // workgroups whose tables fit a compute unit's LDS together, a divisor of its waves
    int wgs = lds_bytes ? (int)(kTqLdsPerCu / lds_bytes) : 4;
    wgs = wgs < 1 ? 1 : wgs > 4 ? 4 : wgs;
    while (cu_waves % wgs) --wgs;
    return cu_waves / wgs;
}

int tq_decode_fast_launch(const FastDecodeParams& prm, int kb, bool kq, int vb, int64_t grid, size_t lds_bytes,
                          hipStream_t stream) {
    const void* kern = tq_decode_fast_kernel_ptr(kb, kq, vb, !prm.sparse ? 0 : prm.skip_stats ? 2 : 1, prm.addr);
    if (!kern) return TQ_ERR_BITS;
    const int arc = tq_decode_fast_lds_attr(kern);
    if (arc) return arc;
    FastDecodeParams p = prm;
    void* args[] = {&p};
    const unsigned threads = 64u * (unsigned)tq_decode_fast_wg_waves(kb, kq, vb, lds_bytes);
    hipError_t le = hipLaunchKernel(kern, dim3((unsigned)grid), dim3(threads), args, lds_bytes, stream);
    if (le != hipSuccess) return (int)le;
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TQ_OK : (int)e;
}
