// Internal interface between tq_decode (tq_decode.hip) and the paged fast-path decode kernel
// (tq_decode_fast.hip).  Not part of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "turboquant_hip.h"

// ---- balanced split-K schedule (tokens_per_chunk = 0) ----
// The work is the stream of 32-token tile pairs of every (sequence, KV head) segment, sequences
// in order and the KV heads of a sequence after each other: segment (s, kh) holds
// np(s) = ceil(min(seq_len[s], len_cap) / 32) pairs and starts at pair hkv * Q(s) + kh * np(s),
// Q(s) being the sum of np over the sequences before s.  With P pairs in all and R workers
// (waves; R <= P, so none is empty) worker w takes pairs [floor(w P / R), floor((w + 1) P / R)),
// which may cross segments.  The partial result of worker w for segment g = s * hkv + kh sits
// in partial slot w + g: along the workers the touched segments never decrease, so w + g never
// repeats, and slots stay below R + num_seqs * hkv.
__host__ __device__ inline int64_t tq_bal_begin(int64_t w, int64_t P, int64_t R) { return w * P / R; }
// the worker holding pair x (0 <= x < P): the largest w with floor(w P / R) <= x
__host__ __device__ inline int64_t tq_bal_worker(int64_t x, int64_t P, int64_t R) { return ((x + 1) * R - 1) / P; }
__host__ __device__ inline int tq_bal_pairs(int len, int len_cap) {
    len = len < len_cap ? len : len_cap;
    return len > 0 ? (len + 31) >> 5 : 0;
}
// Workspace of the balanced schedule: the plan (int64: total pairs per KV head, then Q(s) for
// every sequence, written by the decode kernel for the merge), then acc / m / l rows for
// kTqBalRowsPerCu * CUs + num_seqs * num_q_heads (sequence, query head) partials.
constexpr int kTqBalRowsPerCu = 128;  // 16 resident waves per CU x 8 query heads per group

// Length of sequence s: seq_lens[s], or `uniform` when the caller gave no lengths (every sequence
// holds max_seq_len tokens).
__device__ __forceinline__ int tq_seq_len(const int32_t* seq_lens, int64_t s, int uniform) {
    return seq_lens ? seq_lens[s] : uniform;
}

struct FastDecodeParams {
    const void* q;
    int64_t q_ss, q_sh;
    const void* qp;
    int64_t qp_ss, qp_sh;
    int q_dtype;
    int q_vec;             // q and qp rows 16-byte aligned: vector loads
    int num_seqs, hq, hkv, group;
    // K cache: index region base, head stride, block stride; other regions as byte offsets
    // from the index region of the same tile (rows: idx 16*bits, signs 16, norms 2 bytes)
    const uint8_t* kbase;
    int64_t k_sh;
    uint32_t k_sb;
    uint32_t d_kn, d_krn;  // norm regions (the signs sit in the lane-grouped payload)
    const uint8_t* vbase;
    int64_t v_sh;
    uint32_t v_sb;
    uint32_t d_vn;
    const float* k_cent;
    const float* v_cent;
    float k_cscale, v_cscale, v_cinv;
    uint32_t lds_sign, lds_k, lds_v;  // byte offsets of the LDS tables
    uint32_t rep_s, rep_k, rep_v;     // row tables: replicas - 1 (a power of two minus one)
    uint32_t lds_scratch;             // 512 bytes of scratch (3-bit quad tables' build)
    int block_size, tile_shift;       // block_size = 16 << tile_shift
    int64_t num_blocks;
    const int32_t* bt;
    int64_t bt_stride;
    int max_blocks;
    const int32_t* seq_lens;  // null: every sequence holds uniform_len tokens
    int uniform_len;
    float c_exp;     // sm_scale * log2(e) / k_cscale: raw score units -> log2 units
    float thr_log;   // log2(threshold) / c_exp
    int sparse;
    int sparse_pair; // Sparse-V running max per 32-token pair (block_size >= 32) instead of per tile
    float qp_mul;    // corr_scale * k_cscale
    int chunk, n_chunks;
    int balanced;     // balanced schedule (chunk and n_chunks unused)
    int n_workers;    // balanced: resident waves of the launch (R before the min with P)
    int len_cap;      // balanced: tokens of a sequence processed at most
    int64_t* plan;    // balanced: [1 + num_seqs] int64 written by worker 0
    float* ws_acc;   // chunks: [num_seqs][hq][n_chunks][128]; balanced: [slot][group][128]
    float* ws_m;     // [num_seqs][hq][n_chunks], log2 units
    float* ws_l;
    unsigned long long* skip_stats;
    void* out;
    int out_dtype;
    int64_t out_ss, out_sh;
    int rot_q, rot_qp, rot_out;  // rotate q / q_proj by H on load, the output by H on the write
    float wht_h;                 // 1 / sqrt(128)
    int addr;                    // TQ_ADDR_*: tile addressing and cache policy of the K / V loads
    // TQ_ADDR_CONTIG (decode_contig_kernel): row-major per-sequence arrays, in this order K
    // indices, K sign rows, K norms, K residual norms, V indices, V norms; rows of sequence s,
    // KV head kh at ptr + s * stride_seq + kh * stride_head
    struct {
        const uint8_t* ptr;
        int64_t stride_seq, stride_head;
    } contig[6];
    int contig_perm;             // sign rows in the stride-4 permuted order
};

// Tile addressing and cache policy of decode_fast_kernel's K / V loads.
enum {
    TQ_ADDR_CACHED = 0,  // 32-bit offsets per head; loads allocate in the caches
    TQ_ADDR_STREAM = 1,  // 32-bit offsets per head; non-temporal loads
    TQ_ADDR_BIG = 2,     // 64-bit per-tile bases (a cache spanning 2 GiB or more); non-temporal loads
    TQ_ADDR_CONTIG = 3,  // row-major per-sequence arrays without block tables (decode_contig_kernel)
};
// K + V caches larger than this (the MI355X last-level "Infinity" cache, 256 MB) are read with
// non-temporal loads: every byte is read once per decode and nothing would be kept anyway.
constexpr int64_t kTqStreamBytes = 256ll << 20;

// decode_fast_kernel<kb, kq, vb, spv, addr> (nullptr: unsupported bit widths); spv: Sparse-V off
// (0), on (1), on with skip statistics (2).
const void* tq_decode_fast_kernel_ptr(int kb, bool kq, int vb, int spv = 0, int addr = TQ_ADDR_CACHED);

// LDS layout of decode_fast_kernel / decode_contig_kernel: byte offsets of the fp4 sign table,
// the K and the V tables and a 512-byte scratch, the replica counts - 1 of the row tables (2-bit
// quads, 4-bit pairs, signs; 0 for a 3-bit quad table), and the total (at most kTqFastLdsMax).
struct FastLdsLayout {
    uint32_t sign, k, v, scratch;
    uint32_t rep_s, rep_k, rep_v;
    size_t total;
};
constexpr size_t kTqFastLdsMax = 131584;  // 128 KB of tables + the scratch
void tq_decode_fast_lds_layout(int kb, bool kq, int vb, bool share, FastLdsLayout* l);

// Waves per workgroup of the fast kernels for tables of lds_bytes: the compute unit's resident
// waves (4 x waves per SIMD) split over as many workgroups as the LDS (kTqLdsPerCu) holds.
constexpr size_t kTqLdsPerCu = 163840;
int tq_decode_fast_wg_waves(int kb, bool kq, int vb, size_t lds_bytes);

// Raise a fast kernel instance's dynamic-LDS limit to kTqFastLdsMax on the current device (once
// per instance and device).
int tq_decode_fast_lds_attr(const void* kern);

// Launch decode_fast_kernel (grid of workgroups of tq_decode_fast_wg_waves(..., lds_bytes)
// waves, one work unit or worker each).
int tq_decode_fast_launch(const FastDecodeParams& p, int kb, bool kq, int vb, int64_t grid, size_t lds_bytes,
                          hipStream_t stream);

// The implementation behind tq_decode (rotate = 0) and tq_decode_rotated (rotate = 1): the
// same arguments, checks and launches.
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
                   tq_stream_t stream);
