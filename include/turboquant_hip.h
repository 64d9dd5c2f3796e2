/*
 * turboquant_hip.h — C ABI of libturboquant_hip.so, the MI355X (gfx950) kernels
 * behind the TurboQuant packed-KV hot path.
 *
 * Every entry point:
 *   - takes plain device pointers, sizes and byte strides (no framework types);
 *   - launches asynchronously on the given stream and never allocates device memory
 *     (outputs and workspaces are caller-owned; tq_decode_noalloc uses a fixed array of the
 *     library instead of a workspace);
 *   - returns TQ_OK, a negative TQ_ERR_* code for an argument rejected on the host
 *     before any launch, or a positive hipError_t reported by the launch.
 *
 * Head dimension is fixed at 128 (the only size the reference's kernels support,
 * turboquant/kernels/packed_compress.py:244, packed_attention.py:348, sparse_v.py:19).
 *
 * Bit formats (per token, little-endian bit streams; identical to the reference):
 *   indices, b bits each : index of dim d in bits [b*d, b*d+b) of a 16*b-byte row
 *                          (2-bit: packed_compress.py:79-90; 3-bit: sparse_v.py:57-60,82-98;
 *                           4-bit nibble order: docs/design/AITER_TURBO4_DESIGN.md:57-76)
 *   QJL signs            : bit d of a 16-byte row is 1 when the residual projection is >= 0
 *                          (packed_compress.py:77,92-106); "permuted" rows hold bit 32c+k = dim 4k+c
 *                          (packed_compress.py:180-216)
 *   norms, residual norms: IEEE fp16.
 */
#ifndef TURBOQUANT_HIP_H
#define TURBOQUANT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* tq_stream_t; /* == hipStream_t */

/* ---- status codes ------------------------------------------------------------ */
#define TQ_OK                   0
#define TQ_ERR_INVALID_ARGUMENT (-1)
#define TQ_ERR_HEAD_DIM         (-2)  /* head_dim != 128 */
#define TQ_ERR_BITS             (-3)  /* bits outside the supported set */
#define TQ_ERR_ALIGNMENT        (-4)  /* pointer or stride not aligned as documented */
#define TQ_ERR_WORKSPACE        (-5)  /* workspace smaller than tq_decode_workspace_bytes() */
#define TQ_ERR_GQA              (-6)  /* num_q_heads / num_kv_heads not an integer in [1,16] */
#define TQ_ERR_DTYPE            (-7)
#define TQ_ERR_BLOCK_SIZE       (-8)  /* block_size not a positive multiple of 16 */
#define TQ_ERR_CHUNK            (-9)  /* tokens_per_chunk not 0 or a positive multiple of 16 */
#define TQ_ERR_SCRATCH_LIMIT    (-10) /* tq_decode_noalloc: the call needs more than the fixed scratch */

/* ---- dtype codes ------------------------------------------------------------- */
#define TQ_F32  0
#define TQ_F16  1
#define TQ_BF16 2
#define TQ_I32  3
#define TQ_I64  4

/* Version of this ABI (bumped on any signature or layout change). */
int tq_abi_version(void);

/* Human-readable text for a status code returned by any tq_* function. */
const char* tq_status_string(int status);

/* ---- compression ------------------------------------------------------------- */

/*
 * PolarQuant compression of n_rows vectors of 128 dims, unpacked outputs.
 * Replaces turboquant/core/quantizer.py:111-183 (polarquant_compress).
 *   rotate = 1: x_rot = x @ H with H the normalized Walsh-Hadamard matrix
 *               (core/rotation.py:28-44), H[i][j] = (-1)^popcount(i&j) * wht_scale;
 *   rotate = 0: x is already rotated (rotation_matrix=None).
 *   norms = |x_rot|; x_n = x_rot / (norms + 1e-8); idx = #{boundaries < x_n} (searchsorted,
 *   left), NaN -> 2^bits-1; k_mse = centroids[idx] * norms.
 *   use_qjl: r = (x_n - centroids[idx]) * norms; rnorm = |r|; sign = (r >= 0) ? +1 : -1.
 * x: [n_rows, 128] rows at x_row_stride elements. centroids [2^bits], boundaries [2^bits-1]: f32.
 * Outputs (contiguous): indices int64 [n_rows,128]; norms f32 [n_rows]; k_mse f32 [n_rows,128];
 * signs f32 [n_rows,128] and rnorm f32 [n_rows] (only read when use_qjl; may be NULL otherwise).
 * bits: 1..4.
 */
int tq_polarquant_compress(const void* x, int x_dtype, int64_t x_row_stride, int64_t n_rows,
                           int head_dim, int rotate, float wht_scale,
                           const float* centroids, const float* boundaries, int bits, int use_qjl,
                           int64_t* indices, float* norms, float* k_mse, float* signs, float* rnorm,
                           tq_stream_t stream);

/*
 * polarquant_compress with a general rotation matrix (core/quantizer.py:111-183,
 * rotation_matrix not the Walsh-Hadamard matrix): x_rot = x @ rotation, then the same math and
 * outputs as tq_polarquant_compress.  rotation: f32 [128][128] row-major (contiguous).  The
 * product is fp32 (FMA over d ascending).
 */
int tq_polarquant_compress_matrix(const void* x, int x_dtype, int64_t x_row_stride, int64_t n_rows,
                                  int head_dim, const float* rotation,
                                  const float* centroids, const float* boundaries, int bits, int use_qjl,
                                  int64_t* indices, float* norms, float* k_mse, float* signs, float* rnorm,
                                  tq_stream_t stream);

/*
 * Packed K / V compression with explicit rotation matrices.  Replaces compress_k / compress_v
 * and the _fully_packed_k / _fully_packed_v kernels (kernels/packed_compress.py:44-142,157-177,
 * 226-240):
 *   norm = |x|; x_n = x * (1 / (norm + 1e-8)); rot = x_n @ pit; idx = #{boundaries <= rot};
 *   K (pist != NULL): resid = (rot - centroids[idx]) * norm; rnorm = |resid|;
 *                     proj = resid @ pist; sign bit = proj >= 0.
 * pit, pist: f32 [128][128] row-major.  The products run on the matrix cores with each operand
 * split into fp16 hi + lo (error <= 1.77e-6 x column norm + 3.4e-7, derived in tq_packed.hip);
 * every index within 2^-19 x the largest column norm of pit + 2^-21 of a boundary is decided
 * from the row's fp64 norm and dot product, so the indices equal those of an exact (fp64)
 * computation except within fp32 rounding of a boundary.  The reference's fp16 dot products are not reproduced.  Outputs (contiguous rows):
 * idx_out u8 [n_rows][16*bits] little-endian bit stream (2 bits: byte j = sum_c idx[4j+c] << 2c),
 * signs_out u8 [n_rows][16] (bit b of byte j = dim 8j+b), rnorm_out / norm_out fp16 [n_rows]
 * (uint16 storage).  signs_out and rnorm_out are read only with pist.  bits: 1..4 (the
 * reference: 2).  pit / pist 16-byte aligned.  Needs 139,264 B (K) / 69,632 B (V) of dynamic
 * LDS per workgroup plus the kernel's static arrays (about 2 KB); TQ_ERR_WORKSPACE if the device
 * has less.
 */
int tq_compress_packed(const void* x, int x_dtype, int64_t x_row_stride, int64_t n_rows, int head_dim,
                       const float* pit, const float* pist, const float* centroids, const float* boundaries,
                       int bits, uint8_t* idx_out, uint8_t* signs_out, uint16_t* rnorm_out, uint16_t* norm_out,
                       tq_stream_t stream);

/*
 * Paged tile layouts (tile_layout of tq_compress_paged, layout of tq_kv_view).  A tile holds
 * the block_size tokens of one (physical block, KV head): a payload region of block_size * P
 * bytes, P = 16*bits (+ 16 with QJL signs), then [block_size fp16 norms][block_size fp16
 * residual norms, QJL only].  Per token the bytes are the reference's: the index fields as a
 * little-endian bit stream (16*bits bytes), the 16 sign bytes (bit d = dim d), fp16 norms.  The
 * payload is stored per 16-token sub-tile j (rows 16j..16j+15, 16*P bytes at j*16*P):
 *   TQ_TILE_ROWS   the index rows of all block_size tokens (16*bits bytes each), then their
 *                  sign rows (16 bytes each), at the offsets tq_tile_offsets returns (no
 *                  sub-tile split);
 *   TQ_TILE_KEYS   chunk (4n + g) of C = 4*bits (+ 4) bytes for row n (0..15) and dim quarter
 *                  g (dims 32g..32g+31): the 4*bits index bytes of those dims, then their 4
 *                  sign bytes (QJL) - what one lane of the decode kernel reads for one key;
 *   TQ_TILE_VALUES chunk (16g + n) of 4*bits bytes for row group g (rows 4g..4g+3) and dim
 *                  group n (dims 8n..8n+7): a little-endian stream of 32 bits-wide fields,
 *                  field 4j + r = dim 8n + j of row 4g + r (dimension-major; no QJL) - what
 *                  one lane reads for the value product, the four rows of a dim side by side.
 *                  The fields of one chunk belong to four rows: a one-row write sets its own
 *                  fields with atomic and / or (ABI version 3; version 2 was row-major).
 * The lane-grouped layouts let a decode lane fetch its key data and its value data for a
 * 16-token tile with one load each.
 */
#define TQ_TILE_ROWS   0
#define TQ_TILE_KEYS   1
#define TQ_TILE_VALUES 2

/*
 * Fused paged compression: x [num_tokens, num_heads, 128] -> packed rows written into the
 * paged cache at slot_mapping[t] (block = slot / block_size, row = slot % block_size).
 * Negative slots are skipped (the reference clamps them to 0, integration/vllm_backend.py:223-230).
 * Math as tq_polarquant_compress; stored: index bits, fp16 norm and, with use_qjl, sign bits
 * and fp16 residual norm, in the tile layout tile_layout (TQ_TILE_VALUES: no QJL).
 * Cache: one tile per (physical block, KV head) at cache + block*stride_block + head*stride_head,
 * tq_tile_bytes() bytes.
 * Requirements: cache, strides 16-byte aligned; block_size multiple of 16; bits 2..4.
 * Slots >= num_blocks*block_size are skipped.
 * Replaces turbo4_fp8_compress_and_scatter (integration/vllm_backend.py:179-230) and the
 * per-head _fully_packed_k/_v launches of benchmarks/bench_kernels.py:464-470.
 */
int tq_compress_paged(const void* x, int x_dtype, int64_t x_stride_token, int64_t x_stride_head,
                      int64_t num_tokens, int num_heads, int head_dim,
                      const void* slot_mapping, int slot_dtype,
                      void* cache, int64_t cache_stride_block, int64_t cache_stride_head,
                      int64_t num_blocks, int block_size,
                      int bits, int use_qjl, int tile_layout, int rotate, float wht_scale,
                      const float* centroids, const float* boundaries,
                      tq_stream_t stream);

/* One tensor of a K + V cache update: its rows x[token, head, :] (dtype and strides as in
 * tq_compress_paged), its paged cache and format, and its codebook. */
typedef struct tq_paged_target {
    const void* x;
    int64_t x_stride_token, x_stride_head;   /* elements */
    void* cache;
    int64_t cache_stride_block, cache_stride_head;
    int bits, use_qjl, tile_layout;
    const float* centroids;
    const float* boundaries;
} tq_paged_target;

/* tq_compress_paged of K and of V for the same tokens and slots, in one launch when K and V have
 * the same bits and V has no QJL (otherwise two launches, same results).  Each target follows the
 * rules of tq_compress_paged; num_blocks and block_size are shared.
 * Replaces the pair of turbo4_fp8_compress_and_scatter calls of one attention layer (kv_idx 0
 * and 1, integration/vllm_backend.py:179-230). */
int tq_compress_paged_kv(const tq_paged_target* k, const tq_paged_target* v, int x_dtype,
                         int64_t num_tokens, int num_heads, int head_dim,
                         const void* slot_mapping, int slot_dtype, int64_t num_blocks, int block_size,
                         int rotate, float wht_scale, tq_stream_t stream);

/* Bytes of one (block, KV head) tile (any layout) and the byte offsets of its regions in the
 * TQ_TILE_ROWS layout (the lane-grouped layouts keep off_idx = 0, off_norm and off_rnorm; their
 * signs are inside the payload). */
int64_t tq_tile_bytes(int block_size, int bits, int use_qjl);
int tq_tile_offsets(int block_size, int bits, int use_qjl,
                    int64_t* off_idx, int64_t* off_signs, int64_t* off_norm, int64_t* off_rnorm);

/* ---- decode attention --------------------------------------------------------- */

/* Where one stream of per-token data lives. Address of token row r of block blk, KV head h:
 *   ptr + blk*stride_block + h*stride_head + r*stride_row            (block_tables != NULL)
 *   ptr + s*stride_seq + lb*stride_block + h*stride_head + r*stride_row (block_tables == NULL,
 *                                                                        lb = logical block) */
typedef struct tq_region {
    const void* ptr;
    int64_t stride_block;
    int64_t stride_head;
    int64_t stride_seq;
    int64_t stride_row;
} tq_region;

typedef struct tq_kv_view {
    tq_region idx;           /* 16*bits bytes per token; ptr and strides 4-byte aligned */
    tq_region signs;         /* 16 bytes per token (qjl only); 4-byte aligned */
    tq_region norm;          /* fp16 per token; 2-byte aligned */
    tq_region rnorm;         /* fp16 per token (qjl only); 2-byte aligned */
    const float* centroids;  /* device, 2^bits fp32 */
    int32_t bits;            /* 2, 3 or 4 */
    int32_t qjl;             /* 1: score adds the QJL term (K only) */
    int32_t signs_permuted;  /* 1: sign rows in the stride-4 permuted order */
    float centroid_scale;    /* kernels tabulate fp16(centroid * centroid_scale) and divide the
                                scale back out in fp32; a scale in [1,2) chosen so every scaled
                                centroid is nearly exact in fp16 removes the table's rounding.
                                0 means 1. */
    int32_t layout;          /* TQ_TILE_ROWS: the regions above.  TQ_TILE_KEYS / TQ_TILE_VALUES
                                (paged only): idx describes the payload region of the lane-grouped
                                tiles (stride_row = P bytes per token, the sub-tile of row r at
                                (r & ~15) * P), signs is unused, norm / rnorm as above. */
} tq_kv_view;

/*
 * Paged compression into caller-described row-major regions (dst->layout = TQ_TILE_ROWS): the
 * same math and decisions as tq_compress_paged, with token t / head h written at
 *   region R: R.ptr + block * R.stride_block + h * R.stride_head + row * R.stride_row
 * (block = slot / block_size, row = slot % block_size): 16*bits index bytes (idx), 16 sign bytes
 * and an fp16 residual norm (signs, rnorm: dst->qjl only), the fp16 norm (norm).  All regions
 * share stride_block and stride_head; rnorm shares norm's stride_row; pointers and strides
 * 2-byte aligned (4-byte aligned index / sign rows are written with 32-bit stores).  Codebook:
 * dst->centroids and boundaries (2^bits and 2^bits - 1 fp32).  For the reference's
 * array-of-slots cache [num_blocks, 2, block_size, Hkv, slot] (kernels/sparse_v.py:293-304;
 * per token: index bytes, sign bytes, fp16 norm, fp16 residual norm, padding) this is the
 * scatter of integration/vllm_backend.py:223-230 into that cache, in place.
 */
int tq_compress_regions(const void* x, int x_dtype, int64_t x_stride_token, int64_t x_stride_head,
                        int64_t num_tokens, int num_heads, int head_dim,
                        const void* slot_mapping, int slot_dtype, const tq_kv_view* dst,
                        const float* boundaries, int64_t num_blocks, int block_size,
                        int rotate, float wht_scale, tq_stream_t stream);

/*
 * Packed asymmetric split-K decode attention (one query token per sequence), GQA-shared KV.
 * For sequence s, query head h, KV head kh = h / (num_q_heads/num_kv_heads), token t < seq_lens[s]:
 *   score = sm_scale * ( q.(k_cb[idx_t] * norm_t) + corr_scale * rnorm_t * (qp.sign_t) )
 *   out   = sum_t softmax(score)_t * v_cb[vidx_t] * vnorm_t          (fp32 accumulation)
 * with qp = q_proj (or q when q_proj == NULL). Follows attention_unpacked_ref
 * (kernels/packed_attention.py:273-284) with the correct split combine of kernels/attention.py:121-140.
 * Split-K: tokens_per_chunk > 0 (a multiple of 16) cuts every sequence into chunks of that many
 * tokens, one work unit per (sequence, KV head, chunk).  tokens_per_chunk = 0 selects the
 * balanced schedule on the paged fast path: the 32-token tile pairs of all (sequence, KV head)
 * segments, sequences in order and a sequence's KV heads after each other, are dealt to the
 * R = min(P, resident waves) waves of one launch (tq_decode_concurrent_units), wave w taking
 * pairs [floor(w P / R), floor((w + 1) P / R)) of the P in all; its pieces are the chunks.  On
 * the general kernel 0 picks fixed chunks that fit the same workspace.
 * Sparse-V (sparse_threshold > 0, kernels/sparse_v.py:108-149): within each chunk, processed
 * in tiles of 16 tokens with a running max m, token t's V is skipped when max over the GQA
 * group of exp(score - m) <= sparse_threshold; skipped tokens still count in the softmax
 * denominator.
 * q, q_proj: [num_seqs, num_q_heads, 128] (f32/f16/bf16) at the given element strides.
 * out: [num_seqs, num_q_heads, 128] (f32/f16/bf16) at the given element strides.
 * seq_lens: device int32 [num_seqs], or NULL: every sequence holds max_seq_len tokens.
 * block_tables: int32 [num_seqs, block_table_stride]; entries outside [0, num_blocks) are skipped.
 * max_seq_len: an upper bound of seq_lens (sizes the grid); longer sequences are truncated
 *   (the balanced schedule: to max_seq_len tokens).
 * workspace: >= tq_decode_workspace_bytes(num_seqs, num_q_heads, max_seq_len, tokens_per_chunk),
 *   256-byte aligned (split-K partial results; no initial contents needed).  Calls that overlap
 *   in time must not share a workspace.
 * skip_stats: NULL or device uint64[2], incremented by (skipped, total) (token, KV head) pairs.
 * Replaces packed_attention (kernels/packed_attention.py:290-344) and the paged
 * _tq_v12_sparse_v_kernel / _tq_v11_single_kernel (kernels/sparse_v.py:25-261).
 */
int tq_decode(const void* q, int q_dtype, int64_t q_stride_seq, int64_t q_stride_head,
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

/*
 * packed_attention of the reference (kernels/packed_attention.py:290-344) on its own arrays:
 * split-K decode of one query per head over 2-bit keys with QJL signs and 2-bit values, every
 * head a sequence of sk rows.  q, q_proj: [bh, 128] rows of q_dtype (f32/f16/bf16; the scores
 * are not scaled, the caller pre-scales q); k_idx, v_idx: [bh][sk][32] packed 2-bit indices;
 * k_signs: [bh][sk][16] sign bits (signs_permuted: the stride-4 order of
 * permute_signs_for_chunked); k_rnorm, k_norm, v_norm: [bh][sk] fp16; centroids: 4 fp32 (K and
 * V share them) with the table scale of tq_kv_view.centroid_scale (0 means 1); corr_scale the QJL
 * factor as the caller passes it to the reference (the estimator's sqrt(pi/2)/m for m = 128
 * projections, reference/pytorch_reference.py:153-154); tokens_per_chunk as for tq_decode (0: the library's
 * choice; the reference's num_splits corresponds to ceil(sk / num_splits) rounded up to 16);
 * out: [bh, 128] of out_dtype.  The split combine is the exact (m, l, acc) merge.  Returns
 * tq_decode's status codes.  Same kernels and results as tq_decode on contiguous regions with
 * seq_lens = NULL; workspace >= tq_packed_attention_workspace_bytes(bh, sk, tokens_per_chunk),
 * 256-byte aligned.
 */
int tq_packed_attention(const void* q, const void* q_proj, int q_dtype, const uint8_t* k_idx,
                        const uint8_t* k_signs, int signs_permuted, const uint16_t* k_rnorm,
                        const uint16_t* k_norm, const uint8_t* v_idx, const uint16_t* v_norm,
                        const float* centroids, float centroid_scale, float corr_scale, int bh, int sk,
                        int tokens_per_chunk, void* workspace, size_t workspace_bytes, void* out,
                        int out_dtype, tq_stream_t stream);
size_t tq_packed_attention_workspace_bytes(int bh, int sk, int tokens_per_chunk);

/*
 * tq_decode with the query and the output in the original (unrotated) basis: the kernels use
 * q x H (and q_proj = q x H when q_proj == NULL; a given q_proj is used as it is) and write
 * out x H, H = make_wht_matrix(128) (symmetric, H H = I).  Same arguments, workspace and
 * results as tq_decode on pre-rotated queries followed by a rotation of the output.
 * Replaces the rotate_query -> attention -> rotate_output sequence of the reference backend
 * (integration/vllm_backend.py:158-177, TurboQuantFP8State.rotate_query / rotate_output) with
 * the rotations fused into the decode prologue and the output write (the split-K merge when
 * a sequence spans several chunks).
 */
int tq_decode_rotated(const void* q, int q_dtype, int64_t q_stride_seq, int64_t q_stride_head,
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

/*
 * y = x H for rows of 128 elements (H = make_wht_matrix(128)): x and y are
 * [num_seqs, num_heads, 128] at the given element strides (f32/f16/bf16, fp32 arithmetic,
 * one rounding on the store).  y may be x (in place).  Replaces
 * TurboQuantFP8State.rotate_query / rotate_output (integration/vllm_backend.py:158-177) as
 * stand-alone operations, for callers that rotate outside the decode call.
 */
int tq_wht_rows(const void* x, int x_dtype, int64_t x_stride_seq, int64_t x_stride_head,
                int num_seqs, int num_heads, int head_dim,
                void* y, int y_dtype, int64_t y_stride_seq, int64_t y_stride_head,
                tq_stream_t stream);

/*
 * Prefill / extend attention over the packed paged cache: several query tokens per sequence.
 * Sequence s has n_s = cu_seqlens_q[s+1] - cu_seqlens_q[s] query tokens, rows cu_seqlens_q[s] ..
 * of q [T, num_q_heads, 128] (f32/f16/bf16 at the given element strides), and seq_lens[s] cache
 * tokens in block_tables[s] (already holding the new tokens, written by tq_compress_paged).
 * Query i of sequence s attends to cache tokens t with t <= seq_lens[s] - n_s + i when flags
 * has TQ_PREFILL_CAUSAL (the new tokens are the last n_s of the sequence), to all of them
 * otherwise.  Scores, QJL term and softmax as in tq_decode (no Sparse-V, no split-K); out
 * [T, num_q_heads, 128].  TQ_PREFILL_ROTATE: q (and q_proj when NULL) and out in the original
 * basis, as tq_decode_rotated.  Any GQA group; block-table entries outside [0, num_blocks) mask
 * their tokens; num_blocks >= 1.  max_q_len >= every n_s (sizes the grid).
 * Replaces the Sq > 1 tiled kernel _fused_general (kernels/attention.py:146-196, called from
 * FusedAsymmetricAttention.forward, :248), reading the packed cache instead of dequantised
 * K/V arrays, with the causal limit of an extend step (the reference FP4 backend's prefill
 * fallback, integration/tq_fp4_backend.py:558-601).
 */
#define TQ_PREFILL_CAUSAL 1
#define TQ_PREFILL_ROTATE 2
int tq_prefill(const void* q, int q_dtype, int64_t q_stride_token, int64_t q_stride_head,
               const void* q_proj, int64_t qp_stride_token, int64_t qp_stride_head,
               const int32_t* cu_seqlens_q, int num_seqs, int max_q_len,
               int num_q_heads, int num_kv_heads, int head_dim,
               const tq_kv_view* k, const tq_kv_view* v,
               int block_size, int64_t num_blocks,
               const int32_t* block_tables, int64_t block_table_stride, int max_blocks_per_seq,
               const int32_t* seq_lens, float sm_scale, float corr_scale, int flags,
               void* out, int out_dtype, int64_t out_stride_token, int64_t out_stride_head,
               tq_stream_t stream);

size_t tq_decode_workspace_bytes(int num_seqs, int num_q_heads, int max_seq_len, int tokens_per_chunk);

/*
 * tq_decode without a caller workspace and without any device allocation: the split-K partial
 * results go to a fixed array of TQ_NOALLOC_SCRATCH_BYTES inside this library (one copy per
 * GPU, held from the library's load on that GPU until the process ends; its device address is
 * looked up once per device on the first call there).  Same arguments (minus the workspace),
 * checks, kernels and results as tq_decode.  Before any HIP call it returns TQ_ERR_CHUNK for a
 * tokens_per_chunk that is negative or not a multiple of 16, then TQ_ERR_SCRATCH_LIMIT when
 * tq_decode_workspace_bytes(num_seqs, num_q_heads, max_seq_len, tokens_per_chunk) exceeds
 * TQ_NOALLOC_SCRATCH_BYTES, for fixed chunks (choose a larger tokens_per_chunk) and for the
 * balanced schedule (tokens_per_chunk = 0: about 17 MB plus 520 bytes per (sequence, query
 * head), so beyond about 96k such pairs; choose fixed chunks).  Calls that overlap in time on
 * one GPU share its array and race; nothing is carried between calls.
 * No counterpart in the reference: for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid allocation).
 */
#define TQ_NOALLOC_SCRATCH_BYTES (64u << 20)
int tq_decode_noalloc(const void* q, int q_dtype, int64_t q_stride_seq, int64_t q_stride_head,
                      const void* q_proj, int64_t qp_stride_seq, int64_t qp_stride_head,
                      int num_seqs, int num_q_heads, int num_kv_heads, int head_dim,
                      const tq_kv_view* k, const tq_kv_view* v,
                      int block_size, int64_t num_blocks,
                      const int32_t* block_tables, int64_t block_table_stride, int max_blocks_per_seq,
                      const int32_t* seq_lens, int max_seq_len,
                      float sm_scale, float corr_scale, float sparse_threshold,
                      int tokens_per_chunk,
                      void* out, int out_dtype, int64_t out_stride_seq, int64_t out_stride_head,
                      unsigned long long* skip_stats,
                      tq_stream_t stream);

/* Work units (one per sequence, KV head and chunk of tokens_per_chunk tokens) that tq_decode
 * can run at once on the current device for this configuration: resident waves per compute
 * unit of the kernel variant tq_decode would pick, times the compute units.  Callers size
 * tokens_per_chunk from it so that the grid fills whole rounds; on the paged fast path it is
 * also the wave count R of the balanced schedule (tokens_per_chunk = 0).  No counterpart in the
 * reference (its Triton launcher sizes the split from a fixed program target,
 * kernels/attention.py:202-211).
 * norm_row_bytes: row stride of the K / V norm streams (2 for the paged tile layout). */
int tq_decode_concurrent_units(int k_bits, int k_qjl, int v_bits, int num_q_heads, int num_kv_heads,
                               int norm_row_bytes, int share_codebook, int* units);

/* Waves per workgroup of the kernel tq_decode picks for this configuration: consecutive work
 * units (fixed chunks: (sequence, chunk, KV head) order) share a workgroup, and the dispatcher
 * deals workgroups to the XCDs and their shader engines in turn.  Callers that know the
 * sequence lengths use it to keep every shader engine within one round of resident workgroups
 * when they choose tokens_per_chunk.  No counterpart in the reference (its Triton launcher has
 * fixed programs, kernels/attention.py:202-211).  Same arguments and checks as
 * tq_decode_concurrent_units. */
int tq_decode_workgroup_waves(int k_bits, int k_qjl, int v_bits, int num_q_heads, int num_kv_heads,
                              int norm_row_bytes, int share_codebook, int* waves);

/* ---- packing helpers ----------------------------------------------------------- */

/* Reorder sign rows [n_rows, 16] natural -> stride-4 permuted (out bit 32c+k = in bit 4k+c).
 * Replaces permute_signs_for_chunked (kernels/packed_compress.py:180-216). */
int tq_permute_signs(const uint8_t* in, uint8_t* out, int64_t n_rows, int head_dim, tq_stream_t stream);

/* Unpack rows of b-bit fields [n_rows, 16*b bytes] -> int8 [n_rows, 128] (b in 1..4).
 * Replaces unpack_2bit / unpack_1bit (kernels/packed_compress.py:145-154). */
int tq_unpack_bits(const uint8_t* in, int8_t* out, int64_t n_rows, int head_dim, int bits, tq_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* TURBOQUANT_HIP_H */
