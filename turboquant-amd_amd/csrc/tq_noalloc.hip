// tq_decode_noalloc: tq_decode with the split-K workspace in a fixed device array of this
// library instead of a caller buffer, for callers that cannot allocate device memory (code
// under HIP graph capture, tight serving loops, harnesses that forbid allocation).
//
// The array `scratch` lives in this file.  Its name in host code is a host-side stand-in, not
// a device address: the address is taken once per device with hipGetSymbolAddress (with that
// device current) on the first call there, kept per device, and only that address is passed
// to the kernels.  Each GPU holds its own copy of the array until the process ends.  Every call
// on one GPU uses that GPU's copy: calls that overlap in time on one GPU race.  Nothing carried
// from an earlier call is read (every partial result slot is written before the merge reads
// it), so the array is never cleared.
#include <mutex>

#include "tq_common.h"
#include "tq_decode_internal.h"

namespace {

constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[TQ_NOALLOC_SCRATCH_BYTES];

std::once_flag g_once[kMaxDevices];
void* g_ptr[kMaxDevices];
hipError_t g_err[kMaxDevices];

// The device address of this device's copy of `scratch` (looked up once per device).
int scratch_address(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= kMaxDevices) return TQ_ERR_INVALID_ARGUMENT;
    std::call_once(g_once[dev], [dev] {
        void* p = nullptr;
        g_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        g_ptr[dev] = g_err[dev] == hipSuccess ? p : nullptr;
    });
    if (g_err[dev] != hipSuccess) return (int)g_err[dev];
    if (!g_ptr[dev]) return TQ_ERR_INVALID_ARGUMENT;
    *out = g_ptr[dev];
    return TQ_OK;
}

}  // namespace

extern "C" int tq_decode_noalloc(const void* q, int q_dtype, int64_t q_stride_seq, int64_t q_stride_head,
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
                                 tq_stream_t stream) {
    // Checks first, before any HIP call: an invalid chunk, then a request beyond the fixed
    // array, for fixed chunks and for the balanced schedule (tokens_per_chunk = 0, whose
    // workspace grows with num_seqs * num_q_heads; tq_decode_impl runs a general-kernel fallback
    // of that schedule inside the same workspace size).
    if (tokens_per_chunk < 0 || tokens_per_chunk % 16) return TQ_ERR_CHUNK;
    if (num_seqs > 0 && num_q_heads > 0 &&
        tq_decode_workspace_bytes(num_seqs, num_q_heads, max_seq_len, tokens_per_chunk) > (size_t)TQ_NOALLOC_SCRATCH_BYTES)
        return TQ_ERR_SCRATCH_LIMIT;
    void* ws = nullptr;
    if (num_seqs > 0) {
        const int rc = scratch_address(&ws);
        if (rc) return rc;
    }
    return tq_decode_impl(0, q, q_dtype, q_stride_seq, q_stride_head, q_proj, qp_stride_seq, qp_stride_head, num_seqs,
                          num_q_heads, num_kv_heads, head_dim, k, v, block_size, num_blocks, block_tables,
                          block_table_stride, max_blocks_per_seq, seq_lens, max_seq_len, sm_scale, corr_scale,
                          sparse_threshold, tokens_per_chunk, ws, (size_t)TQ_NOALLOC_SCRATCH_BYTES, out, out_dtype,
                          out_stride_seq, out_stride_head, skip_stats, stream);
}
