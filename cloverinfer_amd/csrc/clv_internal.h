// clv_internal.h - kernel parameter blocks and launcher declarations shared
// by the C-ABI layer (clover_attn_abi.hip) and the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace clv {

// Decode parameters after validation. Strides are in elements.
struct DecodeParams {
  void *out;
  const void *q;
  const void *k_cache;
  const void *v_cache;
  const int32_t *block_tables;
  const int32_t *context_lens;
  int64_t q_stride_seq, q_stride_head;
  int64_t out_stride_seq, out_stride_head;
  int64_t kv_stride_block, kv_stride_token, kv_stride_head;
  int32_t num_seqs, num_heads, num_kv_heads, head_dim;
  int32_t group;          // num_heads / num_kv_heads
  int32_t n_gchunks;      // ceil(group / 16): query-head chunks per kv head
  int32_t block_shift;    // log2(block_size)
  int32_t max_blocks_per_seq, max_context_len, num_blocks;
  float scale_log2;       // scale * log2(e): scores live in the log2 domain
  // Split-K: partition_size > 0 writes partials to the workspace.
  int32_t partition_size; // tokens per workgroup, multiple of 32; 0 = whole context
  int32_t max_parts;      // partitions per sequence held by the workspace
  float *ws_o;            // [num_seqs, num_heads, max_parts, head_dim] normalised contexts
  float *ws_m;            // [num_seqs, num_heads, max_parts] row max (natural-log domain)
  float *ws_l;            // [num_seqs, num_heads, max_parts] row sum
  // Balanced (stream) mode: groups of head_group waves (one workgroup's
  // waves, one kv head each) split the flattened (sequence, kv-head group,
  // query-head chunk, 16-token step) space evenly; the workspace holds one
  // partial per (segment, group, kv head of the group), 16 rows each at row
  // ((segment + group) * head_group + wave in group) * 16, in
  // ws_o/ws_m/ws_l, plus the segment prefix sums written by workgroup 0.
  int32_t num_waves;
  int32_t head_group;     // kv heads read together (1, 2 or 4; divides num_kv_heads)
  int32_t stream_depth;   // steps of loads each wave keeps in flight
  int32_t stream_run_cost;  // phantom steps charged for each segment start (see decode_stream.hip)
  int32_t num_segments;   // num_seqs * (num_kv_heads / head_group) * n_gchunks
  int32_t *seg_prefix;    // [num_segments + 1] exclusive prefix of steps per segment
  // Split by dispatch slot (see StreamSplit in decode_stream.hip): with
  // slot_count > 1, groups [k * slot_groups, (k+1) * slot_groups) form piece
  // k (the last piece takes the groups left), and each group of piece k is
  // weighted slot_q8[k] / 256; slot_count 0 or 1 is the even split.
  int32_t slot_count;
  int32_t slot_groups;
  int32_t slot_q8[4];
  // Fused append (balanced mode): when append_new is set, sequence s's new
  // key/value rows key_new/value_new[s] ([num_kv_heads, head_dim], strides in
  // elements) are written at its context position context_lens[s] - 1 by the
  // wave that computes that position, before it loads it.
  int32_t append_new;
  const void *key_new;
  const void *value_new;
  int64_t new_stride_seq, new_stride_head;
  // Merge with the new token (stream_reduce_append): sequence s's new rows
  // are written at slot_mapping[s] (block * block_size + offset; negative:
  // not written), and attended from key_new/value_new themselves.
  const int64_t *slot_mapping;
  // fp8 pools (balanced mode): k_cache/v_cache hold OCP e4m3 bytes, strides
  // in bytes, with one scale per kv head; q and out are f16/bf16.
  int32_t kv_fp8;
  const float *k_scales;  // [num_kv_heads]
  const float *v_scales;  // [num_kv_heads]
};

// Largest segment count the balanced mode keeps in LDS.
constexpr int kStreamMaxSegments = 4096;

struct CacheParams {
  const void *key;
  const void *value;
  void *k_cache;
  void *v_cache;
  const int64_t *slot_mapping;
  int64_t key_stride_token, key_stride_head;
  int64_t value_stride_token, value_stride_head;
  int64_t kv_stride_block, kv_stride_token, kv_stride_head;
  int32_t num_tokens, num_kv_heads, head_dim, block_shift, num_blocks;
  int64_t num_slots;      // num_blocks * block_size
  int32_t elem_bytes;
};

struct PrefillParams {
  void *out;
  const void *q;
  const void *k_cache;
  const void *v_cache;
  const int32_t *block_tables;
  const int32_t *context_lens;
  const int32_t *query_start_loc;
  int64_t q_stride_token, q_stride_head;
  int64_t out_stride_token, out_stride_head;
  int64_t kv_stride_block, kv_stride_token, kv_stride_head;
  int32_t num_seqs, num_tokens, num_heads, num_kv_heads, head_dim;
  int32_t group, block_shift, max_blocks_per_seq, max_query_len, num_blocks;
  float scale_log2;
  // Compute units per XCD (the device's count / 8), for the prefill's
  // dispatch order; 0 keeps the natural order.
  int32_t cus_per_xcd;
};

enum class DType : int { F32 = 0, F16 = 1, BF16 = 2 };

// Launchers return hipSuccess or the launch error. Shapes are pre-validated.
hipError_t launch_reshape_and_cache(const CacheParams &p, hipStream_t stream);
hipError_t launch_decode_mfma(const DecodeParams &p, DType dt, hipStream_t stream);
// Single-pass grid decode that first writes key_new/value_new[s] at position
// context_lens[s] - 1 (partition_size 0, one query-head chunk per kv head).
hipError_t launch_decode_mfma_append(const DecodeParams &p, DType dt, hipStream_t stream);
hipError_t launch_decode_valu(const DecodeParams &p, DType dt, hipStream_t stream);
hipError_t launch_splitk_reduce(const DecodeParams &p, DType dt, hipStream_t stream);
hipError_t launch_decode_stream(const DecodeParams &p, DType dt, hipStream_t stream);
hipError_t launch_stream_reduce(const DecodeParams &p, DType dt, hipStream_t stream);
// stream_reduce over partials of context_lens[s] tokens plus sequence s's new
// token (key_new/value_new[s]), which it also writes at slot_mapping[s].
hipError_t launch_stream_reduce_append(const DecodeParams &p, DType dt, hipStream_t stream);
hipError_t launch_prefill_mfma(const PrefillParams &p, DType dt, hipStream_t stream);
// Writes key_new/value_new[s] at position context_lens[s] - 1 of every
// sequence (slot from its block table), for the decode shapes whose stream
// kernel does not append itself.
hipError_t launch_append_by_table(const DecodeParams &p, int elem_bytes, hipStream_t stream);
// KV append into fp8 (OCP e4m3) pools: cache = e4m3(clamp(x / scale[h], +-448)),
// rounded to nearest even; key/value in CacheParams' elem_bytes (2 or 4).
hipError_t launch_reshape_and_cache_fp8(const CacheParams &p, int src_dtype, const float *k_scales,
                                        const float *v_scales, hipStream_t stream);
hipError_t launch_prefill_valu(const PrefillParams &p, DType dt, hipStream_t stream);

// Whether the MFMA decode kernel covers this shape/dtype.
bool decode_mfma_supported(DType dt, int head_dim, int block_size);
bool decode_stream_supported(DType dt, int head_dim, int block_size, int64_t num_segments);
// Whether the stream kernel writes the appended token itself (fused append)
// for this shape; otherwise launch_append_by_table runs first.
bool stream_appends_in_kernel(DType dt, int head_dim, int block_size, int group);
bool prefill_mfma_supported(DType dt, int head_dim, int block_size);

}  // namespace clv
