/*
 * clover_attn.h - C ABI of the MI355X (gfx950) paged-attention hot path.
 *
 * Plain C: raw device pointers, element strides and sizes; no torch or HIP
 * types in any signature. Every entry point is stream-ordered (it enqueues
 * work on `stream` and returns), reentrant, and keeps no mutable global
 * state. The caller owns every device buffer, including the split-K
 * workspace, which it sizes with clv_splitk_workspace_bytes().
 *
 * Cache layout (shared by the key and the value pool):
 *     [num_blocks, block_size, num_kv_heads, head_dim]
 * addressed as  base + block*kv_stride_block + offset*kv_stride_token
 *                    + kv_head*kv_stride_head + d     (head_dim contiguous).
 * A token at logical position t of sequence s lives in physical block
 * block_tables[s*max_blocks_per_seq + t/block_size], offset t%block_size.
 *
 * GQA: query head h reads kv head h / (num_heads/num_kv_heads), the same
 * grouping as transformers' repeat_kv.
 *
 * Status codes are returned, never thrown.
 */
#ifndef CLOVER_ATTN_H
#define CLOVER_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CLV_ABI_VERSION 1

/* A hipStream_t; NULL selects the null stream. */
typedef void *clv_stream_t;

enum clv_dtype { CLV_F32 = 0, CLV_F16 = 1, CLV_BF16 = 2 };

enum clv_status {
  CLV_OK = 0,
  CLV_EINVAL = 1,       /* bad shape, stride, pointer or dtype */
  CLV_EUNSUPPORTED = 2, /* valid but not implemented (e.g. head_dim) */
  CLV_ELAUNCH = 3,      /* the HIP runtime rejected a launch */
  CLV_EWORKSPACE = 4,   /* split-K workspace missing or too small */
  CLV_ESCRATCH = 5      /* too large for the no-allocation entry point's scratch */
};

/*
 * Paged decode: one query row per sequence attends to that sequence's first
 * context_lens[s] cached tokens.
 *   out[s, h, :] = softmax_t(scale * q[s,h,:].K[t,kvh,:]) . V[t,kvh,:]
 * Math is fp32 whatever the storage dtype; out is written in `dtype`.
 * A sequence with context length 0 gets an all-zero row.
 * Block-table entries outside [0, num_blocks) inside the context are
 * treated as masked tokens (never dereferenced).
 * context_lens[s] must not exceed max_context_len (larger values are
 * clamped to it and to max_blocks_per_seq*block_size).
 */
typedef struct clv_decode_args {
  void *out;                   /* [num_seqs, num_heads, head_dim]           */
  const void *q;               /* [num_seqs, num_heads, head_dim]           */
  const void *k_cache;         /* [num_blocks, block_size, num_kv_heads, D] */
  const void *v_cache;         /* same layout and strides as k_cache        */
  const int32_t *block_tables; /* [num_seqs, max_blocks_per_seq], -1 pad    */
  const int32_t *context_lens; /* [num_seqs]                                */
  int64_t q_stride_seq, q_stride_head;       /* elements */
  int64_t out_stride_seq, out_stride_head;   /* elements */
  int64_t kv_stride_block, kv_stride_token, kv_stride_head; /* elements */
  int32_t num_seqs, num_heads, num_kv_heads, head_dim;
  int32_t block_size, max_blocks_per_seq, max_context_len, num_blocks;
  int32_t dtype; /* enum clv_dtype, shared by q, out and both caches */
  float scale;   /* softmax scale applied to q.k (1/sqrt(D) in the reference op) */
} clv_decode_args;

/*
 * KV append ("reshape_and_cache"): copies token i's key/value rows into
 * cache slot slot_mapping[i] = block*block_size + offset.
 * A negative slot, or one >= num_blocks*block_size, skips the token.
 */
typedef struct clv_cache_args {
  const void *key;             /* [num_tokens, num_kv_heads, head_dim] */
  const void *value;           /* [num_tokens, num_kv_heads, head_dim] */
  void *k_cache;               /* [num_blocks, block_size, num_kv_heads, D] */
  void *v_cache;
  const int64_t *slot_mapping; /* [num_tokens] */
  int64_t key_stride_token, key_stride_head;     /* elements */
  int64_t value_stride_token, value_stride_head; /* elements */
  int64_t kv_stride_block, kv_stride_token, kv_stride_head; /* elements */
  int32_t num_tokens, num_kv_heads, head_dim, block_size, num_blocks;
  int32_t dtype;
} clv_cache_args;

/*
 * Chunked prefill over paged KV. Sequence s owns query rows
 * [query_start_loc[s], query_start_loc[s+1]) of q/out; its n_s new tokens
 * are the LAST n_s of its context_lens[s] cached tokens (append them with
 * clv_reshape_and_cache first). Query row i of sequence s (0 <= i < n_s)
 * attends to cached positions p <= context_lens[s] - n_s + i (causal inside
 * the chunk, full view of everything cached before it).
 * max_query_len sizes the launch and must be >= every n_s (the host cannot
 * see query_start_loc, a device array): a row i >= max_query_len of its
 * chunk comes out as NaN (every kernel form).
 */
typedef struct clv_prefill_args {
  void *out;                      /* [num_tokens, num_heads, head_dim] */
  const void *q;                  /* [num_tokens, num_heads, head_dim] */
  const void *k_cache;
  const void *v_cache;
  const int32_t *block_tables;    /* [num_seqs, max_blocks_per_seq] */
  const int32_t *context_lens;    /* [num_seqs], including the new tokens */
  const int32_t *query_start_loc; /* [num_seqs + 1], non-decreasing */
  int64_t q_stride_token, q_stride_head;     /* elements */
  int64_t out_stride_token, out_stride_head; /* elements */
  int64_t kv_stride_block, kv_stride_token, kv_stride_head;
  int32_t num_seqs, num_tokens, num_heads, num_kv_heads, head_dim;
  int32_t block_size, max_blocks_per_seq, max_query_len, num_blocks;
  int32_t dtype;
  float scale;
} clv_prefill_args;

/* ABI version of the loaded library (CLV_ABI_VERSION at build time). */
int clv_abi_version(void);

/* Static text for a status code. */
const char *clv_status_string(int status);

/*
 * Replaces the per-token Python index-put of KVCacheManager.write_new_kv
 * (src/core/memory_manager.py:123-132) and the per-block copies of
 * load_initial_kv (src/core/memory_manager.py:74-93): one launch for any
 * number of tokens.
 */
int clv_reshape_and_cache(const clv_cache_args *args, clv_stream_t stream);

/*
 * Replaces clover_kernels.paged_attention (src/kernels/csrc/manager.cpp:19-42,
 * launcher src/kernels/csrc/attention.cu:118-149) with GQA, bf16 and an
 * explicit scale. Single pass: one workgroup per (sequence, kv head) walks
 * the whole context. Needs no workspace.
 */
int clv_paged_decode(const clv_decode_args *args, clv_stream_t stream);

/*
 * Bytes of workspace clv_paged_decode_splitk needs: per (sequence, query
 * head, partition) one fp32 context row plus its row max and row sum.
 */
size_t clv_splitk_workspace_bytes(int32_t num_seqs, int32_t num_heads,
                                  int32_t head_dim, int32_t max_context_len,
                                  int32_t partition_size);

/*
 * Split-K decode: the context is cut into partitions of partition_size
 * tokens (a positive multiple of 32); each (sequence, kv head, partition)
 * produces a normalised partial context with its row max and row sum, and a
 * second kernel merges them with the log-sum-exp rule of the reference's
 * partial-softmax merge (src/core/resident_kv_store.py:2497-2509).
 * Equal to clv_paged_decode_partials followed by clv_splitk_reduce (when
 * max_context_len <= partition_size it runs the single pass instead).
 * No counterpart kernel exists in the reference.
 */
int clv_paged_decode_splitk(const clv_decode_args *args, int32_t partition_size,
                            void *workspace, size_t workspace_bytes,
                            clv_stream_t stream);

/*
 * First half of split-K: writes, for every (sequence s, query head h,
 * partition p < ceil(context_lens[s]/partition_size)), the normalised
 * partial context, its row max (natural-log domain, of scale*q.k) and row
 * sum into the workspace. `out` is not touched. Replaces the per-segment
 * partial attention of src/core/resident_kv_store.py:715-783.
 */
int clv_paged_decode_partials(const clv_decode_args *args, int32_t partition_size,
                              void *workspace, size_t workspace_bytes,
                              clv_stream_t stream);

/*
 * Second half of split-K: merges the partials clv_paged_decode_partials left
 * in the workspace (same args, partition_size and workspace) into `out`.
 * Restates src/core/resident_kv_store.py:2497-2509 over all partitions:
 *   M = max m_i, w_i = l_i e^(m_i - M), out = sum c_i w_i / max(sum w_i, 1e-12).
 */
int clv_splitk_reduce(const clv_decode_args *args, int32_t partition_size,
                      const void *workspace, size_t workspace_bytes,
                      clv_stream_t stream);

/*
 * Balanced decode for ragged batches (fp32/fp16/bf16, head_dim 64 or 128,
 * num_seqs * num_kv_heads * ceil(group/16) <= 4096): num_waves waves split
 * the batch's flattened 16-token steps evenly, crossing sequence borders
 * (in groups of up to four waves of one workgroup that take the same steps of
 * adjacent kv heads; at exactly two or three workgroups of four waves per
 * compute unit the earlier-dispatched workgroups take 10-25 % more steps
 * each, as the hardware runs their waves ahead of the later ones on the same
 * SIMD); each writes one partial per (sequence, kv head) it
 * touches and a second kernel merges them with the same log-sum-exp rule as
 * the split-K reduce.
 * Same result as clv_paged_decode. num_waves <= 0 picks the device default
 * (clv_default_num_waves()). No counterpart kernel exists in the reference.
 */
int clv_paged_decode_balanced(const clv_decode_args *args, int32_t num_waves,
                              void *workspace, size_t workspace_bytes,
                              clv_stream_t stream);

/*
 * The two halves of clv_paged_decode_balanced (same arguments): the stream
 * kernel writing partials and the merge into `out`.
 */
int clv_balanced_partials(const clv_decode_args *args, int32_t num_waves,
                          void *workspace, size_t workspace_bytes,
                          clv_stream_t stream);
int clv_balanced_reduce(const clv_decode_args *args, int32_t num_waves,
                        const void *workspace, size_t workspace_bytes,
                        clv_stream_t stream);

/*
 * clv_paged_decode_balanced without a workspace argument and without any
 * allocation: the workspace is a fixed device array of
 * CLV_NOALLOC_SCRATCH_BYTES inside the library (one per GPU, held for the
 * life of the process), for callers that cannot call hipMalloc (code under
 * HIP graph capture, tight serving loops). No counterpart in the reference.
 * Same arguments, kernels and result as clv_paged_decode_balanced with
 * num_waves waves (<= 0: clv_default_num_waves()). Returns CLV_ESCRATCH,
 * launching nothing, when clv_balanced_workspace_bytes() of the call exceeds
 * the scratch (at head_dim 128 and 1024 waves: up to 3007 (sequence, kv head,
 * 16-query-head chunk) segments). Uses the scratch of the current device;
 * `stream` must belong to it. Every call on a GPU shares that GPU's scratch:
 * calls that overlap on one GPU (on different streams, or from different
 * threads without ordering) race and must be serialised by the caller.
 */
#define CLV_NOALLOC_SCRATCH_BYTES (32u << 20)
int clv_paged_decode_balanced_noalloc(const clv_decode_args *args, int32_t num_waves,
                                      clv_stream_t stream);

/*
 * One decode step of the reference's append-then-attend protocol
 * (CpuAttentionBackend.decode_layer, src/core/attention_backend.py:105-118;
 * KVCacheManager.write_new_kv then .attention,
 * src/core/memory_manager.py:123-190) in one call: sequence s's new key and
 * value rows key_new[s], value_new[s] ([num_kv_heads, head_dim], strides in
 * elements) are written at its context position context_lens[s] - 1 (the
 * slot its block table names), and its query rows attend to all
 * context_lens[s] tokens, the new one included. Same result as
 * clv_reshape_and_cache with those slots followed by
 * clv_paged_decode_balanced, and the same shapes and workspace as the latter
 * (CLV_EUNSUPPORTED otherwise). For 16-bit pools with head_dim 128,
 * block_size >= 16 and at most 16 query heads per kv head, the decode kernel
 * writes the rows itself (no separate append launch). With num_waves <= 0,
 * max_context_len <= 512 and at most 16 query heads per kv head (fp32, fp16
 * or bf16 pools, head_dim 64 or 128, block_size >= 4), the call is instead
 * one single-pass launch that appends and attends (as clv_paged_decode: no
 * merge; the workspace is not used). A sequence appends nothing when
 * context_lens[s] is outside [1, min(max_context_len,
 * max_blocks_per_seq*block_size)] or the slot's block-table entry is outside
 * [0, num_blocks). k_cache and v_cache are written. No counterpart kernel
 * exists in the reference.
 */
int clv_paged_decode_append(const clv_decode_args *args, const void *key_new,
                            const void *value_new, int64_t new_stride_seq,
                            int64_t new_stride_head, int32_t num_waves,
                            void *workspace, size_t workspace_bytes,
                            clv_stream_t stream);

/*
 * The same decode step in two launches, for a caller that can start the
 * decode over the cached context before the new rows are at hand (the node
 * stages each call's payloads on the host while the GPU works):
 * clv_balanced_partials(args) over context_lens[s] cached tokens, then this
 * merge, which attends each sequence's query rows to those tokens plus its
 * new token (key_new[s], value_new[s]: [num_kv_heads, head_dim], strides in
 * elements), and writes the new rows at slot_mapping[s] (block * block_size
 * + offset; no write where negative or at or past num_blocks * block_size)
 * for the steps after this one. Same args (context_lens = the lengths before
 * the new token), num_waves and workspace as the partials call; the new
 * token's score is formed in fp32 from the 16-bit (or fp32) values, so the
 * result equals clv_paged_decode_append's over context_lens[s] + 1 tokens to
 * fp32 rounding. The slots are the caller's, as in clv_reshape_and_cache:
 * the block tables need not hold the new token's block yet. fp32, fp16 and
 * bf16 pools, the balanced decode's shapes (CLV_EUNSUPPORTED otherwise).
 * References: CpuAttentionBackend.decode_layer, src/core/attention_backend.py:105-118
 * (append, then attend); the merge rule of src/core/resident_kv_store.py:2497-2509.
 */
int clv_balanced_reduce_append(const clv_decode_args *args, const void *key_new,
                               const void *value_new, int64_t new_stride_seq,
                               int64_t new_stride_head, const int64_t *slot_mapping,
                               int32_t num_waves, const void *workspace,
                               size_t workspace_bytes, clv_stream_t stream);

/*
 * fp8 KV pools (OCP e4m3, one byte per element, a float32 scale per kv head;
 * the reference keeps its resident KV in fp32 or fp16, the pool dtype knob of
 * src/core/config.py:38, and has no fp8 form). A stored byte b stands for
 * e4m3(b) * scale[kv head].
 *
 * Append: like clv_reshape_and_cache, with the pools in fp8 (kv strides in
 * bytes, multiples of 8, 8-byte aligned pools, head_dim a multiple of 8);
 * `dtype` is the dtype of key/value. Each value is stored as
 *     e4m3(clamp(x / scale[h], -448, 448)), rounded to nearest even
 * (NaN stays NaN).
 */
int clv_reshape_and_cache_fp8(const clv_cache_args *args, const float *k_scales,
                              const float *v_scales, clv_stream_t stream);

/*
 * Balanced decode over fp8 pools: the result of clv_paged_decode_balanced
 * with K = e4m3(k) * k_scales[h] and V = e4m3(v) * v_scales[h] (exact
 * conversion; the key scale is folded into the softmax scale, the value scale
 * into each partial context). `dtype` is that of q and out (f16 or bf16);
 * kv strides are in bytes (multiples of 16); head_dim 128, block_size >= 16.
 * Workspace as clv_paged_decode_balanced, sized for the wave count used:
 * num_waves <= 0 picks clv_default_num_waves_fp8(). No counterpart in the
 * reference.
 */
int clv_paged_decode_fp8(const clv_decode_args *args, const float *k_scales,
                         const float *v_scales, int32_t num_waves, void *workspace,
                         size_t workspace_bytes, clv_stream_t stream);

/*
 * First half of clv_paged_decode_fp8: the per-segment partials (normalised
 * context, row maximum, row sum) into the workspace, for clv_balanced_reduce
 * with the same arguments and the same wave count to merge. num_waves must
 * be positive (CLV_EINVAL otherwise): the partial layout depends on it, and
 * the defaults of this call and of clv_balanced_reduce differ
 * (clv_default_num_waves_fp8() against clv_default_num_waves()). For a caller that times the
 * two kernels apart, or that merges partials from several GPUs of a
 * context-parallel decode. No counterpart in the reference.
 */
int clv_paged_decode_fp8_partials(const clv_decode_args *args, const float *k_scales,
                                  const float *v_scales, int32_t num_waves, void *workspace,
                                  size_t workspace_bytes, clv_stream_t stream);

/* Workspace bytes of clv_paged_decode_balanced (num_waves <= 0: default). */
size_t clv_balanced_workspace_bytes(int32_t num_seqs, int32_t num_heads,
                                    int32_t num_kv_heads, int32_t head_dim,
                                    int32_t num_waves);

/* Default wave count of the balanced decode on the current device. */
int32_t clv_default_num_waves(void);

/* Default wave count of clv_paged_decode_fp8 (two per SIMD). */
int32_t clv_default_num_waves_fp8(void);

/*
 * Chunked prefill over paged KV (MFMA for fp16/bf16). No counterpart in the
 * reference; defined as equal, row by row, to successive append-then-attend
 * decode steps of CpuAttentionBackend.decode_layer
 * (src/core/attention_backend.py:82-123).
 */
int clv_chunked_prefill(const clv_prefill_args *args, clv_stream_t stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* CLOVER_ATTN_H */
