// cache_ops.hip - KV append ("reshape_and_cache") for the paged pools.
//
// Token i's key/value rows [num_kv_heads, head_dim] go to cache slot
// slot_mapping[i] = block*block_size + offset, i.e. to
//   cache[block, offset, h, :]   for every kv head h.
// This is the device-side form of KVCacheManager.write_new_kv's index-put
// (src/core/memory_manager.py:131-132) and of load_initial_kv's per-block
// copies (src/core/memory_manager.py:88-91), for any number of tokens in one
// launch. It is a pure copy: HBM-bound, 2 reads + 2 writes of each row.
#include "clv_device.h"

namespace clv {
namespace {

constexpr int kThreads = 256;

// One thread moves one 16-byte chunk of one (token, head) row of both the key
// and the value. Rows are head_dim*elem_bytes long, a multiple of 16 bytes.
__global__ void __launch_bounds__(kThreads)
reshape_and_cache_vec16(const CacheParams p, int chunks_per_row) {
  // The launcher guarantees num_tokens*num_kv_heads*chunks_per_row < 2^31.
  const uint32_t gid = blockIdx.x * kThreads + threadIdx.x;
  const uint32_t rows = (uint32_t)p.num_tokens * (uint32_t)p.num_kv_heads;
  const uint32_t row = gid / (uint32_t)chunks_per_row;
  if (row >= rows) return;
  const int chunk = (int)(gid - row * (uint32_t)chunks_per_row);
  const int token = (int)(row / (uint32_t)p.num_kv_heads);
  const int head = (int)(row - (uint32_t)token * (uint32_t)p.num_kv_heads);
  const int64_t slot = p.slot_mapping[token];
  if (slot < 0 || slot >= p.num_slots) return;
  const int64_t blk = slot >> p.block_shift;
  const int64_t off = slot & ((1 << p.block_shift) - 1);
  const int64_t eb = p.elem_bytes;
  const int64_t dst =
      (blk * p.kv_stride_block + off * p.kv_stride_token + head * p.kv_stride_head) * eb +
      chunk * 16;
  const int64_t src_k = ((int64_t)token * p.key_stride_token + head * p.key_stride_head) * eb +
                        chunk * 16;
  const int64_t src_v =
      ((int64_t)token * p.value_stride_token + head * p.value_stride_head) * eb + chunk * 16;
  const u32x4 kv = load_vec<u32x4>((const char *)p.key + src_k);
  const u32x4 vv = load_vec<u32x4>((const char *)p.value + src_v);
  store_vec<u32x4>((char *)p.k_cache + dst, kv);
  store_vec<u32x4>((char *)p.v_cache + dst, vv);
}

// Element-wise fallback for rows or strides that are not 16-byte aligned.
template <typename E>
__global__ void __launch_bounds__(kThreads) reshape_and_cache_elem(const CacheParams p) {
  // The launcher guarantees num_tokens*num_kv_heads*head_dim < 2^31.
  const uint32_t gid = blockIdx.x * kThreads + threadIdx.x;
  const uint32_t total = (uint32_t)p.num_tokens * (uint32_t)p.num_kv_heads * (uint32_t)p.head_dim;
  if (gid >= total) return;
  const int d = (int)(gid % (uint32_t)p.head_dim);
  const uint32_t row = gid / (uint32_t)p.head_dim;
  const int token = (int)(row / (uint32_t)p.num_kv_heads);
  const int head = (int)(row - (uint32_t)token * (uint32_t)p.num_kv_heads);
  const int64_t slot = p.slot_mapping[token];
  if (slot < 0 || slot >= p.num_slots) return;
  const int64_t blk = slot >> p.block_shift;
  const int64_t off = slot & ((1 << p.block_shift) - 1);
  const int64_t dst = blk * p.kv_stride_block + off * p.kv_stride_token + head * p.kv_stride_head + d;
  const E *k = (const E *)p.key;
  const E *v = (const E *)p.value;
  ((E *)p.k_cache)[dst] = k[(int64_t)token * p.key_stride_token + head * p.key_stride_head + d];
  ((E *)p.v_cache)[dst] = v[(int64_t)token * p.value_stride_token + head * p.value_stride_head + d];
}

bool aligned16(const void *ptr) { return ((uintptr_t)ptr & 15u) == 0; }

// Append of one decode step, the slot taken from the block table: sequence
// s's new rows key_new/value_new[s] go to its context position
// context_lens[s] - 1 when 1 <= context_lens[s] <= min(max_context_len,
// max_blocks_per_seq * block_size) and that position's block-table entry is
// in [0, num_blocks). One thread per 16-byte chunk of one (sequence, head)
// row of both the key and the value.
__global__ void __launch_bounds__(kThreads)
append_by_table_vec16(const DecodeParams p, int chunks_per_row, int elem_bytes) {
  // The launcher guarantees num_seqs*num_kv_heads*chunks_per_row < 2^31.
  const uint32_t gid = blockIdx.x * kThreads + threadIdx.x;
  const uint32_t rows = (uint32_t)p.num_seqs * (uint32_t)p.num_kv_heads;
  const uint32_t row = gid / (uint32_t)chunks_per_row;
  if (row >= rows) return;
  const int chunk = (int)(gid - row * (uint32_t)chunks_per_row);
  const int s = (int)(row / (uint32_t)p.num_kv_heads);
  const int head = (int)(row - (uint32_t)s * (uint32_t)p.num_kv_heads);
  const int len = p.context_lens[s];
  const int cap = min(p.max_context_len, p.max_blocks_per_seq << p.block_shift);
  if (len < 1 || len > cap) return;
  const int pos = len - 1;
  const int blk = p.block_tables[(int64_t)s * p.max_blocks_per_seq + (pos >> p.block_shift)];
  if ((unsigned)blk >= (unsigned)p.num_blocks) return;
  const int64_t eb = elem_bytes;
  const int64_t dst = ((int64_t)blk * p.kv_stride_block +
                       (int64_t)(pos & ((1 << p.block_shift) - 1)) * p.kv_stride_token +
                       (int64_t)head * p.kv_stride_head) * eb + chunk * 16;
  const int64_t src = ((int64_t)s * p.new_stride_seq + (int64_t)head * p.new_stride_head) * eb +
                      chunk * 16;
  const u32x4 kv = load_vec<u32x4>((const char *)p.key_new + src);
  const u32x4 vv = load_vec<u32x4>((const char *)p.value_new + src);
  store_vec<u32x4>((char *)const_cast<void *>(p.k_cache) + dst, kv);
  store_vec<u32x4>((char *)const_cast<void *>(p.v_cache) + dst, vv);
}

// fp8 append: token i's key/value rows quantised into fp8 (OCP e4m3) pools,
//   cache = e4m3(clamp(x / scale[head], -448, 448)), rounded to nearest even;
// NaN is stored as the positive NaN code 0x7f. One thread per 8 values of
// one (token, head) row.
template <typename S>
__device__ __forceinline__ uint32_t fp8x4(const S *x, float scale) {
  float f[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float y = (float)x[i] / scale;
    f[i] = y > 448.f ? 448.f : (y < -448.f ? -448.f : y);  // NaN passes
  }
  uint32_t w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(f[0], f[1], 0, false);
  w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(f[2], f[3], (int)w, true);
  // The conversion writes NaN as 0xff (in e4m3 nothing else is 0xff): clear
  // bit 7 of every 0xff byte. A byte of m = ~w is zero exactly there.
  const uint32_t m = ~w;
  const uint32_t nonzero = (((m & 0x7f7f7f7fu) + 0x7f7f7f7fu) | m) & 0x80808080u;
  return w ^ (~nonzero & 0x80808080u);
}

template <typename S>
__global__ void __launch_bounds__(kThreads)
reshape_and_cache_fp8(const CacheParams p, const float *__restrict__ ks,
                      const float *__restrict__ vs, int groups_per_row) {
  // The launcher guarantees num_tokens*num_kv_heads*groups_per_row < 2^31.
  const uint32_t gid = blockIdx.x * kThreads + threadIdx.x;
  const uint32_t rows = (uint32_t)p.num_tokens * (uint32_t)p.num_kv_heads;
  const uint32_t row = gid / (uint32_t)groups_per_row;
  if (row >= rows) return;
  const int grp = (int)(gid - row * (uint32_t)groups_per_row);
  const int token = (int)(row / (uint32_t)p.num_kv_heads);
  const int head = (int)(row - (uint32_t)token * (uint32_t)p.num_kv_heads);
  const int64_t slot = p.slot_mapping[token];
  if (slot < 0 || slot >= p.num_slots) return;
  const int64_t blk = slot >> p.block_shift;
  const int64_t off = slot & ((1 << p.block_shift) - 1);
  const int64_t dst = blk * p.kv_stride_block + off * p.kv_stride_token + head * p.kv_stride_head +
                      grp * 8;  // bytes: one byte per element
  const S *k = (const S *)p.key + (int64_t)token * p.key_stride_token +
               (int64_t)head * p.key_stride_head + grp * 8;
  const S *v = (const S *)p.value + (int64_t)token * p.value_stride_token +
               (int64_t)head * p.value_stride_head + grp * 8;
  S kx[8], vx[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    kx[i] = k[i];
    vx[i] = v[i];
  }
  const float kscale = ks[head], vscale = vs[head];
  const u32x2 kw = {fp8x4(kx, kscale), fp8x4(kx + 4, kscale)};
  const u32x2 vw = {fp8x4(vx, vscale), fp8x4(vx + 4, vscale)};
  store_vec<u32x2>((char *)p.k_cache + dst, kw);
  store_vec<u32x2>((char *)p.v_cache + dst, vw);
}

}  // namespace

hipError_t launch_reshape_and_cache_fp8(const CacheParams &p, int src_dtype, const float *k_scales,
                                        const float *v_scales, hipStream_t stream) {
  // Validated by the caller: head_dim a multiple of 8, 8-byte aligned rows.
  if (p.num_tokens == 0 || p.num_kv_heads == 0) return hipSuccess;
  const int groups = p.head_dim / 8;
  const int64_t per_token = (int64_t)p.num_kv_heads * groups;
  const int64_t tokens_per_launch = ((int64_t)1 << 30) / per_token;
  const int64_t eb = p.elem_bytes;
  for (int64_t t0 = 0; t0 < p.num_tokens; t0 += tokens_per_launch) {
    CacheParams q = p;
    const int64_t n = p.num_tokens - t0 < tokens_per_launch ? p.num_tokens - t0 : tokens_per_launch;
    q.num_tokens = (int32_t)n;
    q.key = (const char *)p.key + t0 * p.key_stride_token * eb;
    q.value = (const char *)p.value + t0 * p.value_stride_token * eb;
    q.slot_mapping = p.slot_mapping + t0;
    const unsigned blocks = (unsigned)((n * per_token + kThreads - 1) / kThreads);
    if (src_dtype == (int)DType::F32)
      hipLaunchKernelGGL(reshape_and_cache_fp8<float>, dim3(blocks), dim3(kThreads), 0, stream, q,
                         k_scales, v_scales, groups);
    else if (src_dtype == (int)DType::F16)
      hipLaunchKernelGGL(reshape_and_cache_fp8<_Float16>, dim3(blocks), dim3(kThreads), 0, stream, q,
                         k_scales, v_scales, groups);
    else
      hipLaunchKernelGGL(reshape_and_cache_fp8<__bf16>, dim3(blocks), dim3(kThreads), 0, stream, q,
                         k_scales, v_scales, groups);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

hipError_t launch_append_by_table(const DecodeParams &p, int elem_bytes, hipStream_t stream) {
  // Validated by the caller: 16-byte aligned pointers and strides, rows of
  // head_dim * elem_bytes bytes (a multiple of 16).
  const int chunks = p.head_dim * elem_bytes / 16;
  const int64_t work = (int64_t)p.num_seqs * p.num_kv_heads * chunks;
  if (work == 0) return hipSuccess;
  if (work >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
  const unsigned blocks = (unsigned)((work + kThreads - 1) / kThreads);
  hipLaunchKernelGGL(append_by_table_vec16, dim3(blocks), dim3(kThreads), 0, stream, p, chunks,
                     elem_bytes);
  return hipGetLastError();
}

hipError_t launch_reshape_and_cache(const CacheParams &p, hipStream_t stream) {
  if (p.num_tokens == 0 || p.num_kv_heads == 0) return hipSuccess;
  const int64_t eb = p.elem_bytes;
  const int64_t row_bytes = p.head_dim * eb;
  const bool vec = row_bytes % 16 == 0 && aligned16(p.key) && aligned16(p.value) &&
                   aligned16(p.k_cache) && aligned16(p.v_cache) &&
                   (p.key_stride_token * eb) % 16 == 0 && (p.key_stride_head * eb) % 16 == 0 &&
                   (p.value_stride_token * eb) % 16 == 0 &&
                   (p.value_stride_head * eb) % 16 == 0 && (p.kv_stride_block * eb) % 16 == 0 &&
                   (p.kv_stride_token * eb) % 16 == 0 && (p.kv_stride_head * eb) % 16 == 0;
  const int64_t per_token = (int64_t)p.num_kv_heads * (vec ? row_bytes / 16 : p.head_dim);
  // Keep each launch's thread count below 2^31 (32-bit index math in the kernels).
  const int64_t tokens_per_launch = ((int64_t)1 << 30) / per_token;
  for (int64_t t0 = 0; t0 < p.num_tokens; t0 += tokens_per_launch) {
    CacheParams q = p;
    const int64_t n = p.num_tokens - t0 < tokens_per_launch ? p.num_tokens - t0 : tokens_per_launch;
    q.num_tokens = (int32_t)n;
    q.key = (const char *)p.key + t0 * p.key_stride_token * eb;
    q.value = (const char *)p.value + t0 * p.value_stride_token * eb;
    q.slot_mapping = p.slot_mapping + t0;
    const int64_t work = n * per_token;
    const unsigned blocks = (unsigned)((work + kThreads - 1) / kThreads);
    if (vec)
      hipLaunchKernelGGL(reshape_and_cache_vec16, dim3(blocks), dim3(kThreads), 0, stream, q,
                         (int)(row_bytes / 16));
    else if (eb == 4)
      hipLaunchKernelGGL(reshape_and_cache_elem<uint32_t>, dim3(blocks), dim3(kThreads), 0, stream,
                         q);
    else
      hipLaunchKernelGGL(reshape_and_cache_elem<uint16_t>, dim3(blocks), dim3(kThreads), 0, stream,
                         q);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

}  // namespace clv
