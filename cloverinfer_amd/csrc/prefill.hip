// prefill.hip - chunked prefill over paged KV.
//
// Sequence s owns query rows [query_start_loc[s], query_start_loc[s+1]); its
// n_s new tokens are the last n_s of its context_lens[s] cached tokens, so
// query row i attends to cached positions p <= context_lens[s] - n_s + i.
// Row i therefore equals what CpuAttentionBackend.decode_layer
// (src/core/attention_backend.py:105-118) returns after appending new tokens
// 0..i one at a time (append-then-attend).
//
// This file holds the VALU form (any dtype; one workgroup per query row and
// kv head). The MFMA form for fp16/bf16 is in prefill_mfma.hip. In both, a
// row at index max_query_len or later of its chunk (a chunk longer than the
// caller's max_query_len, a caller error) comes out as NaN.
#include "attn_common.h"

namespace clv {
namespace {

template <typename T, int D, int GM, int NW>
__global__ void __launch_bounds__(NW * 64) chunked_prefill_valu(const PrefillParams p) {
  __shared__ WaveSmem<NW, GM, D> sm;
  const int tok = blockIdx.x;
  const int32_t *qsl = p.query_start_loc;
  if (tok < qsl[0] || tok >= qsl[p.num_seqs]) return;
  // Sequence owning row tok: largest s with qsl[s] <= tok.
  int lo = 0, hi = p.num_seqs;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (qsl[mid] <= tok) lo = mid; else hi = mid;
  }
  const int s = lo;
  const int n_new = qsl[s + 1] - qsl[s];
  const int i = tok - qsl[s];
  const int cap = p.max_blocks_per_seq << p.block_shift;
  const int ctx = max(0, min(p.context_lens[s], cap));
  const int limit = max(0, min(ctx, ctx - n_new + i + 1));

  const int n_gchunks = (p.group + GM - 1) / GM;
  const int kvh = blockIdx.y / n_gchunks;
  const int g0 = (blockIdx.y - kvh * n_gchunks) * GM;
  const int ng = min(GM, p.group - g0);
  const int h0 = kvh * p.group + g0;
  if (i >= p.max_query_len) {
    const T nan = (T)__builtin_nanf("");
    for (int idx = threadIdx.x; idx < ng * D; idx += NW * 64)
      ((T *)p.out)[(int64_t)tok * p.out_stride_token +
                   (int64_t)(h0 + idx / D) * p.out_stride_head + idx % D] = nan;
    return;
  }

  KvView kv;
  kv.bt = p.block_tables + (int64_t)s * p.max_blocks_per_seq;
  kv.kbase = (const char *)p.k_cache + (int64_t)kvh * p.kv_stride_head * (int64_t)sizeof(T);
  kv.vbase = (const char *)p.v_cache + (int64_t)kvh * p.kv_stride_head * (int64_t)sizeof(T);
  kv.sblk = p.kv_stride_block * (int64_t)sizeof(T);
  kv.stok = p.kv_stride_token * (int64_t)sizeof(T);
  kv.block_shift = p.block_shift;
  kv.num_blocks = (unsigned)p.num_blocks;

  const T *q0 = (const T *)p.q + (int64_t)tok * p.q_stride_token + (int64_t)h0 * p.q_stride_head;
  valu_attend<T, D, GM, NW>(q0, p.q_stride_head, ng, kv, 0, limit, p.scale_log2, sm);
  __syncthreads();
  OutDesc<T> od;
  od.split = false;
  od.out = (T *)p.out + (int64_t)tok * p.out_stride_token + (int64_t)h0 * p.out_stride_head;
  od.out_stride = p.out_stride_head;
  od.ws_o = od.ws_m = od.ws_l = nullptr;
  od.ws_stride = 0;
  merge_and_store<T, NW, GM, D>(sm, ng, od);
}

template <typename T, int D>
hipError_t launch_valu_td(const PrefillParams &p, hipStream_t stream) {
  constexpr int NW = D >= 256 ? 2 : 4;
  const int gm = p.group > 4 ? 16 : (p.group > 1 ? 4 : 1);
  const unsigned gch = (unsigned)((p.group + gm - 1) / gm);
  const dim3 grid((unsigned)p.num_tokens, (unsigned)p.num_kv_heads * gch);
  if (gm == 1)
    hipLaunchKernelGGL((chunked_prefill_valu<T, D, 1, NW>), grid, dim3(NW * 64), 0, stream, p);
  else if (gm == 4)
    hipLaunchKernelGGL((chunked_prefill_valu<T, D, 4, NW>), grid, dim3(NW * 64), 0, stream, p);
  else
    hipLaunchKernelGGL((chunked_prefill_valu<T, D, 16, NW>), grid, dim3(NW * 64), 0, stream, p);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_valu_t(const PrefillParams &p, hipStream_t stream) {
  switch (p.head_dim) {
    case 8: return launch_valu_td<T, 8>(p, stream);
    case 16: return launch_valu_td<T, 16>(p, stream);
    case 32: return launch_valu_td<T, 32>(p, stream);
    case 64: return launch_valu_td<T, 64>(p, stream);
    case 128: return launch_valu_td<T, 128>(p, stream);
    case 256: return launch_valu_td<T, 256>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_prefill_valu(const PrefillParams &p, DType dt, hipStream_t stream) {
  switch (dt) {
    case DType::F32: return launch_valu_t<float>(p, stream);
    case DType::F16: return launch_valu_t<_Float16>(p, stream);
    case DType::BF16: return launch_valu_t<__bf16>(p, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace clv
