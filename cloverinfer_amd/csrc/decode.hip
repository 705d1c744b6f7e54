// decode.hip - paged-attention decode for gfx950.
//
// Computes, per (sequence s, query head h):
//   out[s,h,:] = sum_t softmax_t(scale * q[s,h,:].K[t,kvh,:]) V[t,kvh,:]
// over the first context_lens[s] tokens of the sequence's block table,
// kvh = h / group. This is the operation of the reference's
// paged_attention_kernel (src/kernels/csrc/attention.cu:15-115) with GQA and
// an explicit scale, and of CpuAttentionBackend's fp32
// einsum/softmax/einsum (src/core/attention_backend.py:116-118).
//
// Work decomposition: one workgroup per (sequence, kv head, query-head chunk
// of <= 16, partition); split-K workgroups hold up to four of those, adjacent
// kv heads over the same partition, one wave each. The query heads that share
// a kv head are packed, so every K/V byte is read from HBM once per kv head.
// The partition is the whole context (single pass) or partition_size tokens
// (split-K, followed by splitk_reduce).
//
// fp16/bf16 use MFMA (v_mfma_f32_16x16x32_*): per 32-token step a wave runs
//   S^T[t, g]  = K[t, :] . Q[g, :]           (2 x D/32 MFMAs, K straight from HBM)
//   O[g, d]   += P[g, t] V[t, d]             (D/16 MFMAs)
// with the online softmax in fp32 between the two. The token order inside the
// PV contraction is chosen so that each lane's P values (C layout of the first
// MFMA) are exactly its A operand of the second, and V is loaded as 16-byte
// row chunks whose 16-bit elements are regrouped in registers (v_perm) into
// the B operand: no LDS round trip on the hot loop.
// fp32 (and shapes MFMA does not cover) use a VALU kernel with the same
// decomposition and the same epilogue.
#include "decode_mfma.h"

namespace clv {
namespace {

template <typename T>
__device__ __forceinline__ KvView kv_view(const DecodeParams &p, int s, int kvh) {
  KvView v;
  v.bt = p.block_tables + (int64_t)s * p.max_blocks_per_seq;
  v.kbase = (const char *)p.k_cache + (int64_t)kvh * p.kv_stride_head * (int64_t)sizeof(T);
  v.vbase = (const char *)p.v_cache + (int64_t)kvh * p.kv_stride_head * (int64_t)sizeof(T);
  v.sblk = p.kv_stride_block * (int64_t)sizeof(T);
  v.stok = p.kv_stride_token * (int64_t)sizeof(T);
  v.block_shift = p.block_shift;
  v.num_blocks = (unsigned)p.num_blocks;
  return v;
}

template <typename T>
__device__ __forceinline__ OutDesc<T> out_desc(const DecodeParams &p, int s, int h0, int part) {
  OutDesc<T> od;
  od.split = p.partition_size > 0;
  od.out = (T *)p.out + (int64_t)s * p.out_stride_seq + (int64_t)h0 * p.out_stride_head;
  od.out_stride = p.out_stride_head;
  const int64_t row0 = ((int64_t)s * p.num_heads + h0) * p.max_parts + part;
  od.ws_o = p.ws_o + row0 * p.head_dim;
  od.ws_m = p.ws_m + row0;
  od.ws_l = p.ws_l + row0;
  od.ws_stride = p.max_parts;
  return od;
}

// ---------------------------------------------------------------- MFMA kernel
// One workgroup (NW waves) per (sequence, kv head, 16-row query chunk,
// partition); wave w takes the partition's 16-token steps w, w + NW, ...
// with the loads of its next step in flight while the current one is
// computed (two register sets), and the waves' partials are merged in LDS.
// Ring depths: a third register set measured 3-4 % slower.
//
// APPEND (single pass, one query-head chunk per kv head): the workgroup first
// writes sequence s's new key/value row of its kv head at position
// context_lens[s] - 1 (when that position is attended), then attends over it.
// The barrier's workgroup-scope release/acquire orders those stores before
// every wave's loads (the waves of a workgroup share one CU's caches), and no
// other workgroup reads the row.
//
// HG > 1 (split-K, NW = 1): the workgroup holds HG independent waves, wave w
// taking kv head HG * (blockIdx.y / n_gchunks) + w over the same partition,
// so that the rows of a token for HG adjacent kv heads are read together (one
// contiguous range of the token's row in the pools).
template <typename T, int D, int NW, bool UNI, bool APPEND = false, int HG = 1>
__global__ void __launch_bounds__(NW * HG * 64)
paged_decode_mfma(const DecodeParams p, const int32_t *__restrict__ tables) {
  static_assert(HG == 1 || (NW == 1 && !APPEND), "head groups: one wave per kv head");
  typedef typename GridWave<T, D, UNI>::type W;
  __shared__ WaveSmem<NW, 16, D> sms[HG];

  const int hw = HG > 1 ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : 0;
  WaveSmem<NW, 16, D> &sm = sms[hw];
  const int wave = HG > 1 ? 0 : __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int s = blockIdx.z;
  const int kvg = blockIdx.y / p.n_gchunks;
  const int kvh = kvg * HG + hw;
  const int g0 = (blockIdx.y - kvg * p.n_gchunks) * 16;
  const int ng = min(16, p.group - g0);
  const int h0 = kvh * p.group + g0;

  const int ctx = clamp_ctx(p, s);
  if constexpr (APPEND) {
    if (ctx > 0 && ctx == p.context_lens[s]) {
      const int pos = ctx - 1;
      const int blk = tables[(int64_t)s * p.max_blocks_per_seq + (pos >> p.block_shift)];
      if ((unsigned)blk < (unsigned)p.num_blocks) {
        const int64_t row = (int64_t)blk * p.kv_stride_block +
                            (int64_t)(pos & ((1 << p.block_shift) - 1)) * p.kv_stride_token +
                            (int64_t)kvh * p.kv_stride_head;
        const int64_t src = (int64_t)s * p.new_stride_seq + (int64_t)kvh * p.new_stride_head;
        constexpr int C16 = D * (int)sizeof(T) / 16;  // 16-byte chunks per row
        constexpr int E16 = 16 / (int)sizeof(T);
        for (int i = threadIdx.x; i < 2 * C16; i += NW * 64) {
          const bool val = i >= C16;
          const int c = val ? i - C16 : i;
          const T *from = (const T *)(val ? p.value_new : p.key_new) + src + c * E16;
          T *to = (T *)(val ? p.v_cache : p.k_cache) + row + c * E16;
          store_vec<u32x4>(to, load_vec<u32x4>(from));
        }
      }
    }
    __syncthreads();
  }
  int t_begin = 0, t_end = ctx;
  if (p.partition_size > 0) {
    t_begin = blockIdx.x * p.partition_size;
    if (t_begin >= ctx) return;  // whole workgroup: nothing to do
    t_end = min(ctx, t_begin + p.partition_size);
  }

  W w;
  w.init(p);
  typename W::qk_t qop[W::NQK];
  w.load_q(p, s, h0, ng, qop);
  const SegGeom geo = seg_geom<T>(p, s, kvh, t_end, tables);

  // The prefetch is unconditional (a branch around it makes the compiler wait
  // for every outstanding load): past the wave's last step it re-reads that
  // step's rows, which are still in cache, and the data is never used.
  const int stride = NW * W::STEP;
  const int first = t_begin + wave * W::STEP;
  if (first < t_end) {
    const int last = first + ((t_end - 1 - first) / stride) * stride;
    int base = first;
    if constexpr (sizeof(T) == 2) {
      // Two register sets, each refilled right after it is folded (split-K
      // over 16-bit pools: 2.6 % faster than the alternating form below).
      typename W::Regs R[2];
      w.issue(geo, base, R[0]);
      w.issue(geo, min(base + stride, last), R[1]);
      bool done = false;
      while (!done) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          if (!done) {
            w.compute(base, t_end, R[i], qop);
            base += stride;
            if (base > last) done = true;
            else w.issue(geo, min(base + stride, last), R[i]);
          }
        }
      }
    } else {
      // fp32 (16 KiB per step): issuing the next set before folding the
      // current one measured 8 % faster than the form above.
      typename W::Regs A, B;
      w.issue(geo, base, A);
      for (;;) {
        w.issue(geo, min(base + stride, last), B);
        w.compute(base, t_end, A, qop);
        base += stride;
        if (base > last) break;
        w.issue(geo, min(base + stride, last), A);
        w.compute(base, t_end, B, qop);
        base += stride;
        if (base > last) break;
      }
    }
  }

  w.reduce_rowsum();
  if (w.j == 0) {
    sm.m[wave][w.n16] = w.m_run;
    sm.l[wave][w.n16] = w.l_run;
  }
  // Lane holds O[g = 4j + r][d = W::col_of(n16, m)].
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float *dst = &sm.o[wave][4 * w.j + r][0];
#pragma unroll
    for (int m = 0; m < W::CH; m += 4) {
      f32x4 v = {w.o[m][r], w.o[m + 1][r], w.o[m + 2][r], w.o[m + 3][r]};
      store_vec<f32x4>(dst + W::col_of(w.n16, m), v);
    }
  }
  __syncthreads();
  merge_and_store<T, NW, 16, D>(sm, ng, out_desc<T>(p, s, h0, blockIdx.x),
                                HG > 1 ? (int)(threadIdx.x & 63) : (int)threadIdx.x);
}

// ---------------------------------------------------------------- VALU kernel
template <typename T, int D, int GM, int NW>
__global__ void __launch_bounds__(NW * 64) paged_decode_valu(const DecodeParams p) {
  __shared__ WaveSmem<NW, GM, D> sm;
  const int s = blockIdx.z;
  const int kvh = blockIdx.y / p.n_gchunks;
  const int g0 = (blockIdx.y - kvh * p.n_gchunks) * GM;
  const int ng = min(GM, p.group - g0);
  const int h0 = kvh * p.group + g0;

  const int ctx = clamp_ctx(p, s);
  int t_begin = 0, t_end = ctx;
  if (p.partition_size > 0) {
    t_begin = blockIdx.x * p.partition_size;
    if (t_begin >= ctx) return;
    t_end = min(ctx, t_begin + p.partition_size);
  }
  const T *q0 = (const T *)p.q + (int64_t)s * p.q_stride_seq + (int64_t)h0 * p.q_stride_head;
  valu_attend<T, D, GM, NW>(q0, p.q_stride_head, ng, kv_view<T>(p, s, kvh), t_begin, t_end,
                            p.scale_log2, sm);
  __syncthreads();
  merge_and_store<T, NW, GM, D>(sm, ng, out_desc<T>(p, s, h0, blockIdx.x));
}

// ---------------------------------------------------------------- split-K reduce
// One wave per (sequence, query head). Restates the partial-softmax merge of
// src/core/resident_kv_store.py:2497-2509 over all partitions at once:
//   M = max_i m_i,  w_i = l_i e^{m_i - M},  out = sum_i c_i w_i / max(sum_i w_i, 1e-12).
// One workgroup (4 waves) per (sequence, query head): the partitions' partials
// are merged by lse_merge.
template <typename T, int D>
__global__ void __launch_bounds__(256) splitk_reduce(const DecodeParams p) {
  __shared__ float smem[4 * (D + 1)];
  const int64_t idx = blockIdx.x;
  const int s = (int)(idx / p.num_heads);
  const int h = (int)(idx - (int64_t)s * p.num_heads);
  const int ctx = clamp_ctx(p, s);
  const int nparts = (ctx + p.partition_size - 1) / p.partition_size;
  const int64_t row0 = idx * p.max_parts;
  T *dst = (T *)p.out + (int64_t)s * p.out_stride_seq + (int64_t)h * p.out_stride_head;
  lse_merge<T, D, 4>(p.ws_m + row0, p.ws_l + row0, p.ws_o + row0 * D, 1, D, nparts, dst, smem);
}

template <typename T, int D, int NW, bool APPEND = false, int HG = 1>
hipError_t launch_mfma_tdw(const DecodeParams &p, hipStream_t stream) {
  if (p.num_kv_heads % HG != 0) return hipErrorInvalidValue;
  const dim3 grid(p.partition_size > 0 ? (unsigned)p.max_parts : 1u,
                  (unsigned)(p.num_kv_heads / HG * p.n_gchunks), (unsigned)p.num_seqs);
  if (p.block_shift >= 4)
    hipLaunchKernelGGL((paged_decode_mfma<T, D, NW, true, APPEND, HG>), grid, dim3(NW * HG * 64),
                       0, stream, p, p.block_tables);
  else
    hipLaunchKernelGGL((paged_decode_mfma<T, D, NW, false, APPEND, HG>), grid,
                       dim3(NW * HG * 64), 0, stream, p, p.block_tables);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_mfma_append_t(const DecodeParams &p, hipStream_t stream) {
  if (p.head_dim == 128) return launch_mfma_tdw<T, 128, 4, true>(p, stream);
  if (p.head_dim == 64) return launch_mfma_tdw<T, 64, 4, true>(p, stream);
  return hipErrorInvalidValue;
}

// Waves per workgroup: a single pass splits each (possibly long) context over
// four waves (kernel us with 2 / 4 / 8 waves: ragged GQA-7B bf16 303 / 242 /
// 239, MHA Llama-7B fp16 377 / 346 / 355, GQA-7B over fp32 447 / 430 / 437);
// split-K already has a workgroup per partition, and one wave
// each measured best there (partition 512; kernel us with 4 / 2 / 1 waves:
// 16 x 32K-token fp16 365 / 358 / 358, the ragged GQA-7B bf16 batch
// 286 / 274 / 270, the same over fp32 pools 574 / 511 / 484; 8 waves: 414
// on the first).
// Split-K workgroups hold a head group of four one-wave kv heads where the
// kv-head count allows it (16 x 32K-token fp16, 8 kv heads, partition 512:
// kernel 358.8 us with one kv head per workgroup, 364.9 with pairs, 341.5
// with fours, 341.4 with eights). A tuning build may set the preprocessor
// value CLV_SPLITK_HEAD_GROUP (1, 2, 4 or 8).
#ifndef CLV_SPLITK_HEAD_GROUP
#define CLV_SPLITK_HEAD_GROUP 4
#endif
static_assert(CLV_SPLITK_HEAD_GROUP == 1 || CLV_SPLITK_HEAD_GROUP == 2 ||
                  CLV_SPLITK_HEAD_GROUP == 4 || CLV_SPLITK_HEAD_GROUP == 8,
              "split-K head group 1, 2, 4 or 8");
template <typename T, int D>
hipError_t launch_mfma_td(const DecodeParams &p, hipStream_t stream) {
  if (p.partition_size > 0) {
    constexpr int HG = CLV_SPLITK_HEAD_GROUP;
    if constexpr (HG > 1)
      if (p.num_kv_heads % HG == 0) return launch_mfma_tdw<T, D, 1, false, HG>(p, stream);
    return launch_mfma_tdw<T, D, 1>(p, stream);
  }
  return launch_mfma_tdw<T, D, 4>(p, stream);
}

template <typename T>
hipError_t launch_mfma_t(const DecodeParams &p, hipStream_t stream) {
  if (p.head_dim == 128) return launch_mfma_td<T, 128>(p, stream);
  if (p.head_dim == 64) return launch_mfma_td<T, 64>(p, stream);
  return hipErrorInvalidValue;
}

template <typename T, int D>
hipError_t launch_valu_td(const DecodeParams &p, hipStream_t stream) {
  // Two waves for D = 256 keep the per-wave LDS partials within 64 KiB.
  constexpr int NW = D >= 256 ? 2 : 4;
  const int gm = p.n_gchunks > 1 ? 16 : p.group;  // rows per workgroup chunk
  const dim3 grid(p.partition_size > 0 ? (unsigned)p.max_parts : 1u,
                  (unsigned)(p.num_kv_heads * p.n_gchunks), (unsigned)p.num_seqs);
  if (gm <= 1)
    hipLaunchKernelGGL((paged_decode_valu<T, D, 1, NW>), grid, dim3(NW * 64), 0, stream, p);
  else if (gm <= 4)
    hipLaunchKernelGGL((paged_decode_valu<T, D, 4, NW>), grid, dim3(NW * 64), 0, stream, p);
  else
    hipLaunchKernelGGL((paged_decode_valu<T, D, 16, NW>), grid, dim3(NW * 64), 0, stream, p);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_valu_t(const DecodeParams &p, hipStream_t stream) {
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

template <typename T>
hipError_t launch_reduce_t(const DecodeParams &p, hipStream_t stream) {
  const int64_t rows = (int64_t)p.num_seqs * p.num_heads;
  if (rows <= 0) return hipSuccess;
  if (rows > 0x7fffffff) return hipErrorInvalidValue;
  const dim3 grid((unsigned)rows);
  switch (p.head_dim) {
    case 8: hipLaunchKernelGGL((splitk_reduce<T, 8>), grid, dim3(256), 0, stream, p); break;
    case 16: hipLaunchKernelGGL((splitk_reduce<T, 16>), grid, dim3(256), 0, stream, p); break;
    case 32: hipLaunchKernelGGL((splitk_reduce<T, 32>), grid, dim3(256), 0, stream, p); break;
    case 64: hipLaunchKernelGGL((splitk_reduce<T, 64>), grid, dim3(256), 0, stream, p); break;
    case 128: hipLaunchKernelGGL((splitk_reduce<T, 128>), grid, dim3(256), 0, stream, p); break;
    case 256: hipLaunchKernelGGL((splitk_reduce<T, 256>), grid, dim3(256), 0, stream, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

bool decode_mfma_supported(DType dt, int head_dim, int block_size) {
  // fp32 runs on the fp32 MFMA wave (DecodeWaveF32).
  return (dt == DType::F16 || dt == DType::BF16 || dt == DType::F32) &&
         (head_dim == 64 || head_dim == 128) && block_size >= 4;
}

hipError_t launch_decode_mfma(const DecodeParams &p, DType dt, hipStream_t stream) {
  if (dt == DType::BF16) return launch_mfma_t<__bf16>(p, stream);
  if (dt == DType::F16) return launch_mfma_t<_Float16>(p, stream);
  if (dt == DType::F32) return launch_mfma_t<float>(p, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_decode_mfma_append(const DecodeParams &p, DType dt, hipStream_t stream) {
  if (p.partition_size != 0 || p.n_gchunks != 1) return hipErrorInvalidValue;
  if (dt == DType::BF16) return launch_mfma_append_t<__bf16>(p, stream);
  if (dt == DType::F16) return launch_mfma_append_t<_Float16>(p, stream);
  if (dt == DType::F32) return launch_mfma_append_t<float>(p, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_decode_valu(const DecodeParams &p, DType dt, hipStream_t stream) {
  switch (dt) {
    case DType::F32: return launch_valu_t<float>(p, stream);
    case DType::F16: return launch_valu_t<_Float16>(p, stream);
    case DType::BF16: return launch_valu_t<__bf16>(p, stream);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_splitk_reduce(const DecodeParams &p, DType dt, hipStream_t stream) {
  switch (dt) {
    case DType::F32: return launch_reduce_t<float>(p, stream);
    case DType::F16: return launch_reduce_t<_Float16>(p, stream);
    case DType::BF16: return launch_reduce_t<__bf16>(p, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace clv
