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
// of <= 16, partition). The query heads that share a kv head are packed, so
// every K/V byte is read from HBM once per kv head. The partition is the
// whole context (single pass) or partition_size tokens (split-K, followed by
// splitk_reduce).
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
#include "attn_common.h"

namespace clv {
namespace {

constexpr int kStep = 32;  // tokens per wave step in the MFMA kernel

// Clamp a context length to what the grid and the block table cover.
__device__ __forceinline__ int clamp_ctx(const DecodeParams &p, int s) {
  int ctx = p.context_lens[s];
  const int cap = min(p.max_context_len, p.max_blocks_per_seq << p.block_shift);
  return max(0, min(ctx, cap));
}

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

template <int CH> struct VChunk;
template <> struct VChunk<8> { typedef u32x4 type; };  // D = 128: 16 bytes
template <> struct VChunk<4> { typedef u32x2 type; };  // D = 64: 8 bytes

// ---------------------------------------------------------------- MFMA kernel
// Loads of one 16-token step: the K rows (A operands of S^T = K Q^T, lane
// row n16) and the V rows of the 4 tokens 4j..4j+3 whose P values the lane
// holds (B operands of O += P V).
template <int NQK, typename vchunk_t>
struct StepRegs {
  u32x4 k[NQK];
  vchunk_t v[4];
  bool ok;  // this lane's V rows lie in a readable block
};

// Per 16-token step a wave runs D/32 MFMAs 16x16x32 for the scores
//   S^T[t, g] = K[t, :] . Q[g, :]     (lane holds S[g = n16][t = 4j + r])
// and 2 x D/16 MFMAs 16x16x16 for O[g, d] += P[g, t] V[t, d], whose A operand
// is exactly the lane's 4 P values (P split into a 16-bit high part and its
// rounding residual, so P.V keeps fp32-level accuracy) and whose B operand
// for output column block m is element m of the lane's 4 V row chunks,
// regrouped with v_perm. Loads of the next step are in flight while the
// current one is computed (two register sets).
// UNI: block_size >= 16, so each step sits in one block and its block-table
// entry is wave-uniform (scalar load). Otherwise (block_size 4 or 8) lanes
// look up their own rows.
template <typename T, int D, int NW, bool UNI>
__global__ void __launch_bounds__(NW * 64) paged_decode_mfma(const DecodeParams p) {
  typedef Mfma16x16x32<T> MfK;
  typedef Mfma16x16x16<T> MfV;
  typedef typename MfK::op_t qk_t;
  typedef typename MfV::op_t pv_t;
  constexpr int NQK = D / 32;  // QK MFMAs per step
  constexpr int CH = D / 16;   // V elements per lane per token = PV output blocks
  constexpr int EB = (int)sizeof(T);
  constexpr int STEP = 16;
  typedef typename VChunk<CH>::type vchunk_t;
  typedef StepRegs<NQK, vchunk_t> Regs;

  __shared__ WaveSmem<NW, 16, D> sm;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n16 = lane & 15;
  const int j = lane >> 4;
  const int s = blockIdx.z;
  const int kvh = blockIdx.y / p.n_gchunks;
  const int g0 = (blockIdx.y - kvh * p.n_gchunks) * 16;
  const int ng = min(16, p.group - g0);
  const int h0 = kvh * p.group + g0;

  const int ctx = clamp_ctx(p, s);
  int t_begin = 0, t_end = ctx;
  if (p.partition_size > 0) {
    t_begin = blockIdx.x * p.partition_size;
    if (t_begin >= ctx) return;  // whole workgroup: nothing to do
    t_end = min(ctx, t_begin + p.partition_size);
  }

  // Q as the B operand of S^T = K Q^T: lane holds Q[g = n16][d = 32i + 8j .. +8].
  qk_t qop[NQK];
  {
    const T *qrow = (const T *)p.q + (int64_t)s * p.q_stride_seq + (int64_t)(h0 + n16) * p.q_stride_head;
#pragma unroll
    for (int i = 0; i < NQK; ++i) {
      u32x4 w = {0u, 0u, 0u, 0u};
      if (n16 < ng) w = load_vec<u32x4>(qrow + 32 * i + 8 * j);
      qop[i] = __builtin_bit_cast(qk_t, w);
    }
  }

  const int32_t *bt = p.block_tables + (int64_t)s * p.max_blocks_per_seq;
  const char *kbase = (const char *)p.k_cache + (int64_t)kvh * p.kv_stride_head * EB;
  const char *vbase = (const char *)p.v_cache + (int64_t)kvh * p.kv_stride_head * EB;
  const int64_t sblk = p.kv_stride_block * EB;
  const int64_t stok = p.kv_stride_token * EB;
  const int bshift = p.block_shift;
  const int bmask = (1 << bshift) - 1;
  const unsigned nblocks = (unsigned)p.num_blocks;
  // Lane offsets inside a step (bytes, below 16 rows of the token stride):
  // K row n16 at d = 8j (+32 elements per MFMA), V rows 4j + r at d = n16*CH.
  const uint32_t k_lane = (uint32_t)(n16 * stok + 8 * j * EB);
  uint32_t v_lane[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) v_lane[r] = (uint32_t)((4 * j + r) * stok + n16 * CH * EB);

  // Issue every load of the step starting at token `base` (< t_end). All
  // addresses are in bounds: rows past t_end or in unreadable blocks read a
  // readable row and are masked when the step is computed.
  auto issue = [&](int base, Regs &R) {
    if constexpr (UNI) {
      // Wave-uniform block: scalar base address plus 32-bit lane offsets.
      const int blk = bt[base >> bshift];
      const bool ok = (unsigned)blk < nblocks;
      const int64_t off = ok ? blk * sblk + (base & bmask) * stok : 0;
      R.ok = ok;
      const rsrc_t rk = make_rsrc(kbase + off);
      const rsrc_t rv = make_rsrc(vbase + off);
#pragma unroll
      for (int i = 0; i < NQK; ++i) R.k[i] = buf_load<u32x4>(rk, k_lane + 64u * i);
#pragma unroll
      for (int r = 0; r < 4; ++r) R.v[r] = buf_load<vchunk_t>(rv, v_lane[r]);
    } else {
      const int tk = base + n16;
      const int kb = tk < t_end ? bt[tk >> bshift] : 0;
      const bool kok = tk < t_end && (unsigned)kb < nblocks;
      const int64_t koff = (kok ? kb * sblk + (tk & bmask) * stok : 0) + 8 * j * EB;
      const int tv = base + 4 * j;
      const int vb = tv < t_end ? bt[tv >> bshift] : 0;
      const bool vok = tv < t_end && (unsigned)vb < nblocks;
      R.ok = vok;
      const int64_t voff = (vok ? vb * sblk + (tv & bmask) * stok : 0) + n16 * CH * EB;
#pragma unroll
      for (int i = 0; i < NQK; ++i) R.k[i] = load_vec<u32x4>(kbase + koff + 64 * i);
#pragma unroll
      for (int r = 0; r < 4; ++r) R.v[r] = load_vec<vchunk_t>(vbase + voff + r * stok);
    }
  };

  f32x4 o[CH];
#pragma unroll
  for (int m = 0; m < CH; ++m) o[m] = (f32x4){0.f, 0.f, 0.f, 0.f};
  float m_run = kNegInf;  // running max for row g = n16 (log2 domain)
  float l_run = 0.f;      // this lane's share of the row sum

  auto compute = [&](int base, Regs &R) {
    f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NQK; ++i) sacc = MfK::run(__builtin_bit_cast(qk_t, R.k[i]), qop[i], sacc);
    // Masking is needed only on a partial step or an unreadable block.
    const bool full = __all(base + STEP <= t_end && R.ok);
    float x[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool ok = full || (R.ok && base + 4 * j + r < t_end);
      x[r] = ok ? sacc[r] * p.scale_log2 : kNegInf;
    }
    if (!full) {
      const vchunk_t z = {};
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (x[r] == kNegInf) R.v[r] = z;  // keep NaN/Inf of unused slots out of P.V
    }
    float mx = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    mx = fmaxf(mx, shfl_xor(mx, 16));
    mx = fmaxf(mx, shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float msub = (m_new == kNegInf) ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - msub);
    float pf[4], lo[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) pf[r] = fast_exp2(x[r] - msub);
    l_run = l_run * alpha + ((pf[0] + pf[1]) + (pf[2] + pf[3]));
    m_run = m_new;

    // Rescale the accumulator rows g' = 4j + r by alpha of row g'.
    if (__any(alpha != 1.f)) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float a = shfl(alpha, 4 * j + r);
#pragma unroll
        for (int m = 0; m < CH; ++m) o[m][r] *= a;
      }
    }

    const pv_t pa = pack4<T>(pf);
#pragma unroll
    for (int r = 0; r < 4; ++r) lo[r] = pf[r] - (float)pa[r];
    const pv_t pl = pack4<T>(lo);
#pragma unroll
    for (int m = 0; m < CH; ++m) {
      const uint32_t w0 = (m & 1) ? pair_hi(R.v[0][m >> 1], R.v[1][m >> 1])
                                  : pair_lo(R.v[0][m >> 1], R.v[1][m >> 1]);
      const uint32_t w1 = (m & 1) ? pair_hi(R.v[2][m >> 1], R.v[3][m >> 1])
                                  : pair_lo(R.v[2][m >> 1], R.v[3][m >> 1]);
      const u32x2 w = {w0, w1};
      const pv_t vb = __builtin_bit_cast(pv_t, w);
      o[m] = MfV::run(pa, vb, o[m]);
      o[m] = MfV::run(pl, vb, o[m]);
    }
  };

  // The prefetch is unconditional (a branch around it makes the compiler wait
  // for every outstanding load): past the wave's last step it re-reads that
  // step's rows, which are still in cache, and the data is never used.
  const int stride = NW * STEP;
  const int first = t_begin + wave * STEP;
  if (first < t_end) {
    const int last = first + ((t_end - 1 - first) / stride) * stride;
    int base = first;
    Regs A, B;
    issue(base, A);
    for (;;) {
      issue(min(base + stride, last), B);
      compute(base, A);
      base += stride;
      if (base > last) break;
      issue(min(base + stride, last), A);
      compute(base, B);
      base += stride;
      if (base > last) break;
    }
  }

  // Row sums: add the four lane groups holding the same row.
  l_run += shfl_xor(l_run, 16);
  l_run += shfl_xor(l_run, 32);
  if (j == 0) {
    sm.m[wave][n16] = m_run;
    sm.l[wave][n16] = l_run;
  }
  // Lane holds O[g = 4j + r][d = n16*CH + m].
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float *dst = &sm.o[wave][4 * j + r][n16 * CH];
#pragma unroll
    for (int m = 0; m < CH; m += 4) {
      f32x4 v = {o[m][r], o[m + 1][r], o[m + 2][r], o[m + 3][r]};
      store_vec<f32x4>(dst + m, v);
    }
  }
  __syncthreads();
  merge_and_store<T, NW, 16, D>(sm, ng, out_desc<T>(p, s, h0, blockIdx.x));
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
template <typename T, int D>
__global__ void __launch_bounds__(256) splitk_reduce(const DecodeParams p) {
  constexpr int EPL = (D + 63) / 64;  // elements per lane (lanes >= D idle when D < 64)
  const int lane = threadIdx.x & 63;
  const int64_t idx = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (idx >= (int64_t)p.num_seqs * p.num_heads) return;
  const int s = (int)(idx / p.num_heads);
  const int h = (int)(idx - (int64_t)s * p.num_heads);
  const int ctx = clamp_ctx(p, s);
  const int nparts = (ctx + p.partition_size - 1) / p.partition_size;
  const int64_t row0 = idx * p.max_parts;
  const float *wm = p.ws_m + row0;
  const float *wl = p.ws_l + row0;
  const float *wo = p.ws_o + row0 * D;

  float M = kNegInf;
  for (int i = lane; i < nparts; i += 64) M = fmaxf(M, wm[i]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, shfl_xor(M, off));
  const float Msub = (M == kNegInf) ? 0.f : M;

  float L = 0.f;
  float acc[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
  for (int i = 0; i < nparts; ++i) {
    const float w = wl[i] * fast_exp2((wm[i] - Msub) * kLog2e);
    L += w;
#pragma unroll
    for (int e = 0; e < EPL; ++e)
      if (lane + 64 * e < D) acc[e] += wo[(int64_t)i * D + lane + 64 * e] * w;
  }
  const float inv = 1.f / fmaxf(L, 1e-12f);
  T *dst = (T *)p.out + (int64_t)s * p.out_stride_seq + (int64_t)h * p.out_stride_head;
#pragma unroll
  for (int e = 0; e < EPL; ++e)
    if (lane + 64 * e < D) dst[lane + 64 * e] = from_f32<T>(acc[e] * inv);
}

template <typename T, int D>
hipError_t launch_mfma_td(const DecodeParams &p, hipStream_t stream) {
  constexpr int NW = 4;
  const dim3 grid(p.partition_size > 0 ? (unsigned)p.max_parts : 1u,
                  (unsigned)(p.num_kv_heads * p.n_gchunks), (unsigned)p.num_seqs);
  if (p.block_shift >= 4)
    hipLaunchKernelGGL((paged_decode_mfma<T, D, NW, true>), grid, dim3(NW * 64), 0, stream, p);
  else
    hipLaunchKernelGGL((paged_decode_mfma<T, D, NW, false>), grid, dim3(NW * 64), 0, stream, p);
  return hipGetLastError();
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
  const dim3 grid((unsigned)((rows + 3) / 4));
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
  return (dt == DType::F16 || dt == DType::BF16) && (head_dim == 64 || head_dim == 128) &&
         block_size >= 4;
}

hipError_t launch_decode_mfma(const DecodeParams &p, DType dt, hipStream_t stream) {
  if (dt == DType::BF16) return launch_mfma_t<__bf16>(p, stream);
  if (dt == DType::F16) return launch_mfma_t<_Float16>(p, stream);
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
