// decode_stream.hip - balanced ("stream") paged decode.
//
// With ragged contexts a grid of one workgroup per (sequence, kv head,
// partition) leaves the longest sequences running alone at the end. Here a
// fixed number of waves W split the flattened space of 16-token steps
//   (sequence, kv head, query-head chunk, step)    -- one "segment" per
// (sequence, kv head, chunk), N steps in total
// evenly: wave w takes steps [w*N/W, (w+1)*N/W), crossing segment borders
// (W is capped at N, so no wave is idle and a segment's partials come from
// consecutive waves).
// Each wave keeps its loads one step ahead (also across a border) and, for
// every segment it touches, writes one partial (normalised context, row max,
// row sum) to the workspace; stream_reduce merges the partials of each
// (sequence, query head) with the log-sum-exp rule of the reference's
// partial-softmax merge (src/core/resident_kv_store.py:2497-2509).
//
// Every workgroup derives the segment prefix sums itself (in LDS) from
// context_lens; workgroup 0 also stores them for the reduce kernel.
#include "decode_mfma.h"

namespace clv {
namespace {

constexpr int kWaves = 4;  // independent waves per workgroup
constexpr int kThreads = kWaves * 64;

// Wave owning step x when N steps are split over W waves: the largest w
// with floor(w*N/W) <= x.
__device__ __forceinline__ int wave_of(int x, int64_t W, int64_t N) {
  return (int)(((int64_t)(x + 1) * W - 1) / N);
}

__device__ __forceinline__ int span_start(int w, int64_t W, int64_t N) {
  return (int)((int64_t)w * N / W);
}

__device__ __forceinline__ int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }

// In-place exclusive prefix sum of buf[0, n) by the 256 threads of the
// workgroup; buf[n] receives the total, which is also returned.
__device__ int block_exclusive_scan(int *buf, int n, int *tmp) {
  const int tid = threadIdx.x;
  const int per = (n + kThreads - 1) / kThreads;
  const int b = min(n, tid * per), e = min(n, b + per);
  int local = 0;
  for (int i = b; i < e; ++i) local += buf[i];
  int x = local;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if ((tid & 63) >= off) x += y;
  }
  if ((tid & 63) == 63) tmp[tid >> 6] = x;
  __syncthreads();
  int run = x - local;
  for (int w = 0; w < (tid >> 6); ++w) run += tmp[w];
  for (int i = b; i < e; ++i) {
    const int v = buf[i];
    buf[i] = run;
    run += v;
  }
  const int total = tmp[0] + tmp[1] + tmp[2] + tmp[3];
  __syncthreads();
  if (tid == 0) buf[n] = total;
  __syncthreads();
  return total;
}

template <typename T, int D, bool UNI>
__global__ void __launch_bounds__(kThreads) paged_decode_stream(const DecodeParams p) {
  typedef DecodeWave<T, D, UNI> WV;
  typedef typename WV::qk_t qk_t;
  __shared__ int s_seg[kStreamMaxSegments + 1];
  __shared__ int s_slot[kStreamMaxSegments + 1];
  __shared__ int s_tmp[kWaves];

  const int nseg = p.num_segments;
  const int per_seq = p.num_kv_heads * p.n_gchunks;
  for (int i = threadIdx.x; i < nseg; i += kThreads)
    s_seg[i] = (clamp_ctx(p, i / per_seq) + WV::STEP - 1) / WV::STEP;
  __syncthreads();
  const int64_t N = block_exclusive_scan(s_seg, nseg, s_tmp);
  // At most one wave per step, so that every wave owns at least one step and
  // each segment's partials come from consecutive waves.
  const int64_t W = min((int64_t)p.num_waves, N);
  if (N > 0) {
    for (int i = threadIdx.x; i < nseg; i += kThreads) {
      const int a = s_seg[i], b = s_seg[i + 1];
      s_slot[i] = b > a ? wave_of(b - 1, W, N) - wave_of(a, W, N) + 1 : 0;
    }
  } else {
    for (int i = threadIdx.x; i < nseg; i += kThreads) s_slot[i] = 0;
  }
  __syncthreads();
  block_exclusive_scan(s_slot, nseg, s_tmp);
  if (blockIdx.x == 0) {
    for (int i = threadIdx.x; i <= nseg; i += kThreads) {
      p.seg_prefix[i] = s_seg[i];
      p.slot_prefix[i] = s_slot[i];
    }
  }

  const int wid = (int)blockIdx.x * kWaves + uni(threadIdx.x >> 6);
  if (N == 0 || wid >= W) return;
  const int st = span_start(wid, W, N);
  const int en = span_start(wid + 1, W, N);
  if (st >= en) return;

  // Segment holding step st: the last one whose first step is <= st.
  int seg;
  {
    int lo = 0, hi = nseg - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_seg[mid] <= st) lo = mid; else hi = mid - 1;
    }
    seg = uni(lo);
  }

  WV w;
  w.init(p);

  // Per-segment state of the step being computed.
  int cur_s, cur_ng, cur_ctx, cur_first, cur_end;
  SegGeom cur_geo;
  qk_t q_cur[WV::NQK];
  auto open_seg = [&](int sg, int &s_, int &ng_, int &ctx_, int &first_, int &end_, SegGeom &geo_,
                      qk_t (&q_)[WV::NQK]) {
    s_ = sg / per_seq;
    const int rem = sg - s_ * per_seq;
    const int kvh = rem / p.n_gchunks;
    const int g0 = (rem - kvh * p.n_gchunks) * 16;
    ng_ = min(16, p.group - g0);
    ctx_ = clamp_ctx(p, s_);
    first_ = uni(s_seg[sg]);
    end_ = uni(s_seg[sg + 1]);
    geo_ = seg_geom<T>(p, s_, kvh, ctx_);
    w.load_q(p, s_, kvh * p.group + g0, ng_, q_);
  };
  open_seg(seg, cur_s, cur_ng, cur_ctx, cur_first, cur_end, cur_geo, q_cur);

  int x = st;
  typename WV::Regs A, B;
  w.issue(cur_geo, (x - cur_first) * WV::STEP, A);

  // One step: prefetch step x+1 (maybe of the next segment) into `nxt`,
  // fold step x from `cur`, close the segment when it ends here.
  auto step = [&](typename WV::Regs &cur, typename WV::Regs &nxt) -> bool {
    const int nx = x + 1;
    const bool more = nx < en;
    const bool newseg = more && nx >= cur_end;
    int n_seg = seg, n_s = cur_s, n_ng = cur_ng, n_ctx = cur_ctx, n_first = cur_first,
        n_end = cur_end;
    SegGeom n_geo = cur_geo;
    qk_t q_next[WV::NQK];
    if (newseg) {
      n_seg = seg + 1;
      while (uni(s_seg[n_seg + 1]) <= nx) ++n_seg;  // skip empty segments
      open_seg(n_seg, n_s, n_ng, n_ctx, n_first, n_end, n_geo, q_next);
    }
    // Past the span end, re-read step x (cache resident, never used).
    w.issue(n_geo, ((more ? nx : x) - n_first) * WV::STEP, nxt);
    w.compute((x - cur_first) * WV::STEP, cur_ctx, cur, q_cur);
    if (!more || newseg) {
      w.reduce_rowsum();
      const int piece = wid - wave_of(cur_first, W, N);
      const int64_t row0 = ((int64_t)uni(s_slot[seg]) + piece) * 16;
      w.store_partial(p.ws_o, p.ws_m, p.ws_l, row0, cur_ng);
      w.reset();
      if (!more) return false;
      seg = n_seg;
      cur_s = n_s;
      cur_ng = n_ng;
      cur_ctx = n_ctx;
      cur_first = n_first;
      cur_end = n_end;
      cur_geo = n_geo;
#pragma unroll
      for (int i = 0; i < WV::NQK; ++i) q_cur[i] = q_next[i];
    }
    x = nx;
    return true;
  };
  for (;;) {
    if (!step(A, B)) break;
    if (!step(B, A)) break;
  }
}

// Merge n partial rows (row i at index i * stride of wm/wl and i * stride * D
// of wo) into dst, as src/core/resident_kv_store.py:2497-2509 does pairwise:
//   M = max_i m_i, w_i = l_i e^{m_i - M}, out = sum_i c_i w_i / max(sum_i w_i, 1e-12).
template <typename T, int D>
__device__ __forceinline__ void merge_partials(const float *wm, const float *wl, const float *wo,
                                               int64_t stride, int n, T *dst) {
  constexpr int EPL = (D + 63) / 64;
  const int lane = threadIdx.x & 63;
  float M = kNegInf;
  for (int i = lane; i < n; i += 64) M = fmaxf(M, wm[(int64_t)i * stride]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, shfl_xor(M, off));
  const float Msub = (M == kNegInf) ? 0.f : M;
  float L = 0.f;
  float acc[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
  for (int i = 0; i < n; ++i) {
    const int64_t r = (int64_t)i * stride;
    const float wt = wl[r] * fast_exp2((wm[r] - Msub) * kLog2e);
    L += wt;
#pragma unroll
    for (int e = 0; e < EPL; ++e)
      if (lane + 64 * e < D) acc[e] += wo[r * D + lane + 64 * e] * wt;
  }
  const float inv = 1.f / fmaxf(L, 1e-12f);
#pragma unroll
  for (int e = 0; e < EPL; ++e)
    if (lane + 64 * e < D) dst[lane + 64 * e] = from_f32<T>(acc[e] * inv);
}

// One wave per (sequence, query head).
template <typename T, int D>
__global__ void __launch_bounds__(256) stream_reduce(const DecodeParams p) {
  const int64_t idx = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (idx >= (int64_t)p.num_seqs * p.num_heads) return;
  const int s = (int)(idx / p.num_heads);
  const int h = (int)(idx - (int64_t)s * p.num_heads);
  const int kvh = h / p.group;
  const int gall = h - kvh * p.group;
  const int seg = (s * p.num_kv_heads + kvh) * p.n_gchunks + gall / 16;
  const int g = gall % 16;
  const int a = p.seg_prefix[seg], b = p.seg_prefix[seg + 1];
  const int64_t N = p.seg_prefix[p.num_segments];
  const int64_t W = min((int64_t)p.num_waves, N);
  int n = 0;
  if (b > a) n = wave_of(b - 1, W, N) - wave_of(a, W, N) + 1;
  const int64_t row0 = (int64_t)p.slot_prefix[seg] * 16 + g;
  T *dst = (T *)p.out + (int64_t)s * p.out_stride_seq + (int64_t)h * p.out_stride_head;
  merge_partials<T, D>(p.ws_m + row0, p.ws_l + row0, p.ws_o + row0 * D, 16, n, dst);
}

template <typename T, int D>
hipError_t launch_stream_td(const DecodeParams &p, hipStream_t stream) {
  const dim3 grid((unsigned)((p.num_waves + kWaves - 1) / kWaves));
  if (p.block_shift >= 4)
    hipLaunchKernelGGL((paged_decode_stream<T, D, true>), grid, dim3(kThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((paged_decode_stream<T, D, false>), grid, dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_stream_t(const DecodeParams &p, hipStream_t stream) {
  if (p.head_dim == 128) return launch_stream_td<T, 128>(p, stream);
  if (p.head_dim == 64) return launch_stream_td<T, 64>(p, stream);
  return hipErrorInvalidValue;
}

template <typename T>
hipError_t launch_sreduce_t(const DecodeParams &p, hipStream_t stream) {
  const int64_t rows = (int64_t)p.num_seqs * p.num_heads;
  const dim3 grid((unsigned)((rows + 3) / 4));
  if (p.head_dim == 128)
    hipLaunchKernelGGL((stream_reduce<T, 128>), grid, dim3(256), 0, stream, p);
  else if (p.head_dim == 64)
    hipLaunchKernelGGL((stream_reduce<T, 64>), grid, dim3(256), 0, stream, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace

bool decode_stream_supported(DType dt, int head_dim, int block_size, int64_t num_segments) {
  return decode_mfma_supported(dt, head_dim, block_size) && num_segments <= kStreamMaxSegments;
}

hipError_t launch_decode_stream(const DecodeParams &p, DType dt, hipStream_t stream) {
  if (dt == DType::BF16) return launch_stream_t<__bf16>(p, stream);
  if (dt == DType::F16) return launch_stream_t<_Float16>(p, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_stream_reduce(const DecodeParams &p, DType dt, hipStream_t stream) {
  if (dt == DType::BF16) return launch_sreduce_t<__bf16>(p, stream);
  if (dt == DType::F16) return launch_sreduce_t<_Float16>(p, stream);
  return hipErrorInvalidValue;
}

}  // namespace clv
