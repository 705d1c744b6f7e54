// decode_stream.hip - balanced ("stream") paged decode.
//
// With ragged contexts a grid of one workgroup per (sequence, kv head,
// partition) leaves the longest sequences running alone at the end. Here a
// fixed number of waves W split the flattened space of 16-token steps
//   (sequence, kv head, query-head chunk, step)    -- one "segment" per
// (sequence, kv head, chunk), N steps in total
// evenly: wave w takes steps [w*N/W, (w+1)*N/W), crossing segment borders
// (or in one even piece per dispatch slot at several workgroups per compute
// unit: StreamSplit)
// (W is capped at N, so no wave is idle and a segment's partials come from
// consecutive waves).
// Each wave keeps a ring of steps of loads in flight and, for every segment it
// touches, writes one partial (normalised context, row max, row sum) to the
// workspace; stream_reduce merges the partials of each
// (sequence, query head) with the log-sum-exp rule of the reference's
// partial-softmax merge (src/core/resident_kv_store.py:2497-2509).
//
// A run start (Q loads, ring refill) costs about one memory latency, so the
// split charges every non-empty segment `stream_run_cost` phantom steps in
// front of its real ones: a wave that starts more segments gets fewer real
// steps. Segment i covers the flattened range [seg_prefix[i],
// seg_prefix[i+1]), its real steps start stream_run_cost later.
//
// Head groups: the unit of the split is a group of head_group waves of one
// workgroup (one SIMD each), which take the same steps of head_group
// consecutive kv heads, one kv head per wave. The waves of a group then read
// the rows of a token for all their kv heads at about the same time, as one
// contiguous range of the block (a whole 16-token block of the GQA-7B pools
// for head_group 4), which HBM serves faster than the same rows read at
// unrelated times. A "segment" is then (sequence, kv-head group, chunk).
//
// Every workgroup derives the segment prefix sums itself (in LDS) from
// context_lens; workgroup 0 also stores them for the reduce kernel.
#include "decode_mfma.h"

namespace clv {
namespace {

constexpr int kWaves = 4;  // independent waves per workgroup
constexpr int kThreads = kWaves * 64;

// The split of N steps over W groups (N >= W). Even: group w starts at
// floor(w*N/W). By dispatch slot (slot_count = S > 1, slot_groups = Gp):
// the groups form pieces of Gp consecutive groups (piece k: groups
// [k*Gp, (k+1)*Gp), the last piece those left below W), each piece's steps
// split evenly over its groups, and piece k's share of the N steps in
// proportion to its groups times its weight slot_q8[k], every piece held to
// at least one step per group.
//
// Why: at S workgroups (of four waves) per compute unit, the workgroups
// [0, CUs) are dispatched first, one per CU, then [CUs, 2*CUs) into the
// second slot, and so on, so each SIMD runs one wave of each slot. The
// SIMD's issue arbiter favours older waves: with equal spans the slots end
// in dispatch order on every SIMD (fp8 GQA-7B batch, 2048 waves: the second
// slot 5.3 us after the first on average; 3072 waves: 71.6, 78.8 and
// 86.4 us for the three slots), and the youngest waves run their last steps
// alone, at the lower rate of one wave per SIMD. Giving the older slots
// more steps lets every slot end together.
struct StreamSplit {
  static constexpr int kMaxSlots = 4;
  int64_t W, N, Gp;
  int S;
  int64_t b1, b2, b3;  // first steps of pieces 1..3 (N past the last piece)
  // Every product in start() and owner() is a group count (<= W) times a
  // step count (<= N). When W * N fits 32 bits they run in 32-bit unsigned
  // arithmetic, with the same results: a 64-bit division is a long
  // instruction sequence on the GPU, and these sit on every wave's way to
  // its first load and on the merge's way to its partials.
  bool narrow;
  __host__ __device__ StreamSplit(const DecodeParams &p, int64_t W_, int64_t N_)
      : W(W_), N(N_), Gp(p.slot_groups), S(1), b1(N_), b2(N_), b3(N_),
        narrow((uint64_t)W_ * (uint64_t)N_ <= 0xffffffffull) {
    if (p.slot_count > 1 && Gp > 0 && Gp < W) {
      S = (int)min((int64_t)min(p.slot_count, kMaxSlots), (W + Gp - 1) / Gp);
      const int64_t w0 = groups(0) * p.slot_q8[0], w1 = groups(1) * p.slot_q8[1];
      const int64_t w2 = S > 2 ? groups(2) * p.slot_q8[2] : 0;
      const int64_t w3 = S > 3 ? groups(3) * p.slot_q8[3] : 0;
      const int64_t total = w0 + w1 + w2 + w3;
      // Piece k ends at its weighted share, held to at least one step per
      // group of this piece and of every later one.
      auto cut = [&](int k, int64_t acc, int64_t prev) {
        return min(max(N * acc / total, prev + groups(k)), N - (W - (int64_t)(k + 1) * Gp));
      };
      b1 = cut(0, w0, 0);
      if (S > 2) b2 = cut(1, w0 + w1, b1);
      if (S > 3) b3 = cut(2, w0 + w1 + w2, b2);
    }
  }
  // Groups of piece k.
  __host__ __device__ __forceinline__ int64_t groups(int k) const {
    return k + 1 < S ? Gp : W - (int64_t)k * Gp;
  }
  // First step of piece k (0 <= k <= S; N for k >= S).
  __host__ __device__ __forceinline__ int64_t base(int k) const {
    return k <= 0 ? 0 : k == 1 ? b1 : k == 2 ? b2 : k == 3 ? b3 : N;
  }
  // floor((a * b - sub) / c) for 0 <= a <= N, 0 <= b <= W (or the other
  // way round), sub in {0, 1} with a * b >= sub, c > 0.
  __host__ __device__ __forceinline__ int64_t muldiv(int64_t a, int64_t b, int sub,
                                                     int64_t c) const {
    if (narrow) return (int64_t)(((uint32_t)a * (uint32_t)b - (uint32_t)sub) / (uint32_t)c);
    return (a * b - sub) / c;
  }
  // First step of group w (w <= W; start(W) = N).
  __host__ __device__ __forceinline__ int start(int w) const {
    if (S == 1) return (int)muldiv(w, N, 0, W);
    if (w >= W) return (int)N;
    const int k = (int)min((int64_t)w / Gp, (int64_t)S - 1);
    const int64_t lo = base(k);
    return (int)(lo + muldiv(w - (int64_t)k * Gp, base(k + 1) - lo, 0, groups(k)));
  }
  // Group owning step x (0 <= x < N): the largest w with start(w) <= x.
  __host__ __device__ __forceinline__ int owner(int x) const {
    if (S == 1) return (int)muldiv(x + 1, W, 1, N);
    const int k = (S > 3 && b3 <= x) ? 3 : (S > 2 && b2 <= x) ? 2 : b1 <= x ? 1 : 0;
    const int64_t lo = base(k);
    return (int)((int64_t)k * Gp + muldiv(x - lo + 1, groups(k), 1, base(k + 1) - lo));
  }
};

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

// APPEND (K-transpose path only): fused append, see below.
// KV8 (K-transpose path only): fp8 pools, see DecodeWave.
// PART: split-K partials (partition_size > 0). The unit of the split is a
// partition of partition_size tokens instead of a 16-token step (no phantom
// run cost), so every partition lies in one group's span; a run streams its
// partitions through one ring and writes each partition's partial, in the
// split-K layout [sequence, query head, partition] that splitk_reduce
// merges, when the partition's last step is folded.
template <typename T, int D, bool UNI, int DEPTH, bool APPEND = false, bool KV8 = false,
          bool PART = false>
__global__ void __launch_bounds__(kThreads)
paged_decode_stream(const DecodeParams p, const int32_t *__restrict__ tables,
                    const int32_t *__restrict__ lens, float *__restrict__ ws_o,
                    float *__restrict__ ws_m, float *__restrict__ ws_l,
                    int32_t *__restrict__ seg_prefix) {
  // Every global pointer is a separate restrict argument: with stores to the
  // workspace inside the main loop, that is what lets the compiler keep the
  // wave-uniform block-table reads scalar loads.
  typedef typename StreamWave<T, D, UNI, KV8>::type WV;
  constexpr int CEB = KV8 ? 1 : (int)sizeof(T);
  typedef typename WV::qk_t qk_t;
  __shared__ __attribute__((aligned(16))) char s_kt[kWaves][WV::KT_BYTES];
  __shared__ int s_seg[kStreamMaxSegments + 1];
  __shared__ int s_tmp[kWaves];
  // PART: each wave stages its partitions' partials here and writes them to
  // the workspace when the buffer is full or its run ends. Stores issued
  // every partition stalled the load ring (the in-order memory counter holds
  // the next loads behind them, and every wave reaches a partition border on
  // the same step): 16 x 32K-token fp16, 355.6 us against 311.8 without them.
  // 8 partials of 4 rows fit (GQA 32/8 heads); 16 rows at most, so >= 2.
  constexpr int kPartBuf = PART ? 8 * 4 * (D + 2) + 64 : 4;
  static_assert(!PART || kPartBuf >= 2 * 16 * (D + 2), "two partials of 16 rows");
  __shared__ __attribute__((aligned(16))) float s_part[PART ? kWaves : 1][kPartBuf];

  const int nseg = p.num_segments;
  const int HG = p.head_group;
  const int per_seq = (p.num_kv_heads / HG) * p.n_gchunks;
  static_assert(!PART || (!APPEND && !KV8), "split-K partials over 16- or 32-bit pools");
  const int K = PART ? 0 : p.stream_run_cost;
  const int psteps = PART ? p.partition_size / WV::STEP : 1;  // steps per partition
  for (int i = threadIdx.x; i < nseg; i += kThreads) {
    const int steps = (clamp_ctx(p, i / per_seq) + WV::STEP - 1) / WV::STEP;  // vector read
    if constexpr (PART) s_seg[i] = (steps + psteps - 1) / psteps;
    else s_seg[i] = steps > 0 ? steps + K : 0;
  }
  __syncthreads();
  const int64_t N = block_exclusive_scan(s_seg, nseg, s_tmp);
  // At most one group per step, so that every group owns at least one step
  // and each segment's partials come from consecutive groups.
  const int64_t W = min((int64_t)(p.num_waves / HG), N);
  if (!PART && blockIdx.x == 0) {
    for (int i = threadIdx.x; i <= nseg; i += kThreads) seg_prefix[i] = s_seg[i];
  }

  const int wv = (int)blockIdx.x * kWaves + uni(threadIdx.x >> 6);
  const int wid = wv / HG;      // group
  const int wk = wv - wid * HG;  // kv head within the group
  if (N == 0 || wid >= W) return;
  const StreamSplit split(p, W, N);
  const int st = uni(split.start(wid));
  const int en = uni(split.start(wid + 1));
  if (st >= en) return;

  // Segment holding step st: the last one whose first step is <= st. The
  // first steps never decrease and s_seg[0] = 0 <= st, so those segments
  // are a prefix: each round the lanes test 64 evenly spaced candidates at
  // once and the highest passing lane narrows the range (two rounds cover
  // 4096 segments, against twelve dependent LDS reads of a binary search).
  int seg;
  {
    const int lane = threadIdx.x & 63;
    int lo = 0, n = nseg;  // the answer lies in [lo, lo + n); s_seg[lo] <= st
    while (n > 1) {
      const int stride = (n + 63) / 64;
      const bool le = lane * stride < n && s_seg[lo + lane * stride] <= st;
      const uint64_t m = __ballot(le);  // bit 0 is set (s_seg[lo] <= st)
      const int k = 63 - __builtin_clzll(m);
      lo += k * stride;
      n = min(stride, n - k * stride);
    }
    seg = uni(lo);
  }

  WV w;
  w.init(p);
  w.set_k_lds(s_kt[uni(threadIdx.x >> 6)]);

  if constexpr (APPEND) {
    // Fused append: the wave that holds a segment's last step writes the
    // sequence's new token (position ctx - 1) before its run loop. Only that
    // wave ever loads the row (one query-head chunk per kv head on this
    // path), with the lanes that wrote it (kt_store_row).
    static_assert(UNI && D == 128, "the fused append mirrors the K-transpose loads");
    for (int sg = seg; sg < nseg && uni(s_seg[sg + 1]) - 1 < en; ++sg) {
      const int lst = uni(s_seg[sg + 1]) - 1;
      if (lst < st || lst < uni(s_seg[sg]) + K) continue;  // not ours, or no real steps
      const int s_ = sg / per_seq;
      const int kvh = (sg - s_ * per_seq) * HG + wk;  // one query-head chunk per kv head
      const int ctx = clamp_ctx(p, lens, s_);
      if (ctx != scalar_load_i32(lens + s_)) continue;  // the new position is not attended
      const SegGeom geo = seg_geom<T>(p, s_, kvh, ctx, tables);
      const int pos = ctx - 1;
      const int blk = scalar_load_i32(geo.bt + (pos >> p.block_shift));
      if ((unsigned)blk >= (unsigned)p.num_blocks) continue;
      const int64_t row_off =
          ((int64_t)blk * p.kv_stride_block + (int64_t)(pos & ((1 << p.block_shift) - 1)) *
                                                  p.kv_stride_token) * (int64_t)sizeof(T);
      const int64_t src = (int64_t)s_ * p.new_stride_seq + (int64_t)kvh * p.new_stride_head;
      kt_store_row(geo.kbase, geo.vbase, row_off, pos,
                   (const uint16_t *)p.key_new + src, (const uint16_t *)p.value_new + src);
    }
    __builtin_amdgcn_s_waitcnt(0);      // the stores are done before any load is issued
    __asm__ volatile("" ::: "memory");  // and the compiler keeps them ahead of the loads
  }

  // The span is cut at segment borders into runs. Each run loads its Q rows,
  // keeps DEPTH steps of loads in flight (a ring of register sets refilled
  // right after each step is folded) and ends with one partial.
  int x = st;
  while (x < en) {
    while (uni(s_seg[seg + 1]) <= x) ++seg;  // skip empty segments
    const int firstU = uni(s_seg[seg]) + K;   // first real unit (step, or partition)
    const int lastU = min(en, uni(s_seg[seg + 1])) - 1;
    if (max(x, firstU) > lastU) {  // only phantom steps of this segment
      x = lastU + 1;
      continue;
    }
    const int s_ = seg / per_seq;
    const int rem = seg - s_ * per_seq;
    const int kvg = rem / p.n_gchunks;
    const int kvh = kvg * HG + wk;
    const int g0 = (rem - kvg * p.n_gchunks) * 16;
    const int ng = min(16, p.group - g0);
    const int ctx = clamp_ctx(p, lens, s_);
    // The run's steps [xs, last], `first` being the step of the segment's
    // first token: PART counts steps from that token (partitions
    // x..lastU are steps x * psteps ..), otherwise the units are the steps.
    int first, xs, last;
    if constexpr (PART) {
      first = 0;
      xs = (x - firstU) * psteps;
      last = min((lastU + 1 - firstU) * psteps, (ctx + WV::STEP - 1) / WV::STEP) - 1;
    } else {
      first = firstU;
      xs = max(x, firstU);
      last = lastU;
    }
    const SegGeom geo = seg_geom<T, CEB>(p, s_, kvh, ctx, tables);
    if constexpr (KV8) {  // the kv head's scales (wave-uniform, scalar loads)
      const float ks = __builtin_bit_cast(float, scalar_load_i32((const int32_t *)p.k_scales + kvh));
      const float vs = __builtin_bit_cast(float, scalar_load_i32((const int32_t *)p.v_scales + kvh));
      w.set_kv_scales(p.scale_log2 * ks, vs);
    }

    // Q loads go out first and are waited for only after the ring below is
    // issued, so a run start costs one memory latency, not two.
    u32x4 qraw[WV::NQK];
    w.load_q_raw(p, s_, kvh * p.group + g0, ng, qraw);

    // Ring of DEPTH register sets; past the run's last step it re-reads that
    // step (cache resident, never used).
    typename WV::Regs R[DEPTH];
    // UNI: block-table entries are read through the constant address space
    // (the kernel never writes the table), so the compiler issues them as
    // scalar loads it waits for only at use; each is read one issue ahead.
    typedef const int32_t __attribute__((address_space(4))) *cint_t;
    const cint_t brow = (cint_t)(tables + (int64_t)s_ * p.max_blocks_per_seq);
    auto base_of = [&](int step) { return (min(step, last) - first) * WV::STEP; };
    int blk = 0;
    if constexpr (UNI) blk = brow[base_of(xs) >> p.block_shift];
    auto issue = [&](int step, typename WV::Regs &Rg) {
      if constexpr (UNI) {
        w.issue_blk(geo.kbase, geo.vbase, blk, base_of(step) & w.bmask, Rg);
        blk = brow[base_of(step + 1) >> p.block_shift];
      } else {
        w.issue(geo, base_of(step), Rg);
      }
    };
#pragma unroll
    for (int i = 0; i < DEPTH; ++i) issue(xs + i, R[i]);
    qk_t q[WV::NQK];
    w.mask_q(qraw, ng, q);
    int c = xs;
    bool done = false;
    // PART: steps left in the current partition, and its index; the staged
    // partials of partitions pfirst .. pfirst + pcount - 1 (rows of ng query
    // heads: contexts, then row maxima, then row sums).
    int pleft = psteps, part = PART ? xs / psteps : 0;
    int pfirst = part, pcount = 0;
    const int pcap = PART ? kPartBuf / (ng * (D + 2)) : 1;
    float *sp_o = s_part[PART ? uni(threadIdx.x >> 6) : 0];
    float *sp_m = sp_o + pcap * ng * D;
    float *sp_l = sp_m + pcap * ng;
    const int64_t hrow0 = (int64_t)s_ * p.num_heads + kvh * p.group + g0;
    auto flush_staged = [&]() {
      const int lane = threadIdx.x & 63;
      constexpr int C4 = D / 4;  // float4 chunks per row
      for (int idx = lane; idx < pcount * ng * C4; idx += 64) {
        const int kg = idx / C4, c4 = idx - kg * C4;
        const int k = kg / ng, g = kg - k * ng;
        const int64_t row = (hrow0 + g) * p.max_parts + pfirst + k;
        store_vec<f32x4>(ws_o + row * D + 4 * c4, load_vec<f32x4>(sp_o + kg * D + 4 * c4));
      }
      for (int idx = lane; idx < pcount * ng; idx += 64) {
        const int k = idx / ng, g = idx - k * ng;
        const int64_t row = (hrow0 + g) * p.max_parts + pfirst + k;
        ws_m[row] = sp_m[idx];
        ws_l[row] = sp_l[idx];
      }
    };
    while (!done) {
#pragma unroll
      for (int i = 0; i < DEPTH; ++i) {
        if (!done) {
          w.compute((c - first) * WV::STEP, ctx, R[i], q);
          if (++c > last)
            done = true;
          else
            issue(c + DEPTH - 1, R[i]);
          if constexpr (PART) {
            if (--pleft == 0 || done) {  // the partition's last step: stage its partial
              w.reduce_rowsum();
              w.store_partial(sp_o, sp_m, sp_l, (int64_t)pcount * ng, ng);
              w.reset();
              pleft = psteps;
              ++part;
              if (++pcount == pcap || done) {
                flush_staged();
                pfirst = part;
                pcount = 0;
              }
            }
          }
        }
      }
    }
    if constexpr (PART) {
      x = lastU + 1;
      continue;
    }

    w.reduce_rowsum();
    // Partial slot of the (segment, group) pair: seg + wid. Along the
    // flattened steps every change of segment or group raises seg + wid, so
    // the slots are distinct and below num_waves / HG + nseg; each holds HG
    // partials of 16 rows (one per kv head of the group). The merge finds a
    // segment's partials at slot seg + (its first group) onwards.
    const int64_t row0 = (((int64_t)seg + wid) * HG + wk) * 16;
    w.store_partial(ws_o, ws_m, ws_l, row0, ng);
    w.reset();
    x = last + 1;
  }
}

// One wave per (sequence, query head).
// NEW: the partials cover context_lens[s] tokens and the merge takes
// sequence s's new token as one more row: score q[s, h] . key_new[s, kvh]
// in the scale of the partials (fp32 products of the 16-bit values, as the
// score MFMAs form them), sum 1, context value_new[s, kvh]. The wave of the
// kv head's first query head also writes the token's key and value rows at
// slot_mapping[s] (skipped when negative or past the pools), for the decode
// steps after this one.
template <typename T, int D, bool NEW = false>
__global__ void __launch_bounds__(256) stream_reduce(const DecodeParams p) {
  constexpr int EPL = (D + 63) / 64;
  const int64_t idx = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (idx >= (int64_t)p.num_seqs * p.num_heads) return;
  const int s = (int)(idx / p.num_heads);
  const int h = (int)(idx - (int64_t)s * p.num_heads);
  const int kvh = h / p.group;
  const int gall = h - kvh * p.group;
  // NEW: the new token's rows and slot are loaded first; they do not depend
  // on the partials' layout, so their latency overlaps the lookups below.
  const int lane = threadIdx.x & 63;
  T qx[EPL], kx[EPL], vx[EPL];
  int64_t slot = -1;
  if constexpr (NEW) {
    const T *qr = (const T *)p.q + (int64_t)s * p.q_stride_seq + (int64_t)h * p.q_stride_head;
    const int64_t nrow = (int64_t)s * p.new_stride_seq + (int64_t)kvh * p.new_stride_head;
    const T *kr = (const T *)p.key_new + nrow;
    const T *vr = (const T *)p.value_new + nrow;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const int d = lane + 64 * e;
      if (d < D) {
        qx[e] = qr[d];
        kx[e] = kr[d];
        vx[e] = vr[d];
      }
    }
    if (gall == 0) slot = p.slot_mapping[s];
  }
  const int HG = p.head_group;
  const int kvg = kvh / HG, wk = kvh - kvg * HG;
  const int seg = (s * (p.num_kv_heads / HG) + kvg) * p.n_gchunks + gall / 16;
  const int g = gall % 16;
  // The segment bounds and the step total are wave-uniform and read-only
  // here: three scalar loads issued together, one wait (the split's
  // arithmetic then runs on the scalar unit).
  int a, b, n_total;
  {
    const int32_t *ps = p.seg_prefix + __builtin_amdgcn_readfirstlane(seg);
    const int32_t *pn = p.seg_prefix + p.num_segments;
    uint64_t ab;
    // Early-clobber outputs: the first load's destination is written when its
    // data returns, so it must not share registers with the second's address.
    asm volatile("s_load_dwordx2 %0, %2, 0x0\n\ts_load_dword %1, %3, 0x0\n\ts_waitcnt lgkmcnt(0)"
                 : "=&s"(ab), "=&s"(n_total) : "s"(ps), "s"(pn) : "memory");
    a = (int)(uint32_t)ab + p.stream_run_cost;
    b = (int)(uint32_t)(ab >> 32);
  }
  const int64_t N = n_total;
  const int64_t W = min((int64_t)(p.num_waves / HG), N);
  int n = 0, w0 = 0;
  if (b > a) {
    const StreamSplit split(p, W, N);
    w0 = split.owner(a);
    n = split.owner(b - 1) - w0 + 1;
  }
  const int64_t row0 = (n > 0 ? (((int64_t)seg + w0) * HG + wk) * 16 : 0) + g;
  T *dst = (T *)p.out + (int64_t)s * p.out_stride_seq + (int64_t)h * p.out_stride_head;
  if constexpr (!NEW) {
    lse_merge<T, D, 1>(p.ws_m + row0, p.ws_l + row0, p.ws_o + row0 * D, 16 * HG, 16 * HG * D, n,
                       dst, nullptr);
  } else {
    // The new token as one more row: its score q . key_new in the scale of
    // the partials (log2-domain scores times ln 2), fp32 products of the
    // 16-bit values as the score MFMAs form them, sum 1, context value_new.
    float xdot = 0.f, xv[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const bool in = lane + 64 * e < D;
      xdot += in ? to_f32(qx[e]) * to_f32(kx[e]) : 0.f;
      xv[e] = in ? to_f32(vx[e]) : 0.f;
    }
    lse_merge<T, D, 1, true>(p.ws_m + row0, p.ws_l + row0, p.ws_o + row0 * D, 16 * HG,
                             16 * HG * D, n, dst, nullptr, xdot, p.scale_log2 * kLn2, xv);
    // The kv head's first query head writes the token's rows at its slot,
    // for the decode steps after this one (after the merge: no load of this
    // kernel waits behind these stores).
    if (gall == 0 && slot >= 0 && slot < ((int64_t)p.num_blocks << p.block_shift)) {
      const int64_t o = (slot >> p.block_shift) * p.kv_stride_block +
                        (slot & ((1 << p.block_shift) - 1)) * p.kv_stride_token +
                        (int64_t)kvh * p.kv_stride_head;
      T *kd = (T *)p.k_cache + o;
      T *vd = (T *)p.v_cache + o;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const int d = lane + 64 * e;
        if (d < D) {
          kd[d] = kx[e];
          vd[d] = vx[e];
        }
      }
    }
  }
}

template <typename T, int D, int DEPTH>
hipError_t launch_stream_tdd(const DecodeParams &p, hipStream_t stream) {
  const dim3 grid((unsigned)((p.num_waves + kWaves - 1) / kWaves));
  if (p.partition_size > 0) {  // split-K partials (no fused append, no fp8 pools)
    if (p.kv_fp8 || p.append_new || p.partition_size % 32 != 0) return hipErrorInvalidValue;
    if (p.block_shift >= 4)
      hipLaunchKernelGGL((paged_decode_stream<T, D, true, DEPTH, false, false, true>), grid,
                         dim3(kThreads), 0, stream, p, p.block_tables, p.context_lens, p.ws_o,
                         p.ws_m, p.ws_l, p.seg_prefix);
    else
      hipLaunchKernelGGL((paged_decode_stream<T, D, false, DEPTH, false, false, true>), grid,
                         dim3(kThreads), 0, stream, p, p.block_tables, p.context_lens, p.ws_o,
                         p.ws_m, p.ws_l, p.seg_prefix);
    return hipGetLastError();
  }
  if constexpr (D == 128 && sizeof(T) == 2) {
    if (p.kv_fp8) {  // validated: block_size >= 16, no fused append
      if (p.block_shift < 4 || p.append_new) return hipErrorInvalidValue;
      hipLaunchKernelGGL((paged_decode_stream<T, D, true, DEPTH, false, true>), grid, dim3(kThreads),
                         0, stream, p, p.block_tables, p.context_lens, p.ws_o, p.ws_m, p.ws_l,
                         p.seg_prefix);
      return hipGetLastError();
    }
    if (p.append_new) {  // set only where stream_appends_in_kernel holds
      if (p.block_shift < 4) return hipErrorInvalidValue;
      hipLaunchKernelGGL((paged_decode_stream<T, D, true, DEPTH, true>), grid, dim3(kThreads), 0,
                         stream, p, p.block_tables, p.context_lens, p.ws_o, p.ws_m, p.ws_l,
                         p.seg_prefix);
      return hipGetLastError();
    }
  }
  if (p.block_shift >= 4)
    hipLaunchKernelGGL((paged_decode_stream<T, D, true, DEPTH>), grid, dim3(kThreads), 0, stream,
                       p, p.block_tables, p.context_lens, p.ws_o, p.ws_m, p.ws_l, p.seg_prefix);
  else
    hipLaunchKernelGGL((paged_decode_stream<T, D, false, DEPTH>), grid, dim3(kThreads), 0, stream,
                       p, p.block_tables, p.context_lens, p.ws_o, p.ws_m, p.ws_l, p.seg_prefix);
  return hipGetLastError();
}

template <typename T, int D>
hipError_t launch_stream_td(const DecodeParams &p, hipStream_t stream) {
  switch (p.stream_depth) {
    case 2: return launch_stream_tdd<T, D, 2>(p, stream);
    case 6: return launch_stream_tdd<T, D, 6>(p, stream);
    case 3: return launch_stream_tdd<T, D, 3>(p, stream);
    default: return launch_stream_tdd<T, D, 4>(p, stream);
  }
}

template <typename T>
hipError_t launch_stream_t(const DecodeParams &p, hipStream_t stream) {
  if (p.head_dim == 128) return launch_stream_td<T, 128>(p, stream);
  if (p.head_dim == 64) return launch_stream_td<T, 64>(p, stream);
  return hipErrorInvalidValue;
}

template <typename T, bool NEW = false>
hipError_t launch_sreduce_t(const DecodeParams &p, hipStream_t stream) {
  const int64_t rows = (int64_t)p.num_seqs * p.num_heads;
  const dim3 grid((unsigned)((rows + 3) / 4));
  if (p.head_dim == 128)
    hipLaunchKernelGGL((stream_reduce<T, 128, NEW>), grid, dim3(256), 0, stream, p);
  else if (p.head_dim == 64)
    hipLaunchKernelGGL((stream_reduce<T, 64, NEW>), grid, dim3(256), 0, stream, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace

bool decode_stream_supported(DType dt, int head_dim, int block_size, int64_t num_segments) {
  return decode_mfma_supported(dt, head_dim, block_size) && num_segments <= kStreamMaxSegments;
}

bool stream_appends_in_kernel(DType dt, int head_dim, int block_size, int group) {
  // The 16-bit K-transpose path (a 16-token step inside one block, head_dim
  // 128) with one query-head chunk per kv head.
  return (dt == DType::F16 || dt == DType::BF16) && head_dim == 128 && block_size >= 16 &&
         group <= 16;
}

hipError_t launch_decode_stream(const DecodeParams &p, DType dt, hipStream_t stream) {
  if (dt == DType::BF16) return launch_stream_t<__bf16>(p, stream);
  if (dt == DType::F16) return launch_stream_t<_Float16>(p, stream);
  if (dt == DType::F32 && !p.kv_fp8 && !p.append_new) return launch_stream_t<float>(p, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_stream_reduce(const DecodeParams &p, DType dt, hipStream_t stream) {
  if (dt == DType::BF16) return launch_sreduce_t<__bf16>(p, stream);
  if (dt == DType::F16) return launch_sreduce_t<_Float16>(p, stream);
  if (dt == DType::F32) return launch_sreduce_t<float>(p, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_stream_reduce_append(const DecodeParams &p, DType dt, hipStream_t stream) {
  if (p.kv_fp8) return hipErrorInvalidValue;
  if (dt == DType::BF16) return launch_sreduce_t<__bf16, true>(p, stream);
  if (dt == DType::F16) return launch_sreduce_t<_Float16, true>(p, stream);
  if (dt == DType::F32) return launch_sreduce_t<float, true>(p, stream);
  return hipErrorInvalidValue;
}

}  // namespace clv
