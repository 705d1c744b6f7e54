// prefill_mfma.hip - chunked prefill over paged KV with MFMA (fp16/bf16).
//
// Semantics as in prefill.hip: query row i of sequence s sees cached
// positions p <= context_lens[s] - n_s + i.
//
// Work decomposition: one workgroup (8 waves, two per SIMD) per (sequence,
// kv head, query tile). A query tile holds up to 256 rows = bq tokens x G
// query heads of the kv head (row r is token r / G, head r % G), so every K/V
// tile staged in LDS serves all query heads of the group. Each wave owns 32
// rows (two 16-row MFMA tiles) and fits in 256 VGPRs, so two waves share a
// SIMD and one's softmax overlaps the other's MFMAs. Per 64-token K/V tile a
// wave runs
//   S^T[t, r] = K[t, :] . Q[r, :]   4 token tiles x 2 row tiles x D/32 MFMAs
//   O[r, d]  += P[r, t] V[t, d]     2 token halves x 2 row tiles x D/16 MFMAs
// (v_mfma_f32_16x16x32), with an fp32 online softmax between. The C layout
// of the first product (lane holds row n16, tokens 4j..4j+3 of each 16-token
// tile) is the A layout of the second, so P never leaves registers; V's B
// operand comes straight from LDS with transposing reads (ds_read_b64_tr_b16),
// so MFMA m produces output columns d = 16m + n16.
//
// P.V runs in fp16 for both input types. P is in [0, 2^8] (see the lazy
// rescale below), where fp16 keeps 11 significant bits. bf16 V is converted
// to fp16 once, when a tile is staged into LDS; that is exact for every bf16
// value of magnitude below 2^16 (fp16 subnormals lose at most 2^-25 in
// absolute terms). If any tile of a workgroup holds a larger (or infinite)
// bf16 value, the workgroup recomputes its rows with an exact pass that keeps
// V in bf16 and splits P into a bf16 value and its bf16 rounding residual
// (two MFMAs, fp32-level accuracy). The exact pass is a separate loop, so it
// costs the fast loop no registers.
//
// Online softmax: scores stay raw (scale folded into the exponent with one
// fma), the running row maximum is only raised when a tile's maximum exceeds
// it by more than 8 (log2 units), so the accumulator is rarely rescaled and
// P stays below 2^8. Tiles fully below every row's causal limit, with all
// block-table entries valid, skip the per-element masks.
//
// Inside each MFMA phase the LDS operand reads run ahead of the MFMAs that
// use them (K: one k-step ahead; V: three output blocks ahead), held in that
// order by scheduling barriers; left alone, the compiler issues them just
// before their MFMAs and the wave waits out the LDS latency at every pair.
//
// K/V tiles go through a three-stage LDS ring: the global loads of tile k+1
// are in flight while tile k is computed, and the P.V of the last half-step
// of tile k - 1 still reads its V; block-table entries are fetched one tile
// earlier still. Workgroup ids are remapped so that all query tiles of one
// (sequence, kv head) run on the same XCD and share its L2.
#include "attn_common.h"

#include <type_traits>

namespace clv {
namespace {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kRT = 2;                  // 16-row MFMA tiles per wave
constexpr int kWaveRows = kRT * 16;     // query rows per wave
constexpr int kRows = kWaves * kWaveRows; // query rows per workgroup
constexpr int kBK = 64;                 // K/V tokens per tile
constexpr float kRescaleLog2 = 8.f;     // lazy-rescale threshold (log2 units)

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element
// i % 4 of the 8 bytes read by lane 4k + i / 4 as its element k (k = 0..3)
// (measured on gfx950). So when lanes 4k..4k+3 of a group read columns
// c0 + 4(i % 4) .. +3 of one row t_k, lane i gets column c0 + i of rows
// t_0..t_3: four K-consecutive elements of an MFMA B operand. Two such reads
// (rows of k-slots 0..3 and 4..7) make the lane's 8-element operand.
// The reads take 32-bit LDS byte addresses: `lo` and `hi` are a common base
// plus constants, which the instruction's offset field absorbs.
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
__device__ __forceinline__ u32x4 vt_read(uint32_t lo, uint32_t hi) {
  const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(size_t)lo);
  const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(size_t)hi);
  const u32x2 ua = __builtin_bit_cast(u32x2, a), ub = __builtin_bit_cast(u32x2, b);
  return (u32x4){ua[0], ua[1], ub[0], ub[1]};
}

// Two bf16 values (one 32-bit word) as two fp16 values (round to nearest
// even; a magnitude of 65520 or more becomes an fp16 infinity).
__device__ __forceinline__ uint32_t bf16x2_to_f16x2(uint32_t w) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
  const float a = __builtin_bit_cast(float, w << 16);
  const float b = __builtin_bit_cast(float, w & 0xffff0000u);
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2));
}

// Work item of dispatch position i within one XCD. A workgroup holds most of
// a compute unit's LDS, so the XCD's workgroups run in rounds of one per CU
// (`cus` of them), in dispatch order. The items of one (sequence, kv head)
// are its n_q query tiles, consecutive and heaviest first (a later tile
// attends to more keys). The first round takes the items in that natural
// order: the query tiles of one kv head run side by side and share their K/V
// reads in the XCD's L2. Each later round holds the same items as in the
// natural order but dispatches them by weight, heaviest tile of every kv head
// first, so that the CUs that finish first (those given the lightest tiles)
// take the heaviest ones. Of the XCD's per_xcd positions, `valid` hold items;
// when a round does not hold whole kv heads the natural order is kept.
__host__ __device__ inline int dispatch_slot(int i, int per_xcd, int valid, int n_q, int cus) {
  if (valid > per_xcd) valid = per_xcd;
  if (cus <= 0 || n_q <= 1 || cus % n_q != 0 || per_xcd % n_q != 0 || i < cus || i >= valid)
    return i;
  const int r0 = i / cus * cus;
  const int len = valid - r0 < cus ? valid - r0 : cus;
  if (len % n_q != 0) return i;
  const int heads = len / n_q;
  const int u = i - r0;
  return r0 + (u % heads) * n_q + u / heads;
}

template <typename T, int D>
__global__ void __launch_bounds__(kThreads)
chunked_prefill_mfma(const PrefillParams p, int bq, int n_qtiles, int total) {
  typedef Mfma16x16x32<T> MfQK;
  typedef Mfma16x16x32<_Float16> MfPV;
  typedef typename MfQK::op_t qk_t;
  typedef typename MfPV::op_t pv_t;
  constexpr bool kBf16 = sizeof(T) == 2 && !__is_same(T, _Float16);
  constexpr int NQK = D / 32;             // QK k-steps
  constexpr int CH = D / 16;              // PV MFMAs per (half, row tile)
  // LDS row strides (elements), measured on gfx950: the K reads
  // (ds_read_b128, lane row = lane % 16) are conflict-free at a stride of
  // 32 mod 64 bytes; the transposed V reads (four rows per 16-lane group)
  // need a stride that is not a multiple of 64 bytes.
  constexpr int KROW = D + 16;
  constexpr int VROW = D + 16;
  constexpr int CPR = D * 2 / 16;         // 16-byte chunks per row
  constexpr int RPP = kThreads / CPR;     // rows per load pass
  constexpr int PASSES = kBK / RPP;       // load passes per tile

  __shared__ __attribute__((aligned(16))) T sK[3][kBK * KROW];
  // V rows: fp16 in the fast pass, T in the exact pass.
  __shared__ __attribute__((aligned(16))) uint16_t sV[3][kBK * VROW];
  __shared__ __attribute__((aligned(4))) uint8_t sValid[3][kBK];  // 1 = the token's block is readable
  __shared__ int sOvf;  // set when a bf16 V value did not fit fp16

  // XCD-aware remap: consecutive ids go round-robin over the 8 XCDs; give
  // each XCD a contiguous range of logical work items, in the order
  // dispatch_slot sets.
  const int per_xcd = gridDim.x / 8;
  const int xcd0 = (blockIdx.x % 8) * per_xcd;
  const int L = xcd0 + dispatch_slot(blockIdx.x / 8, per_xcd, total - xcd0, n_qtiles,
                                     p.cus_per_xcd);
  if (L >= total) return;
  const int qt = n_qtiles - 1 - L % n_qtiles;  // longest query tiles first
  const int rest = L / n_qtiles;
  const int kvh = rest % p.num_kv_heads;
  const int s = rest / p.num_kv_heads;

  const int qs = p.query_start_loc[s];
  const int n_new = p.query_start_loc[s + 1] - qs;
  const int q0 = qt * bq;
  if (q0 >= n_new) return;
  const int cap = p.max_blocks_per_seq << p.block_shift;
  const int ctx = max(0, min(p.context_lens[s], cap));
  const int base_pos = ctx - n_new;  // cached position of query 0
  const int q_hi = min(q0 + bq, n_new);
  const int kv_end = max(0, min(ctx, base_pos + q_hi));
  const int ntiles = (kv_end + kBK - 1) / kBK;
  const int G = p.group;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n16 = lane & 15;
  const int j = lane >> 4;

  KvView kv;
  kv.bt = p.block_tables + (int64_t)s * p.max_blocks_per_seq;
  kv.kbase = (const char *)p.k_cache + (int64_t)kvh * p.kv_stride_head * (int64_t)sizeof(T);
  kv.vbase = (const char *)p.v_cache + (int64_t)kvh * p.kv_stride_head * (int64_t)sizeof(T);
  kv.sblk = p.kv_stride_block * (int64_t)sizeof(T);
  kv.stok = p.kv_stride_token * (int64_t)sizeof(T);
  kv.block_shift = p.block_shift;
  kv.num_blocks = (unsigned)p.num_blocks;

  // A negative scale is applied as a sign flip of Q, so that the softmax
  // below only ever multiplies by c > 0. A zero scale becomes 2^-126: every
  // weight is then 1 to far below fp32 resolution, and masked scores (-inf)
  // still weigh exactly 0.
  const float c = fmaxf(fabsf(p.scale_log2), 0x1p-126f);
  const uint32_t qflip = p.scale_log2 < 0.f ? 0x80008000u : 0u;

  // Q (B operand of S^T = K Q^T) for this lane's rows kWaveRows*w + 16rt + n16.
  u32x4 qop[kRT][NQK];  // kept as raw words: bit-cast to the operand type at each MFMA
  int lim[kRT];  // last visible position of the lane's softmax row (-1: no row)
#pragma unroll
  for (int rt = 0; rt < kRT; ++rt) {
    const int r = kWaveRows * wave + 16 * rt + n16;
    const int tok = q0 + r / G;
    const bool ok = r < bq * G && tok < n_new;
    lim[rt] = ok ? base_pos + tok : -1;
    const T *qrow = (const T *)p.q + (int64_t)(qs + (ok ? tok : q0)) * p.q_stride_token +
                    (int64_t)(kvh * G + r % G) * p.q_stride_head;
#pragma unroll
    for (int i = 0; i < NQK; ++i) {
      u32x4 w = load_vec<u32x4>(qrow + 32 * i + 8 * j);
      w ^= qflip;
      if (!ok) w = (u32x4){0u, 0u, 0u, 0u};
      qop[rt][i] = w;
    }
  }
  // Smallest causal limit over the wave's real rows (rows are ordered by
  // token): tiles ending at or below it need no causal mask.
  const int wave_row0 = kWaveRows * wave;
  const int wave_lim = (wave_row0 < bq * G && q0 + wave_row0 / G < n_new)
                           ? base_pos + q0 + wave_row0 / G : -1;

  // Tile loader: thread handles chunk (tid % CPR) of rows tid / CPR + RPP*i.
  // One load instruction of a wave covers WROWS consecutive rows, which lie
  // in one block (the launcher requires block_size >= WROWS): the block id is
  // read with a scalar load through the constant address space (the kernel
  // never writes the table) and the row address is a scalar base plus a
  // per-lane constant 32-bit offset.
  constexpr int WROWS = 64 / CPR;
  const int lchunk = tid % CPR;
  const int lrow = tid / CPR;
  const int wrow = WROWS * wave;  // first row of the wave's load instructions
  // Byte strides as 32-bit values (the launcher checks that a block's rows
  // fit in 2^31 bytes, so 0x80000000 is past every block's range).
  const uint32_t sblk32 = (uint32_t)kv.sblk, stok32 = (uint32_t)kv.stok;
  const uint32_t bmask = (1u << kv.block_shift) - 1u;
  const uint32_t lane_off = (uint32_t)(lrow - wrow) * stok32 + (uint32_t)lchunk * 16u;
  typedef const int32_t __attribute__((address_space(4))) *cint_t;
  const cint_t brow = (cint_t)kv.bt;
  u32x4 kreg[PASSES], vreg[PASSES];
  bool rvalid[PASSES];  // the loaded rows are readable tokens
  int rblk[PASSES];     // block of the wave's rows of the tile to load next (-1: none)
  // Block-table entries are fetched one tile before their rows are loaded.
  auto fetch_blocks = [&](int tile) {
#pragma unroll
    for (int i = 0; i < PASSES; ++i) {
      const int t0 = tile * kBK + wrow + RPP * i;
      rblk[i] = (tile < ntiles && t0 < kv_end) ? brow[t0 >> kv.block_shift] : -1;
    }
  };
  // Rows are read through a buffer resource whose range is the rows of one
  // block: a lane whose token is not readable (past the context, or in an
  // unmapped block, which gets an empty range) reads zeros from the hardware
  // range check, so there are no per-lane branches and no zero fills.
  auto load_tile = [&](int tile) {
#pragma unroll
    for (int i = 0; i < PASSES; ++i) {
      const uint32_t t0 = (uint32_t)(tile * kBK + wrow + RPP * i);
      const bool bok = (unsigned)rblk[i] < kv.num_blocks;
      const bool ok = bok && (int)t0 + (lrow - wrow) < kv_end;
      rvalid[i] = ok;
      const uint64_t boff = (uint64_t)(uint32_t)(bok ? rblk[i] : 0) * sblk32;
      const int nrec = bok ? (int)(stok32 << kv.block_shift) : 0;
      const uint32_t voff = ok ? (t0 & bmask) * stok32 + lane_off : 0x80000000u;
      kreg[i] = buf_load<u32x4>(make_rsrc_range(kv.kbase + boff, nrec), voff);
      vreg[i] = buf_load<u32x4>(make_rsrc_range(kv.vbase + boff, nrec), voff);
    }
  };
  // Stage the loaded rows into LDS buffer buf. The fast pass stores V as
  // fp16; the exact pass stores V as is.
  auto store_tile = [&](int buf, auto exact_c) {
    constexpr bool EXACT = decltype(exact_c)::value;
#pragma unroll
    for (int i = 0; i < PASSES; ++i) {
      const int row = lrow + RPP * i;
      store_vec<u32x4>(&sK[buf][row * KROW + lchunk * 8], kreg[i]);
      u32x4 v = vreg[i];
      if constexpr (kBf16 && !EXACT) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = bf16x2_to_f16x2(v[e]);
      }
      store_vec<u32x4>(&sV[buf][row * VROW + lchunk * 8], v);
      if (lchunk == 0) sValid[buf][row] = rvalid[i] ? 1 : 0;
    }
  };

  f32x4 o[kRT][CH];
  float m_run[kRT];
  float thr[kRT];   // rescale threshold per row (see softmax)
  float msub[kRT];  // m_run * c (0 while m_run is -inf)
  // Row sums of P, accumulated by MFMA against an all-ones B operand (so in
  // the C layout of o: element e is row 4j + e), consistent with the
  // rounded P that P.V uses.
  f32x4 lsum[kRT];

  // One pass over the K/V tiles, software-pipelined per 32-token half-step
  // g (tile g / 2, half g % 2):
  //   M(g): scores of g (QK MFMAs), then P.V of g - 1 (PV MFMAs)
  //   V(g): online softmax of g (VALU), producing the P operand of g.
  // Waves 0-3 run M V M V per tile, waves 4-7 (the other wave of each
  // SIMD) run V M V M with their softmax one step behind, so that on every
  // SIMD one wave's softmax overlaps the other's MFMAs. P.V of g - 1 may read
  // the previous tile, hence three LDS stages. Returns whether a bf16 V value
  // did not fit fp16 (fast pass only).
  auto run_tiles = [&](auto exact_c) -> bool {
    constexpr bool EXACT = decltype(exact_c)::value;
    typedef Mfma16x16x32<__bf16> MfB;
    typedef typename std::conditional<EXACT, typename MfB::op_t, pv_t>::type p_t;
#pragma unroll
    for (int rt = 0; rt < kRT; ++rt) {
#pragma unroll
      for (int m = 0; m < CH; ++m) o[rt][m] = (f32x4){0.f, 0.f, 0.f, 0.f};
      m_run[rt] = kNegInf;
      thr[rt] = kNegInf;
      msub[rt] = 0.f;
      lsum[rt] = (f32x4){0.f, 0.f, 0.f, 0.f};
    }
    f32x4 sacc[2][kRT];     // scores of the step between M and V
    p_t pa[kRT], pl[kRT];   // P of the step between V and the next M (pl: exact pass)

    // Scores of step g: sacc[h][rt][e] = S'[row 16rt + n16][token 32(g%2) + 16h + 4j + e].
    auto qk = [&](int g) {
      const T *K = sK[(g >> 1) % 3];
      const int half = g & 1;
      // K operands of k-step i + 1 are read while the MFMAs of k-step i run
      // (the scheduling barriers keep the compiler from sinking the reads).
      auto kread = [&](int h, int i) {
        return load_vec<u32x4>(&K[(32 * half + 16 * h + n16) * KROW + 32 * i + 8 * j]);
      };
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int rt = 0; rt < kRT; ++rt) sacc[h][rt] = (f32x4){0.f, 0.f, 0.f, 0.f};
      u32x4 cur[2] = {kread(0, 0), kread(1, 0)};
#pragma unroll
      for (int i = 0; i < NQK; ++i) {
        u32x4 nxt[2];
        __builtin_amdgcn_sched_barrier(0);
        if (i + 1 < NQK) {
          nxt[0] = kread(0, i + 1);
          nxt[1] = kread(1, i + 1);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int rt = 0; rt < kRT; ++rt)
            sacc[h][rt] = MfQK::run(__builtin_bit_cast(qk_t, cur[h]),
                                    __builtin_bit_cast(qk_t, qop[rt][i]), sacc[h][rt]);
        if (i + 1 < NQK) {
          cur[0] = nxt[0];
          cur[1] = nxt[1];
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    // O += P V for step g. B operand of MFMA m (output columns 16m + n16):
    // lane (n16, j) needs V[token of k-slot 4h + kk][16m + n16], two
    // transposed LDS reads (h = 0, 1) of four tokens each (see vt_read).
    const p_t ones = __builtin_bit_cast(
        p_t, (u32x4){EXACT ? 0x3f803f80u : 0x3c003c00u, EXACT ? 0x3f803f80u : 0x3c003c00u,
                     EXACT ? 0x3f803f80u : 0x3c003c00u, EXACT ? 0x3f803f80u : 0x3c003c00u});
    auto pv = [&](int g) {
      const uint16_t *vrow = &sV[(g >> 1) % 3][(32 * (g & 1) + 4 * j + (n16 >> 2)) * VROW +
                                               4 * (n16 & 3)];
      // One base register per call, opaque to the compiler: left alone, it
      // kept one hoisted address per read and rebuilt each of them from the
      // ring slot with two VALU ops per read on every call.
      uint32_t vbase = (uint32_t)(size_t)(const __attribute__((address_space(3))) uint16_t *)vrow;
      asm volatile("" : "+v"(vbase));
      auto vread = [&](int m) {
        return vt_read(vbase + 32u * m, vbase + 32u * (VROW + m));  // rows +0 / +16
      };
      // V operands go out PVD blocks ahead of their MFMAs (a rolling window,
      // kept in order by the scheduling barriers).
      constexpr int PVD = 3;
      u32x4 vq[PVD];
#pragma unroll
      for (int m = 0; m < PVD; ++m) vq[m] = vread(m);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt) {
        if constexpr (!EXACT) {
          lsum[rt] = MfPV::run(pa[rt], ones, lsum[rt]);
        } else {
          lsum[rt] = MfB::run(pa[rt], ones, lsum[rt]);
          lsum[rt] = MfB::run(pl[rt], ones, lsum[rt]);
        }
      }
#pragma unroll
      for (int m = 0; m < CH; ++m) {
        const p_t vb = __builtin_bit_cast(p_t, vq[m % PVD]);
        __builtin_amdgcn_sched_barrier(0);
        if (m + PVD < CH) vq[m % PVD] = vread(m + PVD);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int rt = 0; rt < kRT; ++rt) {
          if constexpr (!EXACT) {
            o[rt][m] = MfPV::run(pa[rt], vb, o[rt][m]);
          } else {
            o[rt][m] = MfB::run(pa[rt], vb, o[rt][m]);
            o[rt][m] = MfB::run(pl[rt], vb, o[rt][m]);
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    // Scores of step g that a row may not see (unreadable block, past the
    // row's causal limit) become -inf: they drop out of the row max and, as
    // c > 0, weigh exp2(-inf) = 0. Only steps of tiles that are not full.
    auto mask_step = [&](int g) {
      const int buf = (g >> 1) % 3;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t vf =
            *reinterpret_cast<const uint32_t *>(&sValid[buf][32 * (g & 1) + 16 * h + 4 * j]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int pos = 32 * g + 16 * h + 4 * j + e;
          const bool readable = ((vf >> (8 * e)) & 0xffu) != 0;
#pragma unroll
          for (int rt = 0; rt < kRT; ++rt)
            if (!(readable && pos <= lim[rt])) sacc[h][rt][e] = kNegInf;
        }
      }
    };
    // Online softmax of step g. The running max is raised only when some
    // score exceeds it by more than 2^8 (log2 units), or it is still -inf.
    // Each lane tests its own eight scores of the row against the threshold
    // thr = m_run + 8 / c; the row maximum over the four lanes that hold the
    // row is only formed when some lane of the wave passes it.
    auto softmax = [&](int g, bool full) {
      if (!full) mask_step(g);
      float pf[kRT][8];
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt) {
        float mx = kNegInf;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int e = 0; e < 4; ++e) mx = fmaxf(mx, sacc[h][rt][e]);
        if (__any(mx > thr[rt])) {
          mx = fmaxf(mx, shfl_xor(mx, 16));
          mx = fmaxf(mx, shfl_xor(mx, 32));
          const float m_new = fmaxf(m_run[rt], mx);
          // 0 when the row had no visible token yet, 1 if its max is unchanged.
          const float alpha = m_new == kNegInf ? 1.f : fast_exp2((m_run[rt] - m_new) * c);
          m_run[rt] = m_new;
          // m_new + 8 / c is +inf when c is tiny (a zero scale): P is then 1
          // for every visible token and no rescale is ever needed again.
          thr[rt] = m_new == kNegInf ? kNegInf : m_new + kRescaleLog2 / c;
          msub[rt] = m_new == kNegInf ? 0.f : m_new * c;
          // Row 4j + e of o[rt][m] and lsum[rt] is element e.
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float a = shfl(alpha, 4 * j + e);
            lsum[rt][e] *= a;
#pragma unroll
            for (int m = 0; m < CH; ++m) o[rt][m][e] *= a;
          }
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            pf[rt][4 * h + e] = fast_exp2(__builtin_fmaf(sacc[h][rt][e], c, -msub[rt]));
      }
      // P's k-slot 4h + e is token 32(g%2) + 16h + 4j + e, as in pv().
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt) {
        if constexpr (!EXACT) {
          pa[rt] = pack8<_Float16>(pf[rt]);
        } else {
          // P split into its bf16 value and bf16 residual.
          float lo[8];
          pa[rt] = pack8<__bf16>(pf[rt]);
#pragma unroll
          for (int k = 0; k < 8; ++k) lo[k] = pf[rt][k] - (float)pa[rt][k];
          pl[rt] = pack8<__bf16>(lo);
        }
      }
    };
    auto softmax_step = [&](int g, bool full) { softmax(g, full); };
    auto tile_full = [&](int tile) {
      return __all(sValid[tile % 3][lane] != 0) && tile * kBK + kBK - 1 <= wave_lim;
    };

    // Cleared by the fast pass only: every wave reads the flag after the fast
    // pass's last barrier, so a clear at the start of the exact pass could
    // race a slower wave's read, and waves that disagreed on running the
    // exact pass would wait at different barriers.
    if (!EXACT && tid == 0) sOvf = 0;
    fetch_blocks(0);
    if (ntiles > 0) {
      load_tile(0);
      fetch_blocks(1);
      __syncthreads();  // sOvf cleared (and the previous pass done with LDS)
      store_tile(0, exact_c);
    }
    __syncthreads();

    const bool lag = wave >= kWaves / 2;  // softmax one step behind
    bool full_prev = false;
    for (int tile = 0; tile < ntiles; ++tile) {
      const bool more = tile + 1 < ntiles;
      if (more) load_tile(tile + 1);  // block ids fetched last iteration
      const bool full = tile_full(tile);
      const int g = 2 * tile;
      // The MFMA phases run at raised wave priority: the SIMD's arbiter then
      // issues the next MFMA as soon as the matrix core takes it, and the
      // other wave's softmax fills the issue slots in between.
      if (lag && tile > 0) softmax_step(g - 1, full_prev);
      __builtin_amdgcn_s_setprio(1);
      qk(g);
      if (tile > 0) pv(g - 1);
      __builtin_amdgcn_s_setprio(0);
      // Block-table entries for the tile after next, issued before a softmax
      // (VALU only on full tiles): the scalar loads share the LDS wait
      // counter, so issued right before an LDS read they would be waited for
      // there.
      if (more) fetch_blocks(tile + 2);
      softmax_step(g, full);
      __builtin_amdgcn_s_setprio(1);
      qk(g + 1);
      pv(g);
      __builtin_amdgcn_s_setprio(0);
      if (!lag) softmax_step(g + 1, full);
      full_prev = full;

      if (more) store_tile((tile + 1) % 3, exact_c);
      __syncthreads();
    }
    if (ntiles > 0) {
      if (lag) softmax_step(2 * ntiles - 1, full_prev);
      pv(2 * ntiles - 1);
    }
    if constexpr (kBf16 && !EXACT) {
      // A bf16 V value that did not fit fp16 became an infinity (or was
      // one, or a NaN): every P.V product of its half-step then made the
      // accumulators of all rows of every wave infinite or NaN (0 * inf
      // included), so a non-finite accumulator of any wave flags it.
      float acc = 0.f;
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt)
#pragma unroll
        for (int m = 0; m < CH; ++m)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc += o[rt][m][e] * 0.f;
      if (__any(acc != 0.f)) sOvf = 1;  // x * 0 is 0 for every finite x
    }
    __syncthreads();  // sOvf final; LDS free for a second pass
    return kBf16 && !EXACT && sOvf != 0;
  };

  const bool overflow = run_tiles(std::false_type{});
  if constexpr (kBf16) {
    if (overflow) run_tiles(std::true_type{});
  }

  // ---- normalise and store rows kWaveRows*w + 16rt + 4j + e
#pragma unroll
  for (int rt = 0; rt < kRT; ++rt) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float l = lsum[rt][e];
      const int row = kWaveRows * wave + 16 * rt + 4 * j + e;
      const int tok = q0 + row / G;
      if (row >= bq * G || tok >= n_new) continue;
      // A row at or past max_query_len (a caller error) is marked with NaN.
      const float inv = tok >= p.max_query_len ? __builtin_nanf("") : l > 0.f ? 1.f / l : 0.f;
      // Lane n16 of MFMA m holds column d = 16m + n16.
      T *dst = (T *)p.out + (int64_t)(qs + tok) * p.out_stride_token +
               (int64_t)(kvh * G + row % G) * p.out_stride_head + n16;
#pragma unroll
      for (int m = 0; m < CH; ++m) dst[16 * m] = (T)(o[rt][m][e] * inv);
    }
  }

  // Rows past the grid's query tiles (a chunk longer than max_query_len, a
  // caller error) are filled with NaN by the workgroup of the last tile, so
  // that the error shows in the output instead of stale memory.
  if (qt == n_qtiles - 1 && q_hi < n_new) {
    const T nan = (T)__builtin_nanf("");
    for (int idx = tid; idx < (n_new - q_hi) * G * D; idx += kThreads) {
      const int d = idx % D;
      const int h = (idx / D) % G;
      const int tok = q_hi + idx / (D * G);
      ((T *)p.out)[(int64_t)(qs + tok) * p.out_stride_token +
                   (int64_t)(kvh * G + h) * p.out_stride_head + d] = nan;
    }
  }
}

template <typename T>
hipError_t launch_t(const PrefillParams &p, hipStream_t stream) {
  const int bq = kRows / p.group;
  // At least one query tile per (sequence, kv head): its workgroup marks the
  // rows of chunks longer than max_query_len (see the kernel's end).
  const int n_qtiles = max(1, (p.max_query_len + bq - 1) / bq);
  const int64_t total = (int64_t)p.num_seqs * p.num_kv_heads * n_qtiles;
  if (total <= 0) return hipSuccess;
  if (total > (int64_t)1 << 30) return hipErrorInvalidValue;
  const unsigned grid = (unsigned)((total + 7) / 8 * 8);
  if (p.head_dim == 128)
    hipLaunchKernelGGL((chunked_prefill_mfma<T, 128>), dim3(grid), dim3(kThreads), 0, stream, p,
                       bq, n_qtiles, (int)total);
  else
    hipLaunchKernelGGL((chunked_prefill_mfma<T, 64>), dim3(grid), dim3(kThreads), 0, stream, p,
                       bq, n_qtiles, (int)total);
  return hipGetLastError();
}

}  // namespace

bool prefill_mfma_supported(DType dt, int head_dim, int block_size) {
  // A wave's load instruction covers 512 / head_dim rows of one block.
  return (dt == DType::F16 || dt == DType::BF16) && (head_dim == 64 || head_dim == 128) &&
         block_size >= 512 / head_dim;
}

hipError_t launch_prefill_mfma(const PrefillParams &p, DType dt, hipStream_t stream) {
  // The tile loader computes addresses inside a block with 32-bit byte
  // offsets below 2^31; pools with larger blocks take the VALU kernel.
  const uint64_t eb = 2, lim = (uint64_t)1 << 31;
  const bool narrow = (uint64_t)p.kv_stride_block * eb < lim &&
                      ((uint64_t)p.kv_stride_token * eb << p.block_shift) < lim;
  if (p.group > kRows || !narrow) return launch_prefill_valu(p, dt, stream);
  if (dt == DType::BF16) return launch_t<__bf16>(p, stream);
  if (dt == DType::F16) return launch_t<_Float16>(p, stream);
  return hipErrorInvalidValue;
}

}  // namespace clv
