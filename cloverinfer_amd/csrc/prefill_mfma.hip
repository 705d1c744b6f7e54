// prefill_mfma.hip - chunked prefill over paged KV with MFMA (fp16/bf16).
//
// Semantics as in prefill.hip: query row i of sequence s sees cached
// positions p <= context_lens[s] - n_s + i.
//
// Work decomposition: one workgroup (4 waves) per (sequence, kv head,
// query tile). A query tile holds 128 rows = bq tokens x G query heads of
// the kv head (row r is token r / G, head r % G), so the K/V tile staged in
// LDS serves every query head of the group. Each wave owns 32 rows (two
// 16-row MFMA tiles). Per 64-token KV tile a wave runs
//   S^T[t, r] = K[t, :] . Q[r, :]    4 token tiles x 2 row tiles x D/32 MFMAs
//   O[r, d]  += P[r, t] V[t, d]      2 token halves x 2 row tiles x 2 x D/16 MFMAs
// (v_mfma_f32_16x16x32_{bf16,f16}), with an fp32 online softmax between.
// As in the decode kernel, each lane's P values are already its A operand
// of the PV product, and V is regrouped from 16-byte row chunks with v_perm.
// K/V tiles are double-buffered in LDS: the global loads of tile k+1 are in
// flight while tile k is computed. Workgroup ids are remapped so that all
// query tiles of one (sequence, kv head) run on the same XCD and share its L2.
#include "attn_common.h"

namespace clv {
namespace {

constexpr int kThreads = 256;
constexpr int kRows = 128;  // query rows per workgroup
constexpr int kBK = 64;     // KV tokens per tile

template <int CH> struct VChunkP;
template <> struct VChunkP<8> { typedef u32x4 type; };
template <> struct VChunkP<4> { typedef u32x2 type; };

template <typename T, int D>
__global__ void __launch_bounds__(kThreads)
chunked_prefill_mfma(const PrefillParams p, int bq, int n_qtiles, int total) {
  typedef Mfma16x16x32<T> Mf;
  typedef typename Mf::op_t op_t;
  constexpr int NQK = D / 32;             // QK k-steps
  constexpr int CH = D / 16;              // PV MFMAs per (half, row tile)
  constexpr int LROW = D + 8;             // padded LDS row (elements)
  constexpr int CPR = D * 2 / 16;         // 16-byte chunks per row
  constexpr int RPP = kThreads / CPR;     // rows per load pass
  constexpr int PASSES = kBK / RPP;       // load passes per tile
  typedef typename VChunkP<CH>::type vchunk_t;

  __shared__ __attribute__((aligned(16))) T sK[2][kBK * LROW];
  __shared__ __attribute__((aligned(16))) T sV[2][kBK * LROW];
  __shared__ uint32_t sValid[2][kBK / 4];  // one byte per token: 1 = readable

  // XCD-aware remap: consecutive ids go round-robin over the 8 XCDs; give
  // each XCD a contiguous range of logical work items.
  const int per_xcd = gridDim.x / 8;
  const int L = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (L >= total) return;
  const int qt = L % n_qtiles;
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
  const int wave = tid >> 6;
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

  // Q (B operand of S^T = K Q^T) for this lane's rows 32w + 16rt + n16.
  op_t qop[2][NQK];
  int lim[2];  // last visible position of the lane's softmax row
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int r = 32 * wave + 16 * rt + n16;
    const int tok = q0 + r / G;
    const bool ok = r < bq * G && tok < n_new;
    lim[rt] = ok ? base_pos + tok : -1;
    const T *qrow = (const T *)p.q + (int64_t)(qs + tok) * p.q_stride_token +
                    (int64_t)(kvh * G + r % G) * p.q_stride_head;
#pragma unroll
    for (int i = 0; i < NQK; ++i) {
      u32x4 w = {0u, 0u, 0u, 0u};
      if (ok) w = load_vec<u32x4>(qrow + 32 * i + 8 * j);
      qop[rt][i] = __builtin_bit_cast(op_t, w);
    }
  }

  // Tile loader: thread handles chunk (tid % CPR) of rows tid / CPR + RPP*i.
  const int lchunk = tid % CPR;
  const int lrow = tid / CPR;
  u32x4 kreg[PASSES], vreg[PASSES];
  bool rvalid[PASSES];
  auto load_tile = [&](int tile) {
#pragma unroll
    for (int i = 0; i < PASSES; ++i) {
      const int t = tile * kBK + lrow + RPP * i;
      const int64_t off = t < kv_end ? kv.row_offset(t) : -1;
      rvalid[i] = off >= 0;
      const u32x4 z = {0u, 0u, 0u, 0u};
      kreg[i] = rvalid[i] ? load_vec<u32x4>(kv.kbase + off + lchunk * 16) : z;
      vreg[i] = rvalid[i] ? load_vec<u32x4>(kv.vbase + off + lchunk * 16) : z;
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < PASSES; ++i) {
      const int row = lrow + RPP * i;
      store_vec<u32x4>(&sK[buf][row * LROW + lchunk * 8], kreg[i]);
      store_vec<u32x4>(&sV[buf][row * LROW + lchunk * 8], vreg[i]);
      if (lchunk == 0) ((uint8_t *)sValid[buf])[row] = rvalid[i] ? 1 : 0;
    }
  };

  f32x4 o[2][CH];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int m = 0; m < CH; ++m) o[rt][m] = (f32x4){0.f, 0.f, 0.f, 0.f};
  float m_run[2] = {kNegInf, kNegInf};
  float l_run[2] = {0.f, 0.f};

  if (ntiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int tile = 0; tile < ntiles; ++tile) {
    const int buf = tile & 1;
    const bool more = tile + 1 < ntiles;
    if (more) load_tile(tile + 1);
    const T *K = sK[buf];
    const T *V = sV[buf];
    const int t0 = tile * kBK;

    // ---- scores: sacc[tt][rt][r] = S[row 16rt + n16][token t0 + 16tt + 4j + r]
    f32x4 sacc[4][2];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      sacc[tt][0] = (f32x4){0.f, 0.f, 0.f, 0.f};
      sacc[tt][1] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < NQK; ++i) {
        const op_t a = __builtin_bit_cast(
            op_t, load_vec<u32x4>(&K[(16 * tt + n16) * LROW + 32 * i + 8 * j]));
        sacc[tt][0] = Mf::run(a, qop[0][i], sacc[tt][0]);
        sacc[tt][1] = Mf::run(a, qop[1][i], sacc[tt][1]);
      }
    }

    // ---- online softmax per row tile
    uint32_t vflags[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) vflags[tt] = sValid[buf][4 * tt + j];
    float pf[2][16];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      float mx = kNegInf;
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int pos = t0 + 16 * tt + 4 * j + r;
          const bool ok = ((vflags[tt] >> (8 * r)) & 0xffu) != 0 && pos <= lim[rt];
          const float x = ok ? sacc[tt][rt][r] * p.scale_log2 : kNegInf;
          pf[rt][4 * tt + r] = x;
          mx = fmaxf(mx, x);
        }
      }
      mx = fmaxf(mx, shfl_xor(mx, 16));
      mx = fmaxf(mx, shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run[rt], mx);
      const float msub = (m_new == kNegInf) ? 0.f : m_new;
      const float alpha = fast_exp2(m_run[rt] - msub);
      float psum = 0.f;
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        pf[rt][k] = fast_exp2(pf[rt][k] - msub);
        psum += pf[rt][k];
      }
      l_run[rt] = l_run[rt] * alpha + psum;
      m_run[rt] = m_new;
      if (__any(alpha != 1.f)) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float a = shfl(alpha, 4 * j + r);
#pragma unroll
          for (int m = 0; m < CH; ++m) o[rt][m][r] *= a;
        }
      }
    }

    // ---- O += P V, two 32-token halves
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      vchunk_t vr[8];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          vr[4 * h + r] = load_vec<vchunk_t>(&V[(32 * half + 16 * h + 4 * j + r) * LROW + n16 * CH]);
      // P split into its 16-bit value and the 16-bit rounding residual, so
      // that P.V keeps fp32-level accuracy.
      op_t pa[2], pl[2];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        float x[8], lo[8];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int r = 0; r < 4; ++r) x[4 * h + r] = pf[rt][4 * (2 * half + h) + r];
        pa[rt] = pack8<T>(x);
#pragma unroll
        for (int k = 0; k < 8; ++k) lo[k] = x[k] - (float)pa[rt][k];
        pl[rt] = pack8<T>(lo);
      }
#pragma unroll
      for (int m = 0; m < CH; ++m) {
        u32x4 w;
#pragma unroll
        for (int q2 = 0; q2 < 4; ++q2) {
          const uint32_t a = vr[2 * q2][m >> 1];
          const uint32_t b = vr[2 * q2 + 1][m >> 1];
          w[q2] = (m & 1) ? pair_hi(a, b) : pair_lo(a, b);
        }
        const op_t vb = __builtin_bit_cast(op_t, w);
        o[0][m] = Mf::run(pa[0], vb, o[0][m]);
        o[1][m] = Mf::run(pa[1], vb, o[1][m]);
        o[0][m] = Mf::run(pl[0], vb, o[0][m]);
        o[1][m] = Mf::run(pl[1], vb, o[1][m]);
      }
    }

    if (more) store_tile(buf ^ 1);
    __syncthreads();
  }

  // ---- normalise and store rows 32w + 16rt + 4j + r
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    l_run[rt] += shfl_xor(l_run[rt], 16);
    l_run[rt] += shfl_xor(l_run[rt], 32);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float l = shfl(l_run[rt], 4 * j + r);
      const int row = 32 * wave + 16 * rt + 4 * j + r;
      const int tok = q0 + row / G;
      if (row >= bq * G || tok >= n_new) continue;
      const float inv = l > 0.f ? 1.f / l : 0.f;
      T *dst = (T *)p.out + (int64_t)(qs + tok) * p.out_stride_token +
               (int64_t)(kvh * G + row % G) * p.out_stride_head + n16 * CH;
      uint32_t u[CH / 2];
#pragma unroll
      for (int m = 0; m < CH; m += 2) {
        const uint32_t lo = __builtin_bit_cast(uint16_t, (T)(o[rt][m][r] * inv));
        const uint32_t hi = __builtin_bit_cast(uint16_t, (T)(o[rt][m + 1][r] * inv));
        u[m / 2] = lo | (hi << 16);
      }
      if constexpr (CH == 8) {
        const u32x4 w = {u[0], u[1], u[2], u[3]};
        store_vec<u32x4>(dst, w);
      } else {
        const u32x2 w = {u[0], u[1]};
        store_vec<u32x2>(dst, w);
      }
    }
  }
}

template <typename T>
hipError_t launch_t(const PrefillParams &p, hipStream_t stream) {
  const int bq = kRows / p.group;
  const int n_qtiles = (p.max_query_len + bq - 1) / bq;
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
  (void)block_size;
  return (dt == DType::F16 || dt == DType::BF16) && (head_dim == 64 || head_dim == 128);
}

hipError_t launch_prefill_mfma(const PrefillParams &p, DType dt, hipStream_t stream) {
  if (p.group > kRows) return launch_prefill_valu(p, dt, stream);
  if (dt == DType::BF16) return launch_t<__bf16>(p, stream);
  if (dt == DType::F16) return launch_t<_Float16>(p, stream);
  return hipErrorInvalidValue;
}

}  // namespace clv
