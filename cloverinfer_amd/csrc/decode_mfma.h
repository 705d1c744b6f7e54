// decode_mfma.h - the per-wave MFMA decode machinery shared by the grid
// kernel (one workgroup per sequence/kv head/partition, decode.hip) and the
// balanced stream kernel (decode_stream.hip).
//
// A wave attends up to 16 query rows (the query heads of one kv head, or a
// 16-row chunk of them) over 16-token steps of one sequence's paged context.
// Per step it runs D/32 MFMAs 16x16x32 for the scores
//   S^T[t, g] = K[t, :] . Q[g, :]       (lane holds S[g = n16][t = 4j + r])
// and 2 x D/16 MFMAs 16x16x16 for O[g, d] += P[g, t] V[t, d]. The A operand
// of the second product is exactly the lane's 4 P values (split into a
// 16-bit value and its 16-bit rounding residual, so P.V keeps fp32-level
// accuracy; over fp8 pools one fp16 value); its B operand for output column
// block m is element m of the lane's 4 V row chunks, regrouped with v_perm. Loads go through buffer
// resources (a wave-uniform base in SGPRs plus 32-bit lane offsets). V rows
// are read whole by each instruction and once per kv head, so they use the
// streaming cache policy; a K instruction reads half of each 128-byte line
// (the next one reads the other half), so K keeps the default policy, which
// lets the second half hit in cache.
#pragma once

#include "attn_common.h"

namespace clv {

template <int CH> struct VChunk;
template <> struct VChunk<8> { typedef u32x4 type; };  // D = 128: 16 bytes per lane
template <> struct VChunk<4> { typedef u32x2 type; };  // D = 64: 8 bytes per lane

// Clamp a context length to what the grid and the block table cover.
__device__ __forceinline__ int clamp_ctx(const DecodeParams &p, int s) {
  const int ctx = p.context_lens[s];
  const int cap = min(p.max_context_len, p.max_blocks_per_seq << p.block_shift);
  return max(0, min(ctx, cap));
}

// Same for a wave-uniform s, read through the scalar unit (for kernels that
// store to global memory inside their main loop).
__device__ __forceinline__ int clamp_ctx(const DecodeParams &p, const int32_t *__restrict__ lens,
                                         int s) {
  const int ctx = scalar_load_i32(lens + s);
  const int cap = min(p.max_context_len, p.max_blocks_per_seq << p.block_shift);
  return max(0, min(ctx, cap));
}

// Where one (sequence, kv head) lives: its block-table row and pool bases.
struct SegGeom {
  const int32_t *bt;
  const char *kbase;
  const char *vbase;
  int t_end;  // tokens [.., t_end) are attended
};

// CEB: bytes per cache element (sizeof(T), or 1 for fp8 pools).
template <typename T, int CEB = (int)sizeof(T)>
__device__ __forceinline__ SegGeom seg_geom(const DecodeParams &p, int s, int kvh, int t_end,
                                           const int32_t *__restrict__ tables) {
  SegGeom g;
  g.bt = tables + (int64_t)s * p.max_blocks_per_seq;
  g.kbase = (const char *)p.k_cache + (int64_t)kvh * p.kv_stride_head * CEB;
  g.vbase = (const char *)p.v_cache + (int64_t)kvh * p.kv_stride_head * CEB;
  g.t_end = t_end;
  return g;
}

// One token's key/value rows (16-bit elements, head_dim 128, at knew / vnew)
// written at byte offset `row_off` of the pools at kbase / vbase, by the
// lanes that load them back in the K-transpose path of DecodeWave: a row r
// of a step is loaded by the lanes with j = r / 4, each its 16-byte chunk
// n16. A load in the same wave that follows the store therefore sees the new
// values without any cross-lane ordering.
__device__ __forceinline__ void kt_store_row(const char *kbase, const char *vbase, int64_t row_off,
                                             int r, const uint16_t *knew, const uint16_t *vnew) {
  const int lane = threadIdx.x & 63;
  if ((lane >> 4) == (r & 15) >> 2) {
    const int64_t off = row_off + (lane & 15) * 16;
    const u32x4 kv = load_vec<u32x4>(knew + (lane & 15) * 8);
    const u32x4 vv = load_vec<u32x4>(vnew + (lane & 15) * 8);
    store_vec<u32x4>(const_cast<char *>(kbase) + off, kv);
    store_vec<u32x4>(const_cast<char *>(vbase) + off, vv);
  }
}

// Two e4m3 values (bytes 0, 1, or 2, 3 with hi) of w as two fp16, exact.
__device__ __forceinline__ uint32_t cvt_fp8x2_f16(uint32_t w, bool hi) {
  return __builtin_bit_cast(uint32_t, hi ? __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.f, true)
                                         : __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.f, false));
}

// Eight fp8 (OCP e4m3) values, bytes of w in order, as eight T values (exact
// for both 16-bit types: e4m3 has 3 mantissa bits and an exponent range
// inside theirs).
template <typename T>
__device__ __forceinline__ u32x4 fp8x8_to(u32x2 w) {
  u32x4 r;
  if constexpr (__is_same(T, __bf16)) {
    r[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[0], 1.f, false));
    r[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[0], 1.f, true));
    r[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[1], 1.f, false));
    r[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[1], 1.f, true));
  } else {
    r[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[0], 1.f, false));
    r[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[0], 1.f, true));
    r[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[1], 1.f, false));
    r[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[1], 1.f, true));
  }
  return r;
}

// UNI: block_size >= 16, so a step sits in one block and its block-table
// entry is wave-uniform (scalar load, buffer loads). Otherwise (block_size 4
// or 8) lanes look up their own rows.
// KT (UNI, head_dim 128): K is loaded like V, whole 256-byte rows with the
// streaming policy (four rows per instruction), and turned into the MFMA A
// layout through a per-wave LDS buffer of 16 rows (set_k_lds). A pure read of
// that pattern runs about 3 % faster than the A-layout loads, which read half
// of each 128-byte line per instruction.
// KV8 (KT only): the pools hold fp8 (OCP e4m3) values with a scale per kv
// head. Each lane loads the same rows as in the 16-bit case at half the width
// (8 bytes = 8 values) and converts them exactly to T in registers; the key
// scale is folded into the softmax scale and the value scale into the
// partial context (set_kv_scales).
template <typename T, int D, bool UNI, bool KT = false, bool KV8 = false>
struct DecodeWave {
  typedef Mfma16x16x32<T> MfK;
  typedef Mfma16x16x16<T> MfV;
  typedef typename MfK::op_t qk_t;
  typedef typename MfV::op_t pv_t;
  static constexpr int NQK = D / 32;  // QK MFMAs per step
  static constexpr int CH = D / 16;   // V elements per lane per token = PV output blocks
  static constexpr int EB = (int)sizeof(T);
  static constexpr int STEP = 16;
  // LDS row stride of the K transpose buffer: 32 mod 64 bytes keeps both the
  // row writes and the A-layout reads (lane row = lane % 16) conflict-free.
  static constexpr int KT_ROW = D * EB + 32;
  static constexpr int KT_BYTES = KT ? 16 * KT_ROW : 16;  // 16: no transpose buffer
  static_assert(!KT || (UNI && D == 128), "K transpose needs block_size >= 16 and head_dim 128");
  static_assert(!KV8 || KT, "fp8 pools are read on the K-transpose path");
  static constexpr int EBC = KV8 ? 1 : EB;  // bytes per cache element
  typedef typename VChunk<CH>::type vchunk_t;

  // Loads of one step: K rows (lane row n16) and the V rows 4j..4j+3.
  struct Regs {
    u32x4 k[NQK];
    vchunk_t v[4];
    u32x2 k8[KV8 ? NQK : 1], v8[KV8 ? 4 : 1];  // KV8: the loaded fp8 values
    bool ok;  // the lane's V rows lie in a readable block
  };

  int n16, j;
  int64_t sblk, stok;
  int bshift, bmask;
  unsigned nblocks;
  float scale_log2;
  uint32_t k_lane;     // byte offset of K row n16, d = 8j, inside a step
  uint32_t v_lane[4];  // byte offsets of V rows 4j + r, d = n16 * CH (KT: also K's)
  char *k_lds;         // KT: this wave's transpose buffer
  f32x4 o[CH];         // O[g = 4j + r][d = n16 * CH + m]
  float m_run;         // running max of row g = n16 (log2 domain)
  float l_run;         // this lane's share of the row sum
  float vscale;        // KV8: value scale of the kv head

  __device__ __forceinline__ void init(const DecodeParams &p) {
    const int lane = threadIdx.x & 63;
    n16 = lane & 15;
    j = lane >> 4;
    sblk = p.kv_stride_block * EBC;
    stok = p.kv_stride_token * EBC;
    bshift = p.block_shift;
    bmask = (1 << bshift) - 1;
    nblocks = (unsigned)p.num_blocks;
    scale_log2 = p.scale_log2;
    k_lane = (uint32_t)(n16 * stok + 8 * j * EB);
#pragma unroll
    for (int r = 0; r < 4; ++r) v_lane[r] = (uint32_t)((4 * j + r) * stok + n16 * CH * EBC);
    vscale = 1.f;
    reset();
  }

  // Output column of accumulator element m in lane group n16 (o[m] holds
  // O[g = 4j + r][col_of(n16, m)]; four consecutive m from a multiple of 4
  // are four consecutive columns).
  __device__ __forceinline__ static int col_of(int n16, int m) { return n16 * CH + m; }

  // KV8: the scales of the kv head a run reads (the key scale times the
  // softmax scale in the log2 domain, and the value scale).
  __device__ __forceinline__ void set_kv_scales(float scale_log2_k, float vs) {
    scale_log2 = scale_log2_k;
    vscale = vs;
  }

  __device__ __forceinline__ void reset() {
#pragma unroll
    for (int m = 0; m < CH; ++m) o[m] = (f32x4){0.f, 0.f, 0.f, 0.f};
    m_run = kNegInf;
    l_run = 0.f;
  }

  // Q rows h0 .. h0+ng-1 of sequence s as the B operand of S^T = K Q^T:
  // lane holds Q[g = n16][d = 32i + 8j .. +8] (zero for g >= ng).
  // Every lane loads (a row >= ng re-reads row ng - 1 and is zeroed), so the
  // number of loads in flight never depends on the lane mask.
  __device__ __forceinline__ void load_q(const DecodeParams &p, int s, int h0, int ng,
                                         qk_t (&q)[NQK]) const {
    u32x4 raw[NQK];
    load_q_raw(p, s, h0, ng, raw);
    mask_q(raw, ng, q);
  }

  // The two halves of load_q, for callers that prefetch: the loads, and the
  // zeroing of rows >= ng (which waits for them).
  __device__ __forceinline__ void load_q_raw(const DecodeParams &p, int s, int h0, int ng,
                                             u32x4 (&raw)[NQK]) const {
    const int row = min(n16, ng - 1);
    const T *qrow = (const T *)p.q + (int64_t)s * p.q_stride_seq + (int64_t)(h0 + row) * p.q_stride_head;
#pragma unroll
    for (int i = 0; i < NQK; ++i) raw[i] = load_vec<u32x4>(qrow + 32 * i + 8 * j);
  }
  __device__ __forceinline__ void mask_q(const u32x4 (&raw)[NQK], int ng, qk_t (&q)[NQK]) const {
#pragma unroll
    for (int i = 0; i < NQK; ++i)
      q[i] = __builtin_bit_cast(qk_t, n16 < ng ? raw[i] : (u32x4){0u, 0u, 0u, 0u});
  }

  // UNI: issue the loads of the 16-token step at token `tok` of block `blk`
  // of a kv head whose pools start at kbase / vbase. A block id outside
  // [0, num_blocks) reads a readable row and is masked when computed.
  __device__ __forceinline__ void issue_blk(const char *kbase, const char *vbase, int blk, int tok,
                                            Regs &R) const {
    const bool ok = (unsigned)blk < nblocks;
    const int64_t off = ok ? blk * sblk + tok * stok : 0;
    R.ok = ok;
    const rsrc_t rk = make_rsrc(kbase + off);
    const rsrc_t rv = make_rsrc(vbase + off);
    if constexpr (KV8) {
#pragma unroll
      for (int i = 0; i < NQK; ++i) R.k8[i] = buf_load<u32x2, kCacheStream>(rk, v_lane[i]);
#pragma unroll
      for (int r = 0; r < 4; ++r) R.v8[r] = buf_load<u32x2, kCacheStream>(rv, v_lane[r]);
      return;
    } else if constexpr (KT) {
#pragma unroll
      for (int i = 0; i < NQK; ++i) R.k[i] = buf_load<u32x4, kCacheStream>(rk, v_lane[i]);
    } else {
#pragma unroll
      for (int i = 0; i < NQK; ++i) R.k[i] = buf_load<u32x4, kCacheDefault>(rk, k_lane + 64u * i);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) R.v[r] = buf_load<vchunk_t, kCacheStream>(rv, v_lane[r]);
  }

  __device__ __forceinline__ void set_k_lds(char *buf) { k_lds = buf; }

  // Issue every load of the step starting at token `base` (< g.t_end). All
  // addresses are in bounds: rows past t_end or in unreadable blocks read a
  // readable row and are masked when the step is computed.
  __device__ __forceinline__ void issue(const SegGeom &g, int base, Regs &R) const {
    if constexpr (UNI) {
      issue_blk(g.kbase, g.vbase, scalar_load_i32(g.bt + (base >> bshift)), base & bmask, R);
    } else {
      const int tk = base + n16;
      const int kb = tk < g.t_end ? g.bt[tk >> bshift] : 0;
      const bool kok = tk < g.t_end && (unsigned)kb < nblocks;
      const int64_t koff = (kok ? kb * sblk + (tk & bmask) * stok : 0) + 8 * j * EB;
      const int tv = base + 4 * j;
      const int vb = tv < g.t_end ? g.bt[tv >> bshift] : 0;
      const bool vok = tv < g.t_end && (unsigned)vb < nblocks;
      R.ok = vok;
      const int64_t voff = (vok ? vb * sblk + (tv & bmask) * stok : 0) + n16 * CH * EB;
#pragma unroll
      for (int i = 0; i < NQK; ++i) R.k[i] = load_vec<u32x4>(g.kbase + koff + 64 * i);
#pragma unroll
      for (int r = 0; r < 4; ++r) R.v[r] = load_vec<vchunk_t>(g.vbase + voff + r * stok);
    }
  }

  // Fold the step starting at `base` into (o, m_run, l_run).
  __device__ __forceinline__ void compute(int base, int t_end, Regs &R, const qk_t (&q)[NQK]) {
    if constexpr (KV8) {
      // fp8 -> 16 bits, exact, eight values per row chunk (the layout of the
      // 16-bit loads): K to T for the score MFMAs. V is converted to fp16,
      // which holds every e4m3 value, while its B operands are built below.
#pragma unroll
      for (int i = 0; i < NQK; ++i) R.k[i] = fp8x8_to<T>(R.k8[i]);
    }
    if constexpr (KT) {
      // R.k[i] holds row 4j + i, bytes 16 n16 .. +16 (the V pattern). Through
      // LDS into the A layout: row n16, bytes 64 i + 16 j .. +16. A wave's LDS
      // operations run in order, so the reads see this step's writes and the
      // next step's writes come after these reads.
#pragma unroll
      for (int i = 0; i < NQK; ++i) store_vec<u32x4>(k_lds + (4 * j + i) * KT_ROW + 16 * n16, R.k[i]);
#pragma unroll
      for (int i = 0; i < NQK; ++i) R.k[i] = load_vec<u32x4>(k_lds + n16 * KT_ROW + 64 * i + 16 * j);
    }
    f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NQK; ++i) sacc = MfK::run(__builtin_bit_cast(qk_t, R.k[i]), q[i], sacc);
    // Masking is needed only on a partial step or an unreadable block.
    const bool full = __all(base + STEP <= t_end && R.ok);
    float x[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool ok = full || (R.ok && base + 4 * j + r < t_end);
      x[r] = ok ? sacc[r] * scale_log2 : kNegInf;
    }
    if (!full) {
      const vchunk_t z = {};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (x[r] == kNegInf) {  // keep NaN/Inf of unused slots out of P.V
          if constexpr (KV8) R.v8[r] = (u32x2){0u, 0u};
          else R.v[r] = z;
        }
      }
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

    // B operand of output block m: element m of the lane's four V rows.
    auto vcol = [&](int m) -> u32x2 {
      const uint32_t w0 = (m & 1) ? pair_hi(R.v[0][m >> 1], R.v[1][m >> 1])
                                  : pair_lo(R.v[0][m >> 1], R.v[1][m >> 1]);
      const uint32_t w1 = (m & 1) ? pair_hi(R.v[2][m >> 1], R.v[3][m >> 1])
                                  : pair_lo(R.v[2][m >> 1], R.v[3][m >> 1]);
      return (u32x2){w0, w1};
    };
    if constexpr (KV8) {
      // fp8 pools: P.V in fp16, one MFMA per block. P lies in [0, 1], where
      // fp16 keeps 11 significant bits (relative rounding <= 2^-12, below
      // the rounding of a 16-bit output).
      // B operands straight from the fp8 bytes: element m of row r is byte
      // m & 3 of word m >> 2 of R.v8[r]; one byte permute gathers elements
      // m, m + 1 of two rows, and each fp8 pair converts into one B word
      // (8 permutes and 16 conversions per step instead of 16 + 16).
      typedef Mfma16x16x16<_Float16> MfH;
      const typename MfH::op_t ph = pack4<_Float16>(pf);
#pragma unroll
      for (int m = 0; m < CH; m += 2) {
        const int w = m >> 2, a = m & 3;
        const uint32_t sel = (uint32_t)a | (uint32_t)(a + 4) << 8 | (uint32_t)(a + 1) << 16 |
                             (uint32_t)(a + 5) << 24;
        // bytes (row 2c, m), (row 2c + 1, m), (row 2c, m + 1), (row 2c + 1, m + 1)
        const uint32_t x01 = __builtin_amdgcn_perm(R.v8[1][w], R.v8[0][w], sel);
        const uint32_t x23 = __builtin_amdgcn_perm(R.v8[3][w], R.v8[2][w], sel);
        const u32x2 b0 = {cvt_fp8x2_f16(x01, false), cvt_fp8x2_f16(x23, false)};
        const u32x2 b1 = {cvt_fp8x2_f16(x01, true), cvt_fp8x2_f16(x23, true)};
        o[m] = MfH::run(ph, __builtin_bit_cast(typename MfH::op_t, b0), o[m]);
        o[m + 1] = MfH::run(ph, __builtin_bit_cast(typename MfH::op_t, b1), o[m + 1]);
      }
    } else {
      const pv_t pa = pack4<T>(pf);
#pragma unroll
      for (int r = 0; r < 4; ++r) lo[r] = pf[r] - (float)pa[r];
      const pv_t pl = pack4<T>(lo);
#pragma unroll
      for (int m = 0; m < CH; ++m) {
        const pv_t vb = __builtin_bit_cast(pv_t, vcol(m));
        o[m] = MfV::run(pa, vb, o[m]);
        o[m] = MfV::run(pl, vb, o[m]);
      }
    }
  }

  // Sum the row sums over the four lane groups that hold each row.
  __device__ __forceinline__ void reduce_rowsum() {
    l_run += shfl_xor(l_run, 16);
    l_run += shfl_xor(l_run, 32);
  }

  // After reduce_rowsum(): write this wave's normalised partial of rows
  // g < ng as rows (row0 + g * rstride) of the workspace: context, row max
  // (natural log domain) and row sum.
  __device__ __forceinline__ void store_partial(float *ws_o, float *ws_m, float *ws_l,
                                                int64_t row0, int ng,
                                                int64_t rstride = 1) const {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int g = 4 * j + r;
      const float l = shfl(l_run, g);
      const float mrow = shfl(m_run, g);
      if (g >= ng) continue;
      const int64_t row = row0 + g * rstride;
      const float inv = (l > 0.f ? 1.f / l : 0.f) * (KV8 ? vscale : 1.f);
      float *dst = ws_o + row * D + n16 * CH;
#pragma unroll
      for (int m = 0; m < CH; m += 4) {
        const f32x4 v = {o[m][r] * inv, o[m + 1][r] * inv, o[m + 2][r] * inv, o[m + 3][r] * inv};
        store_vec<f32x4>(dst + m, v);
      }
      if (n16 == 0) {
        ws_m[row] = l > 0.f ? mrow * kLn2 : kNegInf;
        ws_l[row] = l;
      }
    }
  }
};

// fp32 pools: the per-wave decode of DecodeWave on v_mfma_f32_16x16x4f32
// (fp32 operands and accumulation: K, V, Q and P are never rounded, as in
// CpuAttentionBackend's fp32 einsums). Operand layout of that instruction
// for lane l (measured on gfx950): A[row l%16][k l/16], B[k l/16][col l%16],
// C rows 4(l/16) .. +4, col l%16. The fragments are DecodeWave's: the score
// MFMAs leave S[g = n16][t = 4j + r] in the lane, which is its P operand
// (k = j <-> token 4j + c for MFMA c) of the P.V MFMAs. The order of the
// score sum over d and the placement of output columns are free, and are
// chosen so that each load instruction reads contiguous runs: score MFMA
// c = 4i + e takes d = 16i + 4j + e in lane group j (load i of a K row reads
// 64 consecutive bytes across the four lane groups; the lane holds the same
// Q floats), and o[4w + e] holds O[g = 4j + r][d = 64w + 4 n16 + e] (load w
// of a V row reads 256 consecutive bytes across the 16 lanes of a group).
template <int D, bool UNI>
struct DecodeWaveF32 {
  typedef u32x4 qk_t;                 // four fp32 Q values
  static constexpr int NQK = D / 16;  // Q / K words per lane (D / 4 floats)
  static constexpr int CH = D / 16;   // V floats per lane per row = P.V output blocks
  static constexpr int VW = CH / 4;   // V words per lane per row (64 columns apart)
  static constexpr int EB = 4;
  static constexpr int STEP = 16;
  static constexpr int KT_BYTES = 16;  // no transpose buffer

  struct Regs {
    u32x4 k[NQK];     // K row n16, floats 16i + 4j .. +4
    u32x4 v[4][VW];   // V rows 4j + c, floats 64w + 4 n16 .. +4
    bool ok;          // the lane's V rows lie in a readable block
  };

  int n16, j;
  int64_t sblk, stok;
  int bshift, bmask;
  unsigned nblocks;
  float scale_log2;
  uint32_t k_lane;     // byte offset of K row n16, float 4j, inside a step
  uint32_t v_lane[4];  // byte offsets of V rows 4j + c, float 4 n16
  f32x4 o[CH];         // O[g = 4j + r][d = 64 (m / 4) + 4 n16 + m % 4]
  float m_run;         // running max of row g = n16 (log2 domain)
  float l_run;         // this lane's share of the row sum

  __device__ __forceinline__ void init(const DecodeParams &p) {
    const int lane = threadIdx.x & 63;
    n16 = lane & 15;
    j = lane >> 4;
    sblk = p.kv_stride_block * EB;
    stok = p.kv_stride_token * EB;
    bshift = p.block_shift;
    bmask = (1 << bshift) - 1;
    nblocks = (unsigned)p.num_blocks;
    scale_log2 = p.scale_log2;
    k_lane = (uint32_t)(n16 * stok + 4 * j * EB);
#pragma unroll
    for (int c = 0; c < 4; ++c) v_lane[c] = (uint32_t)((4 * j + c) * stok + 4 * n16 * EB);
    reset();
  }

  __device__ __forceinline__ void set_k_lds(char *) {}

  // As DecodeWave::col_of, for this wave's column placement.
  __device__ __forceinline__ static int col_of(int n16, int m) {
    return 64 * (m >> 2) + 4 * n16 + (m & 3);
  }

  __device__ __forceinline__ void reset() {
#pragma unroll
    for (int m = 0; m < CH; ++m) o[m] = (f32x4){0.f, 0.f, 0.f, 0.f};
    m_run = kNegInf;
    l_run = 0.f;
  }

  // Q rows h0 .. h0+ng-1 of sequence s: word i of the lane holds
  // Q[g = n16][d = 16i + 4j .. +4] (zero for g >= ng; every lane loads, a
  // row >= ng re-reads row ng - 1).
  __device__ __forceinline__ void load_q_raw(const DecodeParams &p, int s, int h0, int ng,
                                             u32x4 (&raw)[NQK]) const {
    const int row = min(n16, ng - 1);
    const float *qrow = (const float *)p.q + (int64_t)s * p.q_stride_seq +
                        (int64_t)(h0 + row) * p.q_stride_head + 4 * j;
#pragma unroll
    for (int i = 0; i < NQK; ++i) raw[i] = load_vec<u32x4>(qrow + 16 * i);
  }
  __device__ __forceinline__ void mask_q(const u32x4 (&raw)[NQK], int ng, qk_t (&q)[NQK]) const {
#pragma unroll
    for (int i = 0; i < NQK; ++i) q[i] = n16 < ng ? raw[i] : (u32x4){0u, 0u, 0u, 0u};
  }
  __device__ __forceinline__ void load_q(const DecodeParams &p, int s, int h0, int ng,
                                         qk_t (&q)[NQK]) const {
    u32x4 raw[NQK];
    load_q_raw(p, s, h0, ng, raw);
    mask_q(raw, ng, q);
  }

  // UNI: the loads of the 16-token step at token `tok` of block `blk` (an
  // unreadable block reads a readable row and is masked when computed).
  __device__ __forceinline__ void issue_blk(const char *kbase, const char *vbase, int blk, int tok,
                                            Regs &R) const {
    const bool ok = (unsigned)blk < nblocks;
    const int64_t off = ok ? blk * sblk + tok * stok : 0;
    R.ok = ok;
    const rsrc_t rk = make_rsrc(kbase + off);
    const rsrc_t rv = make_rsrc(vbase + off);
#pragma unroll
    for (int i = 0; i < NQK; ++i) R.k[i] = buf_load<u32x4, kCacheDefault>(rk, k_lane + 64u * i);
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int w = 0; w < VW; ++w) R.v[c][w] = buf_load<u32x4, kCacheStream>(rv, v_lane[c] + 256u * w);
  }

  // Block sizes below 16: each lane looks up the blocks of its own rows.
  __device__ __forceinline__ void issue(const SegGeom &g, int base, Regs &R) const {
    if constexpr (UNI) {
      issue_blk(g.kbase, g.vbase, scalar_load_i32(g.bt + (base >> bshift)), base & bmask, R);
    } else {
      const int tk = base + n16;
      const int kb = tk < g.t_end ? g.bt[tk >> bshift] : 0;
      const bool kok = tk < g.t_end && (unsigned)kb < nblocks;
      const int64_t koff = (kok ? kb * sblk + (tk & bmask) * stok : 0) + 4 * j * EB;
      const int tv = base + 4 * j;
      const int vb = tv < g.t_end ? g.bt[tv >> bshift] : 0;
      const bool vok = tv < g.t_end && (unsigned)vb < nblocks;
      R.ok = vok;
      const int64_t voff = (vok ? vb * sblk + (tv & bmask) * stok : 0) + 4 * n16 * EB;
#pragma unroll
      for (int i = 0; i < NQK; ++i) R.k[i] = load_vec<u32x4>(g.kbase + koff + 64 * i);
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int w = 0; w < VW; ++w)
          R.v[c][w] = load_vec<u32x4>(g.vbase + voff + c * stok + 256 * w);
    }
  }

  __device__ __forceinline__ static f32x4 mfma(uint32_t a, uint32_t b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(__builtin_bit_cast(float, a),
                                                __builtin_bit_cast(float, b), c, 0, 0, 0);
  }

  // Fold the step starting at `base` into (o, m_run, l_run).
  __device__ __forceinline__ void compute(int base, int t_end, Regs &R, const qk_t (&q)[NQK]) {
    // Two accumulators (even / odd k-steps) keep consecutive MFMAs independent.
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NQK; ++i) {
      s0 = mfma(R.k[i][0], q[i][0], s0);
      s1 = mfma(R.k[i][1], q[i][1], s1);
      s0 = mfma(R.k[i][2], q[i][2], s0);
      s1 = mfma(R.k[i][3], q[i][3], s1);
    }
    const f32x4 sacc = s0 + s1;
    const bool full = __all(base + STEP <= t_end && R.ok);
    float x[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool ok = full || (R.ok && base + 4 * j + r < t_end);
      x[r] = ok ? sacc[r] * scale_log2 : kNegInf;
    }
    if (!full) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (x[r] == kNegInf) {
#pragma unroll
          for (int w = 0; w < VW; ++w) R.v[r][w] = (u32x4){0u, 0u, 0u, 0u};  // NaN/Inf of unused slots
        }
    }
    float mx = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    mx = fmaxf(mx, shfl_xor(mx, 16));
    mx = fmaxf(mx, shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float msub = (m_new == kNegInf) ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - msub);
    float pf[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) pf[r] = fast_exp2(x[r] - msub);
    l_run = l_run * alpha + ((pf[0] + pf[1]) + (pf[2] + pf[3]));
    m_run = m_new;
    if (__any(alpha != 1.f)) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float a = shfl(alpha, 4 * j + r);
#pragma unroll
        for (int m = 0; m < CH; ++m) o[m][r] *= a;
      }
    }
    // P.V: MFMA (c, m) takes token 4j + c (k = j) and output column
    // 64 (m / 4) + 4 n16 + m % 4.
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t a = __builtin_bit_cast(uint32_t, pf[c]);
#pragma unroll
      for (int m = 0; m < CH; ++m) o[m] = mfma(a, R.v[c][m >> 2][m & 3], o[m]);
    }
  }

  __device__ __forceinline__ void reduce_rowsum() {
    l_run += shfl_xor(l_run, 16);
    l_run += shfl_xor(l_run, 32);
  }

  // As DecodeWave::store_partial, with this wave's output columns.
  __device__ __forceinline__ void store_partial(float *ws_o, float *ws_m, float *ws_l,
                                                int64_t row0, int ng,
                                                int64_t rstride = 1) const {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int g = 4 * j + r;
      const float l = shfl(l_run, g);
      const float mrow = shfl(m_run, g);
      if (g >= ng) continue;
      const int64_t row = row0 + g * rstride;
      const float inv = l > 0.f ? 1.f / l : 0.f;
      float *dst = ws_o + row * D + 4 * n16;
#pragma unroll
      for (int m = 0; m < CH; m += 4) {
        const f32x4 v = {o[m][r] * inv, o[m + 1][r] * inv, o[m + 2][r] * inv, o[m + 3][r] * inv};
        store_vec<f32x4>(dst + 16 * m, v);
      }
      if (n16 == 0) {
        ws_m[row] = l > 0.f ? mrow * kLn2 : kNegInf;
        ws_l[row] = l;
      }
    }
  }
};

// The per-wave decode type of the grid kernel (paged_decode_mfma). K stays
// in the A layout here: the K transpose of the stream kernel measured 6 %
// slower in this kernel (16 x 32K-token split-K decode: 364 -> 387 us, also
// at three waves per SIMD).
template <typename T, int D, bool UNI>
struct GridWave {
  typedef DecodeWave<T, D, UNI> type;
};
template <int D, bool UNI>
struct GridWave<float, D, UNI> {
  typedef DecodeWaveF32<D, UNI> type;
};

// The per-wave decode type of the balanced stream kernel.
template <typename T, int D, bool UNI, bool KV8>
struct StreamWave {
  typedef DecodeWave<T, D, UNI, UNI && D == 128, KV8> type;
};
template <int D, bool UNI>
struct StreamWave<float, D, UNI, false> {
  typedef DecodeWaveF32<D, UNI> type;
};

// Log-sum-exp merge of n partial rows, the rule of the reference's
// partial-softmax merge (src/core/resident_kv_store.py:2497-2509) over all
// rows at once:
//   M = max_i m_i, w_i = l_i e^(m_i - M), out = sum_i c_i w_i / max(sum_i w_i, 1e-12).
// Row i: row max m[i * ms] (natural-log domain), row sum l[i * ms], context
// c[i * cs .. + D]. NW waves (consecutive in the workgroup, NW > 1 only for a
// one-row workgroup) split the rows in chunks of C = min(64, ceil(n / NW));
// each lane weighs one row of a chunk, and R context rows are loaded per
// round so that their latencies overlap (R = 16 for NW > 1: 64 partitions
// then take one round per wave). NW > 1 combines the waves through smem
// (NW * (D + 1) floats) and needs every thread of the workgroup to call this.
// X: an extra row of max xm, sum 1 and context xv (element lane + 64 e in
// xv[e]) joins the merge, a single token's own term (score, value), so that
// a decode over a context can take one more token after its partials are
// written. The score is xm = (sum over the wave of xdot) * xscale, summed
// here after the rows' loads are issued so that its shuffles overlap them.
template <typename T, int D, int NW, bool X = false>
__device__ __forceinline__ void lse_merge(const float *m, const float *l, const float *c,
                                          int64_t ms, int64_t cs, int n, T *dst, float *smem,
                                          float xdot = 0.f, float xscale = 0.f,
                                          const float *xv = nullptr) {
  constexpr int EPL = (D + 63) / 64;
  constexpr int R = NW > 1 ? 16 : 8;
  const int lane = threadIdx.x & 63;
  const int wv = NW > 1 ? (int)(threadIdx.x >> 6) : 0;
  const int C = NW > 1 ? max(1, min(64, (n + NW - 1) / NW)) : 64;
  // The row's max needs every m_i; the first chunk's (m, l) and its first
  // R context rows are loaded together, before any reduction, so that a
  // row with at most C * NW partials costs one round trip to memory.
  const int base0 = C * wv;
  const int cnt0 = max(0, min(C, n - base0));
  float m0 = kNegInf, l0 = 0.f;
  if (lane < cnt0) {
    m0 = m[(int64_t)(base0 + lane) * ms];
    l0 = l[(int64_t)(base0 + lane) * ms];
  }
  float v[R][EPL];
#pragma unroll
  for (int u = 0; u < R; ++u)
#pragma unroll
    for (int e = 0; e < EPL; ++e)
      v[u][e] = (u < cnt0 && lane + 64 * e < D) ? c[(int64_t)(base0 + u) * cs + lane + 64 * e] : 0.f;
  float xm = kNegInf;
  if constexpr (X) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) xdot += shfl_xor(xdot, off);
    xm = xdot * xscale;
  }
  float M = fmaxf(m0, xm);
  for (int i = lane; i < n; i += 64)
    if (i < base0 || i >= base0 + cnt0) M = fmaxf(M, m[i * ms]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, shfl_xor(M, off));
  const float Msub = (M == kNegInf) ? 0.f : M;
  float L = 0.f;
  float acc[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
  for (int base = base0; base < n; base += C * NW) {
    const int cnt = min(C, n - base);
    float wl = 0.f;
    if (base == base0) {
      if (lane < cnt) wl = l0 * fast_exp2((m0 - Msub) * kLog2e);
    } else if (lane < cnt) {
      const int64_t r = (int64_t)(base + lane) * ms;
      wl = l[r] * fast_exp2((m[r] - Msub) * kLog2e);
    }
    L += wl;
    for (int k = 0; k < cnt; k += R) {
      if (base != base0 || k != 0) {
#pragma unroll
        for (int u = 0; u < R; ++u)
#pragma unroll
          for (int e = 0; e < EPL; ++e)
            v[u][e] = (k + u < cnt && lane + 64 * e < D)
                          ? c[(int64_t)(base + k + u) * cs + lane + 64 * e] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < R; ++u) {
        const float w = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), k + u < 64 ? k + u : 63));
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[e] += v[u][e] * w;
      }
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) L += shfl_xor(L, off);
  if constexpr (NW > 1) {
    float *sl = smem;
    float *sa = smem + NW;
    if (lane == 0) sl[wv] = L;
#pragma unroll
    for (int e = 0; e < EPL; ++e)
      if (lane + 64 * e < D) sa[wv * D + lane + 64 * e] = acc[e];
    __syncthreads();
    if (wv != 0) return;
    L = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) L += sl[w];
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      acc[e] = 0.f;
      if (lane + 64 * e < D)
#pragma unroll
        for (int w = 0; w < NW; ++w) acc[e] += sa[w * D + lane + 64 * e];
    }
  }
  if constexpr (X) {  // the extra row, after the waves are combined
    const float wx = fast_exp2((xm - Msub) * kLog2e);
    L += wx;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] += xv[e] * wx;
  }
  const float inv = 1.f / fmaxf(L, 1e-12f);
#pragma unroll
  for (int e = 0; e < EPL; ++e)
    if (lane + 64 * e < D) dst[lane + 64 * e] = from_f32<T>(acc[e] * inv);
}

}  // namespace clv
