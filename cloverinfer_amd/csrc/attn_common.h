// attn_common.h - pieces shared by the decode and prefill kernels: the view
// of one kv head of the paged pools, the per-wave LDS partials, the
// workgroup epilogue that merges them, and the VALU attention body.
#pragma once

#include "clv_device.h"

namespace clv {

// One kv head of the paged pools plus one sequence's block-table row.
struct KvView {
  const int32_t *bt;   // block-table row of the sequence
  const char *kbase;   // k_cache + kv_head * kv_stride_head (bytes)
  const char *vbase;   // v_cache + kv_head * kv_stride_head (bytes)
  int64_t sblk, stok;  // block and token strides in bytes
  int block_shift;
  unsigned num_blocks;

  // Byte offset of token t's row, or -1 when its block-table entry is out of
  // range (the token is then masked and never dereferenced).
  __device__ __forceinline__ int64_t row_offset(int t) const {
    const int blk = bt[t >> block_shift];
    if ((unsigned)blk >= num_blocks) return -1;
    return blk * sblk + (t & ((1 << block_shift) - 1)) * stok;
  }
};

// Per-wave partial results handed to the workgroup epilogue through LDS:
// row max (log2 domain), row sum, unnormalised context.
template <int NW, int GR, int D>
struct WaveSmem {
  float m[NW][GR];
  float l[NW][GR];
  float o[NW][GR][D];
};

// Where the epilogue writes row g (0 <= g < ng) of a workgroup.
template <typename T>
struct OutDesc {
  bool split;        // true: split-K partial into the workspace
  T *out;            // row 0 of the final output
  int64_t out_stride;
  float *ws_o;       // row 0 of the partial contexts (fp32, D per row)
  float *ws_m;
  float *ws_l;
  int64_t ws_stride; // rows between consecutive g in the workspace
};

// Merge the NW wave partials of rows [0, ng) and store normalised contexts.
// Split-K partials also record the row max in the natural-log domain and the
// row sum, the (context, row_max, row_sum) triple of the reference's
// partial-softmax segments (src/core/resident_kv_store.py:715-783).
// `tid` numbers the NW * 64 threads that share the work (by default the
// workgroup's; a wave that merges on its own passes its lane).
template <typename T, int NW, int GR, int D>
__device__ __forceinline__ void merge_and_store(const WaveSmem<NW, GR, D> &sm, int ng,
                                                const OutDesc<T> &od, int tid = threadIdx.x) {
  constexpr int CPR = D / 8;  // 8-element chunks per row
  for (int idx = tid; idx < GR * CPR; idx += NW * 64) {
    const int g = idx / CPR;
    const int c = idx - g * CPR;
    if (g >= ng) continue;
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, sm.m[w][g]);
    const float Msub = (M == kNegInf) ? 0.f : M;
    float L = 0.f;
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float wt = fast_exp2(sm.m[w][g] - Msub);
      L += sm.l[w][g] * wt;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += sm.o[w][g][c * 8 + e] * wt;
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    if (od.split) {
      const int64_t row = (int64_t)g * od.ws_stride;
      float *dst = od.ws_o + row * D + c * 8;
      const f32x4 a = {acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
      const f32x4 b = {acc[4] * inv, acc[5] * inv, acc[6] * inv, acc[7] * inv};
      store_vec<f32x4>(dst, a);
      store_vec<f32x4>(dst + 4, b);
      if (c == 0) {
        od.ws_m[row] = L > 0.f ? M * kLn2 : kNegInf;
        od.ws_l[row] = L;
      }
    } else {
      T *dst = od.out + (int64_t)g * od.out_stride + c * 8;
      if constexpr (sizeof(T) == 2) {
        uint32_t r[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) r[e] = __builtin_bit_cast(uint16_t, (T)(acc[e] * inv));
        const u32x4 w = {r[0] | (r[1] << 16), r[2] | (r[3] << 16), r[4] | (r[5] << 16),
                         r[6] | (r[7] << 16)};
        store_vec<u32x4>(dst, w);
      } else {
        const f32x4 a = {acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
        const f32x4 b = {acc[4] * inv, acc[5] * inv, acc[6] * inv, acc[7] * inv};
        store_vec<f32x4>(dst, a);
        store_vec<f32x4>(dst + 4, b);
      }
    }
  }
}

// VALU attention of ng (<= GM) query rows over tokens [t_begin, t_end) of
// one kv head; leaves each wave's partial in sm (caller syncs and merges).
// Lane layout: a token row of D elements is split into 16-byte chunks, LPT
// lanes per token, TPI tokens per wave iteration. Each lane keeps its own
// online-softmax state per query row; the TPI token rows are merged at the
// end with the log-sum-exp rule.
template <typename T, int D, int GM, int NW>
__device__ __forceinline__ void valu_attend(const T *q0, int64_t q_stride_head, int ng,
                                            const KvView &kv, int t_begin, int t_end,
                                            float scale_log2, WaveSmem<NW, GM, D> &sm) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int LPT = D / VEC;
  constexpr int TPI = 64 / LPT;
  static_assert(LPT <= 64 && (64 % LPT) == 0, "token row must fit a wave");

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row = lane / LPT;
  const int col = lane - row * LPT;

  float qf[GM][VEC];
#pragma unroll
  for (int g = 0; g < GM; ++g) {
    if (g < ng) {
      const u32x4 w = load_vec<u32x4>(q0 + (int64_t)g * q_stride_head + col * VEC);
      const T *e = (const T *)&w;
#pragma unroll
      for (int v = 0; v < VEC; ++v) qf[g][v] = to_f32(e[v]);
    } else {
#pragma unroll
      for (int v = 0; v < VEC; ++v) qf[g][v] = 0.f;
    }
  }

  float m[GM], l[GM], acc[GM][VEC];
#pragma unroll
  for (int g = 0; g < GM; ++g) {
    m[g] = kNegInf;
    l[g] = 0.f;
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[g][v] = 0.f;
  }

  for (int base = t_begin + wave * TPI; base < t_end; base += NW * TPI) {
    const int t = base + row;
    int64_t off = t < t_end ? kv.row_offset(t) : -1;
    const bool ok = off >= 0;
    off = ok ? off + col * 16 : 0;
    u32x4 kw = {0u, 0u, 0u, 0u}, vw = {0u, 0u, 0u, 0u};
    if (ok) {
      kw = load_vec<u32x4>(kv.kbase + off);
      vw = load_vec<u32x4>(kv.vbase + off);
    }
    const T *ke = (const T *)&kw;
    const T *ve = (const T *)&vw;
    float kf[VEC], vf[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      kf[v] = to_f32(ke[v]);
      vf[v] = to_f32(ve[v]);
    }
    // Rows g >= ng are skipped by a guard, not a break: a loop with one exit
    // and a constant trip count unrolls, which keeps the per-row arrays in
    // registers.
#pragma unroll
    for (int g = 0; g < GM; ++g) {
      if (g < ng) {
        float sc = 0.f;
#pragma unroll
        for (int v = 0; v < VEC; ++v) sc += qf[g][v] * kf[v];
#pragma unroll
        for (int o2 = 1; o2 < LPT; o2 <<= 1) sc += shfl_xor(sc, o2);
        const float x = ok ? sc * scale_log2 : kNegInf;
        const float m_new = fmaxf(m[g], x);
        const float msub = (m_new == kNegInf) ? 0.f : m_new;
        const float a = fast_exp2(m[g] - msub);
        const float pr = fast_exp2(x - msub);
        l[g] = l[g] * a + pr;
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[g][v] = acc[g][v] * a + pr * vf[v];
        m[g] = m_new;
      }
    }
  }

  // Merge the TPI token rows of the wave (lanes that share `col`).
#pragma unroll
  for (int off = LPT; off < 64; off <<= 1) {
#pragma unroll
    for (int g = 0; g < GM; ++g) {
      if (g < ng) {
        const float m2 = shfl_xor(m[g], off);
        const float l2 = shfl_xor(l[g], off);
        const float M = fmaxf(m[g], m2);
        const float Msub = (M == kNegInf) ? 0.f : M;
        const float a1 = fast_exp2(m[g] - Msub);
        const float a2 = fast_exp2(m2 - Msub);
        l[g] = l[g] * a1 + l2 * a2;
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          const float o2 = shfl_xor(acc[g][v], off);
          acc[g][v] = acc[g][v] * a1 + o2 * a2;
        }
        m[g] = M;
      }
    }
  }
  if (row == 0) {
#pragma unroll
    for (int g = 0; g < GM; ++g) {
      if (col == 0) {
        sm.m[wave][g] = m[g];
        sm.l[wave][g] = l[g];
      }
#pragma unroll
      for (int v = 0; v < VEC; ++v) sm.o[wave][g][col * VEC + v] = acc[g][v];
    }
  }
}

}  // namespace clv
