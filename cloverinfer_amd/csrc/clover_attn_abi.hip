// clover_attn_abi.hip - the extern "C" boundary declared in include/clover_attn.h.
//
// Validates every argument block, turns it into the kernels' parameter
// structs and dispatches. Nothing here allocates device memory; the only
// state kept between calls is per-device: the compute-unit count and the
// address of the fixed scratch array of clv_paged_decode_balanced_noalloc.
// Errors come back as status codes.
#include <math.h>
#include <stddef.h>
#include <stdlib.h>

#include <atomic>
#include <mutex>

#include "clover_attn.h"
#include "clv_internal.h"

namespace {

using clv::DType;

bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

int log2_int(int64_t x) {
  int r = 0;
  while ((int64_t(1) << r) < x) ++r;
  return r;
}

bool supported_head_dim(int d) {
  return d == 8 || d == 16 || d == 32 || d == 64 || d == 128 || d == 256;
}

int elem_bytes(int dtype) { return dtype == CLV_F32 ? 4 : 2; }

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

bool stride16(int64_t stride, int eb) { return (stride * eb) % 16 == 0; }

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

size_t round256(size_t x) { return (x + 255) & ~(size_t)255; }

// Compute units of the current device, queried once per device and cached
// (the default wave counts depend on it). 0 is "not queried yet"; a failed
// query answers 256 (MI355X) without caching.
constexpr int kMaxDevices = 64;
std::atomic<int> g_device_cus[kMaxDevices];

int device_compute_units() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < kMaxDevices) {
    const int c = g_device_cus[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    return 256;
  if (dev < kMaxDevices) g_device_cus[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

// Fixed scratch of clv_paged_decode_balanced_noalloc: the balanced decode's
// workspace (segment prefix sums and per-wave partials) for callers that
// cannot allocate. Every GPU the library runs on holds one copy for the life
// of the process. In host code `scratch` names a host-side stand-in, never
// the device array: only the address hipGetSymbolAddress returns for the
// current device (scratch_address) may reach a kernel.
static __device__ __align__(256) unsigned char scratch[CLV_NOALLOC_SCRATCH_BYTES];

std::atomic<void *> g_scratch_dev[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of the current device's scratch array, looked up once per
// device (with that device current) and kept; CLV_ELAUNCH if the runtime
// cannot resolve it.
int scratch_address(void **out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return CLV_ELAUNCH;
  void *ptr = g_scratch_dev[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ptr = g_scratch_dev[dev].load(std::memory_order_relaxed);
    if (ptr == nullptr) {
      if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr)
        return CLV_ELAUNCH;
      g_scratch_dev[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return CLV_OK;
}

// Validates a decode argument block and fills the kernel parameters.
int fill_decode(const clv_decode_args *a, clv::DecodeParams *p) {
  if (a == nullptr) return CLV_EINVAL;
  if (a->dtype != CLV_F32 && a->dtype != CLV_F16 && a->dtype != CLV_BF16) return CLV_EINVAL;
  if (a->num_seqs < 0 || a->num_heads <= 0 || a->num_kv_heads <= 0 || a->head_dim <= 0)
    return CLV_EINVAL;
  if (a->num_heads % a->num_kv_heads != 0) return CLV_EINVAL;
  if (!is_pow2(a->block_size)) return CLV_EUNSUPPORTED;
  if (!supported_head_dim(a->head_dim)) return CLV_EUNSUPPORTED;
  if (a->max_blocks_per_seq < 0 || a->max_context_len < 0 || a->num_blocks <= 0) return CLV_EINVAL;
  if (!isfinite(a->scale)) return CLV_EINVAL;
  if (a->num_seqs > 65535) return CLV_EUNSUPPORTED;  // grid z limit
  const int eb = elem_bytes(a->dtype);
  if (a->num_seqs > 0) {
    if (!a->out || !a->q || !a->k_cache || !a->v_cache || !a->context_lens) return CLV_EINVAL;
    if (a->max_blocks_per_seq > 0 && !a->block_tables) return CLV_EINVAL;
    if (!aligned16(a->out) || !aligned16(a->q) || !aligned16(a->k_cache) || !aligned16(a->v_cache))
      return CLV_EINVAL;
    if (!stride16(a->q_stride_seq, eb) || !stride16(a->q_stride_head, eb) ||
        !stride16(a->out_stride_seq, eb) || !stride16(a->out_stride_head, eb) ||
        !stride16(a->kv_stride_block, eb) || !stride16(a->kv_stride_token, eb) ||
        !stride16(a->kv_stride_head, eb))
      return CLV_EINVAL;
  }
  *p = clv::DecodeParams{};
  p->out = a->out;
  p->q = a->q;
  p->k_cache = a->k_cache;
  p->v_cache = a->v_cache;
  p->block_tables = a->block_tables;
  p->context_lens = a->context_lens;
  p->q_stride_seq = a->q_stride_seq;
  p->q_stride_head = a->q_stride_head;
  p->out_stride_seq = a->out_stride_seq;
  p->out_stride_head = a->out_stride_head;
  p->kv_stride_block = a->kv_stride_block;
  p->kv_stride_token = a->kv_stride_token;
  p->kv_stride_head = a->kv_stride_head;
  p->num_seqs = a->num_seqs;
  p->num_heads = a->num_heads;
  p->num_kv_heads = a->num_kv_heads;
  p->head_dim = a->head_dim;
  p->group = a->num_heads / a->num_kv_heads;
  p->n_gchunks = (int32_t)ceil_div(p->group, 16);
  p->block_shift = log2_int(a->block_size);
  p->max_blocks_per_seq = a->max_blocks_per_seq;
  p->max_context_len = a->max_context_len;
  p->num_blocks = a->num_blocks;
  p->scale_log2 = a->scale * 1.4426950408889634f;
  return CLV_OK;
}

// Longest context for which clv_paged_decode_append runs the single pass
// (the schedule the Python layer picks for such batches: no merge launch).
constexpr int32_t kAppendSinglePassMaxLen = 512;

int launch_decode(const clv::DecodeParams &p, int dtype, int block_size, hipStream_t stream) {
  const DType dt = (DType)dtype;
  hipError_t err;
  if (clv::decode_mfma_supported(dt, p.head_dim, block_size))
    err = clv::launch_decode_mfma(p, dt, stream);
  else
    err = clv::launch_decode_valu(p, dt, stream);
  return err == hipSuccess ? CLV_OK : CLV_ELAUNCH;
}

}  // namespace

extern "C" {

int clv_abi_version(void) { return CLV_ABI_VERSION; }

const char *clv_status_string(int status) {
  switch (status) {
    case CLV_OK: return "ok";
    case CLV_EINVAL: return "invalid argument (shape, stride, alignment, pointer or dtype)";
    case CLV_EUNSUPPORTED: return "unsupported configuration (head_dim, block_size or size limit)";
    case CLV_ELAUNCH: return "kernel launch failed";
    case CLV_EWORKSPACE: return "split-K workspace missing, misaligned or too small";
    case CLV_ESCRATCH:
      return "problem needs more than the fixed scratch of the no-allocation entry point "
             "(CLV_NOALLOC_SCRATCH_BYTES)";
    default: return "unknown status";
  }
}

int clv_reshape_and_cache(const clv_cache_args *a, clv_stream_t stream) {
  if (a == nullptr) return CLV_EINVAL;
  if (a->dtype != CLV_F32 && a->dtype != CLV_F16 && a->dtype != CLV_BF16) return CLV_EINVAL;
  if (a->num_tokens < 0 || a->num_kv_heads <= 0 || a->head_dim <= 0 || a->num_blocks <= 0)
    return CLV_EINVAL;
  if (!is_pow2(a->block_size)) return CLV_EUNSUPPORTED;
  if (a->num_tokens == 0) return CLV_OK;
  if (!a->key || !a->value || !a->k_cache || !a->v_cache || !a->slot_mapping) return CLV_EINVAL;
  clv::CacheParams p{};
  p.key = a->key;
  p.value = a->value;
  p.k_cache = a->k_cache;
  p.v_cache = a->v_cache;
  p.slot_mapping = a->slot_mapping;
  p.key_stride_token = a->key_stride_token;
  p.key_stride_head = a->key_stride_head;
  p.value_stride_token = a->value_stride_token;
  p.value_stride_head = a->value_stride_head;
  p.kv_stride_block = a->kv_stride_block;
  p.kv_stride_token = a->kv_stride_token;
  p.kv_stride_head = a->kv_stride_head;
  p.num_tokens = a->num_tokens;
  p.num_kv_heads = a->num_kv_heads;
  p.head_dim = a->head_dim;
  p.block_shift = log2_int(a->block_size);
  p.num_blocks = a->num_blocks;
  p.num_slots = (int64_t)a->num_blocks * a->block_size;
  p.elem_bytes = elem_bytes(a->dtype);
  return clv::launch_reshape_and_cache(p, (hipStream_t)stream) == hipSuccess ? CLV_OK
                                                                              : CLV_ELAUNCH;
}

int clv_reshape_and_cache_fp8(const clv_cache_args *a, const float *k_scales,
                              const float *v_scales, clv_stream_t stream) {
  if (a == nullptr) return CLV_EINVAL;
  if (a->dtype != CLV_F32 && a->dtype != CLV_F16 && a->dtype != CLV_BF16) return CLV_EINVAL;
  if (a->num_tokens < 0 || a->num_kv_heads <= 0 || a->head_dim <= 0 || a->num_blocks <= 0)
    return CLV_EINVAL;
  if (!is_pow2(a->block_size)) return CLV_EUNSUPPORTED;
  if (a->head_dim % 8 != 0) return CLV_EUNSUPPORTED;
  if (a->num_tokens == 0) return CLV_OK;
  if (!a->key || !a->value || !a->k_cache || !a->v_cache || !a->slot_mapping || !k_scales ||
      !v_scales)
    return CLV_EINVAL;
  // fp8 pools: one byte per element, rows written 8 bytes at a time.
  if (((uintptr_t)a->k_cache & 7u) || ((uintptr_t)a->v_cache & 7u) || (a->kv_stride_block & 7) ||
      (a->kv_stride_token & 7) || (a->kv_stride_head & 7))
    return CLV_EINVAL;
  clv::CacheParams p{};
  p.key = a->key;
  p.value = a->value;
  p.k_cache = a->k_cache;
  p.v_cache = a->v_cache;
  p.slot_mapping = a->slot_mapping;
  p.key_stride_token = a->key_stride_token;
  p.key_stride_head = a->key_stride_head;
  p.value_stride_token = a->value_stride_token;
  p.value_stride_head = a->value_stride_head;
  p.kv_stride_block = a->kv_stride_block;
  p.kv_stride_token = a->kv_stride_token;
  p.kv_stride_head = a->kv_stride_head;
  p.num_tokens = a->num_tokens;
  p.num_kv_heads = a->num_kv_heads;
  p.head_dim = a->head_dim;
  p.block_shift = log2_int(a->block_size);
  p.num_blocks = a->num_blocks;
  p.num_slots = (int64_t)a->num_blocks * a->block_size;
  p.elem_bytes = elem_bytes(a->dtype);
  return clv::launch_reshape_and_cache_fp8(p, a->dtype, k_scales, v_scales, (hipStream_t)stream) ==
                 hipSuccess
             ? CLV_OK
             : CLV_ELAUNCH;
}

int clv_paged_decode(const clv_decode_args *a, clv_stream_t stream) {
  clv::DecodeParams p;
  const int st = fill_decode(a, &p);
  if (st != CLV_OK) return st;
  if (p.num_seqs == 0) return CLV_OK;
  p.partition_size = 0;
  return launch_decode(p, a->dtype, a->block_size, (hipStream_t)stream);
}

size_t clv_splitk_workspace_bytes(int32_t num_seqs, int32_t num_heads, int32_t head_dim,
                                  int32_t max_context_len, int32_t partition_size) {
  if (num_seqs <= 0 || num_heads <= 0 || head_dim <= 0 || partition_size <= 0 ||
      max_context_len < 0)
    return 0;
  const size_t parts = (size_t)(max_context_len > 0 ? ceil_div(max_context_len, partition_size) : 1);
  const size_t rows = (size_t)num_seqs * (size_t)num_heads * parts;
  return round256(rows * (size_t)head_dim * 4) + 2 * round256(rows * 4);
}

}  // extern "C"

namespace {

// Fills the split-K fields of p from the workspace; CLV_OK or an error.
int head_group(int num_kv_heads, int num_waves);
int stream_depth_setting(int def);

int fill_splitk(const clv_decode_args *a, int32_t partition_size, const void *workspace,
                size_t workspace_bytes, clv::DecodeParams *p) {
  if (partition_size <= 0 || partition_size % 32 != 0) return CLV_EINVAL;
  const size_t need = clv_splitk_workspace_bytes(a->num_seqs, a->num_heads, a->head_dim,
                                                 a->max_context_len, partition_size);
  if (workspace == nullptr || workspace_bytes < need || ((uintptr_t)workspace & 255u) != 0)
    return CLV_EWORKSPACE;
  const int64_t parts = a->max_context_len > 0 ? ceil_div(a->max_context_len, partition_size) : 1;
  if (parts > 65535) return CLV_EUNSUPPORTED;
  const size_t rows = (size_t)a->num_seqs * (size_t)a->num_heads * (size_t)parts;
  char *ws = (char *)workspace;
  p->partition_size = partition_size;
  p->max_parts = (int32_t)parts;
  p->ws_o = (float *)ws;
  p->ws_m = (float *)(ws + round256(rows * (size_t)a->head_dim * 4));
  p->ws_l = (float *)(ws + round256(rows * (size_t)a->head_dim * 4) + round256(rows * 4));
  return CLV_OK;
}

}  // namespace

extern "C" {

int clv_paged_decode_partials(const clv_decode_args *a, int32_t partition_size, void *workspace,
                              size_t workspace_bytes, clv_stream_t stream) {
  clv::DecodeParams p;
  int st = fill_decode(a, &p);
  if (st != CLV_OK) return st;
  if (p.num_seqs == 0) return partition_size > 0 && partition_size % 32 == 0 ? CLV_OK : CLV_EINVAL;
  st = fill_splitk(a, partition_size, workspace, workspace_bytes, &p);
  if (st != CLV_OK) return st;
  // The partitions on the balanced stream kernel where it covers the shape:
  // its waves split the batch's partitions evenly and stream each run of
  // consecutive partitions through one ring (16 x 32K-token fp16, partition
  // 512: 339 -> 316 us), writing the same partials as the grid kernel below.
  const int64_t nseg = (int64_t)p.num_seqs * p.num_kv_heads * p.n_gchunks;
  if (clv::decode_stream_supported((DType)a->dtype, a->head_dim, a->block_size, nseg)) {
    const int nw = clv_default_num_waves();
    const int hg = head_group(p.num_kv_heads, nw);
    p.num_waves = nw;
    p.head_group = hg;
    p.stream_depth = stream_depth_setting(a->dtype == CLV_F32 ? 2 : 3);
    p.stream_run_cost = 0;
    p.num_segments = (int32_t)(nseg / hg);
    return clv::launch_decode_stream(p, (DType)a->dtype, (hipStream_t)stream) == hipSuccess
               ? CLV_OK
               : CLV_ELAUNCH;
  }
  return launch_decode(p, a->dtype, a->block_size, (hipStream_t)stream);
}

int clv_splitk_reduce(const clv_decode_args *a, int32_t partition_size, const void *workspace,
                      size_t workspace_bytes, clv_stream_t stream) {
  clv::DecodeParams p;
  int st = fill_decode(a, &p);
  if (st != CLV_OK) return st;
  if (p.num_seqs == 0) return partition_size > 0 && partition_size % 32 == 0 ? CLV_OK : CLV_EINVAL;
  st = fill_splitk(a, partition_size, workspace, workspace_bytes, &p);
  if (st != CLV_OK) return st;
  return clv::launch_splitk_reduce(p, (DType)a->dtype, (hipStream_t)stream) == hipSuccess
             ? CLV_OK
             : CLV_ELAUNCH;
}

int clv_paged_decode_splitk(const clv_decode_args *a, int32_t partition_size, void *workspace,
                            size_t workspace_bytes, clv_stream_t stream) {
  clv::DecodeParams p;
  const int st = fill_decode(a, &p);
  if (st != CLV_OK) return st;
  if (partition_size <= 0 || partition_size % 32 != 0) return CLV_EINVAL;
  if (p.num_seqs == 0) return CLV_OK;
  // A context that fits one partition needs no merge.
  if (a->max_context_len <= partition_size) {
    p.partition_size = 0;
    return launch_decode(p, a->dtype, a->block_size, (hipStream_t)stream);
  }
  const int rc = clv_paged_decode_partials(a, partition_size, workspace, workspace_bytes, stream);
  if (rc != CLV_OK) return rc;
  return clv_splitk_reduce(a, partition_size, workspace, workspace_bytes, stream);
}

int32_t clv_default_num_waves(void) {
  // One wave per SIMD (4 per compute unit), each keeping three steps of
  // loads in flight: on MI355X this streams the paged cache faster than more
  // waves with shallower pipelines.
  return device_compute_units() * 4;
}

int32_t clv_default_num_waves_fp8(void) { return 2 * clv_default_num_waves(); }

size_t clv_balanced_workspace_bytes(int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                                    int32_t head_dim, int32_t num_waves) {
  if (num_seqs <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 ||
      num_heads % num_kv_heads != 0)
    return 0;
  if (num_waves <= 0) num_waves = clv_default_num_waves();
  const int64_t group = num_heads / num_kv_heads;
  const size_t nseg = (size_t)num_seqs * (size_t)num_kv_heads * (size_t)ceil_div(group, 16);
  const size_t rows = ((size_t)num_waves + nseg) * 16;
  return round256((nseg + 1) * 4) + 2 * round256(rows * 4) + round256(rows * (size_t)head_dim * 4);
}

}  // extern "C"

namespace {

// Ring depth of the balanced decode: steps of loads each wave keeps in
// flight (2, 3, 4 or 6): three for 16-bit and fp8 pools, two for fp32 pools
// (twice the bytes per step). Fixed at build time; a tuning build may set
// CLV_STREAM_DEPTH (a preprocessor value) to force one depth for every dtype.
int stream_depth_setting(int def) {
#ifdef CLV_STREAM_DEPTH
  (void)def;
  static_assert(CLV_STREAM_DEPTH == 2 || CLV_STREAM_DEPTH == 3 || CLV_STREAM_DEPTH == 4 ||
                    CLV_STREAM_DEPTH == 6,
                "ring depth 2, 3, 4 or 6");
  return CLV_STREAM_DEPTH;
#else
  return def;
#endif
}

// Phantom steps the balanced decode charges for each segment a wave starts
// (a run start costs one memory latency: measured per-wave durations grow by
// ~2.5 us per extra run). With head groups 4 measured best (GQA-7B batch:
// 172.9 us at 2, 172.3 at 4, 173.5 at 6, 173.9 at 8). Fixed at build time
// (preprocessor value CLV_STREAM_RUN_COST, default 4).
#ifndef CLV_STREAM_RUN_COST
#define CLV_STREAM_RUN_COST 4
#endif
static_assert(CLV_STREAM_RUN_COST >= 0 && CLV_STREAM_RUN_COST <= 64, "run cost 0..64 steps");
constexpr int kStreamRunCost = CLV_STREAM_RUN_COST;

// Steps per group of each dispatch slot of the balanced decode, times 256
// against the last slot, when the grid is two or three workgroups (of four
// waves) per compute unit (see StreamSplit in decode_stream.hip); all 256 is
// the even split. fp8 GQA-7B batch, wave end times read from the realtime
// counter: at 2048 waves and equal spans the second-slot waves end 5.3 us
// after the first-slot ones on average; at 282 (1.10) both slots end within
// 0.5 us of each other, the launch span falls from 87.5 to 86.7 us and
// back-to-back launches from 91.2-92.0 to 89.3-90.3 us (320 and 345: slower
// than 256). At 3072 waves the three slots end at 71.6, 78.8 and 86.4 us on
// average with equal spans; back to back (another box): 99.3-99.6 us at
// 256/256, 98.0-98.7 at 282/269, 96.7-97.1 at 300/278, 96.1-96.2 at
// 320/288, 96.4-96.8 at 345/300 (2048 waves there: 95.4-96.3, and per step
// 0.0981 against 0.1045 ms, the merge reading more partials, so the fp8
// default stays at two slots). Fixed at build time (preprocessor values
// CLV_STREAM_SLOT2_Q8 for the first of two slots, CLV_STREAM_SLOT3_Q8_0 and
// _1 for the first two of three).
#ifndef CLV_STREAM_SLOT2_Q8
#define CLV_STREAM_SLOT2_Q8 282
#endif
#ifndef CLV_STREAM_SLOT3_Q8_0
#define CLV_STREAM_SLOT3_Q8_0 320
#endif
#ifndef CLV_STREAM_SLOT3_Q8_1
#define CLV_STREAM_SLOT3_Q8_1 288
#endif
static_assert(CLV_STREAM_SLOT2_Q8 >= 128 && CLV_STREAM_SLOT2_Q8 <= 512 &&
                  CLV_STREAM_SLOT3_Q8_0 >= 128 && CLV_STREAM_SLOT3_Q8_0 <= 512 &&
                  CLV_STREAM_SLOT3_Q8_1 >= 128 && CLV_STREAM_SLOT3_Q8_1 <= 512,
              "slot weights 0.5..2");
constexpr int kSlotQ8[2][3] = {{CLV_STREAM_SLOT2_Q8, 256, 256},
                               {CLV_STREAM_SLOT3_Q8_0, CLV_STREAM_SLOT3_Q8_1, 256}};

// kv heads that one workgroup of the balanced decode reads together (one
// wave each): all of them up to four (a token's whole row of the pools; GQA-7B
// batch, 4 kv heads: 175.3 -> 173.1 us), else pairs (MHA Llama-7B batch, 32
// kv heads: 329.0 -> 326.9 us with pairs, 336.4 with fours). A tuning build
// may cap the group with the preprocessor value CLV_HEAD_GROUP_MAX.
#ifndef CLV_HEAD_GROUP_MAX
#define CLV_HEAD_GROUP_MAX 4
#endif
static_assert(CLV_HEAD_GROUP_MAX == 1 || CLV_HEAD_GROUP_MAX == 2 || CLV_HEAD_GROUP_MAX == 4,
              "head group 1, 2 or 4");
int head_group(int num_kv_heads, int num_waves) {
  int hg = num_kv_heads <= 4 ? num_kv_heads : 2;
  hg = std::min(hg, CLV_HEAD_GROUP_MAX);
  if (hg == 3 || num_kv_heads % hg != 0) hg = 1;
  while (hg > num_waves) hg /= 2;
  return std::max(hg, 1);
}

// Validates a balanced-decode call and lays the workspace out in p.
int fill_balanced(const clv_decode_args *a, int32_t num_waves, void *workspace,
                  size_t workspace_bytes, clv::DecodeParams *p) {
  const int st = fill_decode(a, p);
  if (st != CLV_OK) return st;
  if (num_waves <= 0) num_waves = clv_default_num_waves();
  if (num_waves > (1 << 22)) return CLV_EINVAL;
  const int64_t nseg = (int64_t)p->num_seqs * p->num_kv_heads * p->n_gchunks;
  const int hg = head_group(p->num_kv_heads, num_waves);
  if (!clv::decode_stream_supported((DType)a->dtype, a->head_dim, a->block_size, nseg))
    return CLV_EUNSUPPORTED;
  if (p->num_seqs == 0) return CLV_OK;
  const size_t need = clv_balanced_workspace_bytes(a->num_seqs, a->num_heads, a->num_kv_heads,
                                                   a->head_dim, num_waves);
  if (workspace == nullptr || workspace_bytes < need || ((uintptr_t)workspace & 255u) != 0)
    return CLV_EWORKSPACE;
  const size_t rows = ((size_t)num_waves + (size_t)nseg) * 16;
  char *ws = (char *)workspace;
  p->num_waves = num_waves;
  p->head_group = hg;
  // fp32 steps are twice the bytes: two steps in flight (a sweep over 2-4).
  p->stream_depth = stream_depth_setting(a->dtype == CLV_F32 ? 2 : 3);
  p->stream_run_cost = kStreamRunCost;
  p->num_segments = (int32_t)(nseg / hg);
  // Two or three workgroups (of four waves) per compute unit: one piece of
  // the split per dispatch slot, the older slots taking more steps
  // (decode_stream.hip, StreamSplit). Partials and merge derive the same
  // split from num_waves.
  const int cus = device_compute_units();
  for (int slots = 2; slots <= 3; ++slots) {
    if (num_waves != slots * 4 * cus) continue;
    p->slot_count = slots;
    p->slot_groups = 4 * cus / hg;
    for (int k = 0; k < slots; ++k) p->slot_q8[k] = kSlotQ8[slots - 2][k];
  }
  p->seg_prefix = (int32_t *)ws;
  ws += round256(((size_t)nseg + 1) * 4);
  p->ws_m = (float *)ws;
  ws += round256(rows * 4);
  p->ws_l = (float *)ws;
  ws += round256(rows * 4);
  p->ws_o = (float *)ws;
  return CLV_OK;
}

}  // namespace

extern "C" {

int clv_balanced_partials(const clv_decode_args *a, int32_t num_waves, void *workspace,
                          size_t workspace_bytes, clv_stream_t stream) {
  clv::DecodeParams p;
  const int st = fill_balanced(a, num_waves, workspace, workspace_bytes, &p);
  if (st != CLV_OK || p.num_seqs == 0) return st;
  return clv::launch_decode_stream(p, (DType)a->dtype, (hipStream_t)stream) == hipSuccess
             ? CLV_OK
             : CLV_ELAUNCH;
}

int clv_balanced_reduce(const clv_decode_args *a, int32_t num_waves, const void *workspace,
                        size_t workspace_bytes, clv_stream_t stream) {
  clv::DecodeParams p;
  const int st = fill_balanced(a, num_waves, const_cast<void *>(workspace), workspace_bytes, &p);
  if (st != CLV_OK || p.num_seqs == 0) return st;
  return clv::launch_stream_reduce(p, (DType)a->dtype, (hipStream_t)stream) == hipSuccess
             ? CLV_OK
             : CLV_ELAUNCH;
}

int clv_paged_decode_balanced(const clv_decode_args *a, int32_t num_waves, void *workspace,
                              size_t workspace_bytes, clv_stream_t stream) {
  const int rc = clv_balanced_partials(a, num_waves, workspace, workspace_bytes, stream);
  if (rc != CLV_OK) return rc;
  return clv_balanced_reduce(a, num_waves, workspace, workspace_bytes, stream);
}

int clv_paged_decode_balanced_noalloc(const clv_decode_args *a, int32_t num_waves,
                                      clv_stream_t stream) {
  if (a == nullptr) return CLV_EINVAL;
  if (num_waves <= 0) num_waves = clv_default_num_waves();
  // 0 for arguments the balanced decode refuses anyway (it reports them).
  const size_t need = clv_balanced_workspace_bytes(a->num_seqs, a->num_heads, a->num_kv_heads,
                                                   a->head_dim, num_waves);
  if (need > (size_t)CLV_NOALLOC_SCRATCH_BYTES) return CLV_ESCRATCH;
  void *ws = nullptr;
  if (need > 0 && a->num_seqs > 0) {
    const int st = scratch_address(&ws);
    if (st != CLV_OK) return st;
  }
  // The stream kernel writes the prefix sums and every partial the merge
  // reads before it reads them: nothing in the scratch has to start at zero.
  return clv_paged_decode_balanced(a, num_waves, ws, (size_t)CLV_NOALLOC_SCRATCH_BYTES, stream);
}

int clv_paged_decode_append(const clv_decode_args *a, const void *key_new, const void *value_new,
                            int64_t new_stride_seq, int64_t new_stride_head, int32_t num_waves,
                            void *workspace, size_t workspace_bytes, clv_stream_t stream) {
  clv::DecodeParams p;
  // Short contexts (the single-pass schedule's range) with at most 16 query
  // heads per kv head: one grid launch that appends and attends, no merge.
  if (a != nullptr && num_waves <= 0 && a->max_context_len <= kAppendSinglePassMaxLen &&
      a->num_kv_heads > 0 && a->num_heads % a->num_kv_heads == 0 &&
      a->num_heads / a->num_kv_heads <= 16 &&
      clv::decode_mfma_supported((DType)a->dtype, a->head_dim, a->block_size)) {
    const int st = fill_decode(a, &p);
    if (st != CLV_OK || p.num_seqs == 0) return st;
    const int eb = elem_bytes(a->dtype);
    if (!key_new || !value_new || !aligned16(key_new) || !aligned16(value_new) ||
        !stride16(new_stride_seq, eb) || !stride16(new_stride_head, eb))
      return CLV_EINVAL;
    p.partition_size = 0;
    p.key_new = key_new;
    p.value_new = value_new;
    p.new_stride_seq = new_stride_seq;
    p.new_stride_head = new_stride_head;
    return clv::launch_decode_mfma_append(p, (DType)a->dtype, (hipStream_t)stream) == hipSuccess
               ? CLV_OK
               : CLV_ELAUNCH;
  }
  const int st = fill_balanced(a, num_waves, workspace, workspace_bytes, &p);
  if (st != CLV_OK || p.num_seqs == 0) return st;
  const int eb = elem_bytes(a->dtype);
  if (!key_new || !value_new || !aligned16(key_new) || !aligned16(value_new) ||
      !stride16(new_stride_seq, eb) || !stride16(new_stride_head, eb))
    return CLV_EINVAL;
  p.key_new = key_new;
  p.value_new = value_new;
  p.new_stride_seq = new_stride_seq;
  p.new_stride_head = new_stride_head;
  const hipStream_t s = (hipStream_t)stream;
  if (clv::stream_appends_in_kernel((DType)a->dtype, a->head_dim, a->block_size, p.group)) {
    p.append_new = 1;
  } else if (clv::launch_append_by_table(p, eb, s) != hipSuccess) {
    return CLV_ELAUNCH;
  }
  if (clv::launch_decode_stream(p, (DType)a->dtype, s) != hipSuccess) return CLV_ELAUNCH;
  return clv::launch_stream_reduce(p, (DType)a->dtype, s) == hipSuccess ? CLV_OK : CLV_ELAUNCH;
}

int clv_balanced_reduce_append(const clv_decode_args *a, const void *key_new,
                               const void *value_new, int64_t new_stride_seq,
                               int64_t new_stride_head, const int64_t *slot_mapping,
                               int32_t num_waves, const void *workspace, size_t workspace_bytes,
                               clv_stream_t stream) {
  clv::DecodeParams p;
  const int st = fill_balanced(a, num_waves, const_cast<void *>(workspace), workspace_bytes, &p);
  if (st != CLV_OK || p.num_seqs == 0) return st;
  const int eb = elem_bytes(a->dtype);
  if (!key_new || !value_new || !slot_mapping || !aligned16(key_new) || !aligned16(value_new) ||
      !stride16(new_stride_seq, eb) || !stride16(new_stride_head, eb))
    return CLV_EINVAL;
  p.key_new = key_new;
  p.value_new = value_new;
  p.new_stride_seq = new_stride_seq;
  p.new_stride_head = new_stride_head;
  p.slot_mapping = slot_mapping;
  return clv::launch_stream_reduce_append(p, (DType)a->dtype, (hipStream_t)stream) == hipSuccess
             ? CLV_OK
             : CLV_ELAUNCH;
}

int clv_paged_decode_fp8(const clv_decode_args *a, const float *k_scales, const float *v_scales,
                         int32_t num_waves, void *workspace, size_t workspace_bytes,
                         clv_stream_t stream) {
  if (num_waves <= 0) num_waves = clv_default_num_waves_fp8();
  const int rc = clv_paged_decode_fp8_partials(a, k_scales, v_scales, num_waves, workspace,
                                               workspace_bytes, stream);
  if (rc != CLV_OK) return rc;
  return clv_balanced_reduce(a, num_waves, workspace, workspace_bytes, stream);
}

int clv_paged_decode_fp8_partials(const clv_decode_args *a, const float *k_scales,
                                  const float *v_scales, int32_t num_waves, void *workspace,
                                  size_t workspace_bytes, clv_stream_t stream) {
  if (a == nullptr) return CLV_EINVAL;
  if (a->dtype != CLV_F16 && a->dtype != CLV_BF16) return CLV_EINVAL;
  if (a->head_dim != 128 || a->block_size < 16) return CLV_EUNSUPPORTED;
  // The wave count sets the partial layout that clv_balanced_reduce reads,
  // whose own default differs: it must be explicit here.
  if (num_waves <= 0) return CLV_EINVAL;
  clv::DecodeParams p;
  const int st = fill_balanced(a, num_waves, workspace, workspace_bytes, &p);
  if (st != CLV_OK || p.num_seqs == 0) return st;
  if (!k_scales || !v_scales) return CLV_EINVAL;
  // fp8 pools: strides are bytes; each lane reads 8-byte row chunks.
  if ((a->kv_stride_block & 15) || (a->kv_stride_token & 15) || (a->kv_stride_head & 15))
    return CLV_EINVAL;
  // Half the bytes per step make the per-step compute the longer part: two
  // waves per SIMD (clv_default_num_waves_fp8) with three steps in flight
  // (GQA-7B batch: step 0.0979 ms at depth 3, 0.0991 at depth 4; 2560 or
  // 3072 waves at depth 3, 3072 or 4096 at depth 2: slower).
  p.stream_depth = stream_depth_setting(3);
  p.kv_fp8 = 1;
  p.k_scales = k_scales;
  p.v_scales = v_scales;
  return clv::launch_decode_stream(p, (DType)a->dtype, (hipStream_t)stream) == hipSuccess
             ? CLV_OK
             : CLV_ELAUNCH;
}

int clv_chunked_prefill(const clv_prefill_args *a, clv_stream_t stream) {
  if (a == nullptr) return CLV_EINVAL;
  if (a->dtype != CLV_F32 && a->dtype != CLV_F16 && a->dtype != CLV_BF16) return CLV_EINVAL;
  if (a->num_seqs < 0 || a->num_tokens < 0 || a->num_heads <= 0 || a->num_kv_heads <= 0 ||
      a->head_dim <= 0 || a->num_blocks <= 0 || a->max_blocks_per_seq < 0 || a->max_query_len < 0)
    return CLV_EINVAL;
  if (a->num_heads % a->num_kv_heads != 0) return CLV_EINVAL;
  if (!is_pow2(a->block_size)) return CLV_EUNSUPPORTED;
  if (!supported_head_dim(a->head_dim)) return CLV_EUNSUPPORTED;
  if (!isfinite(a->scale)) return CLV_EINVAL;
  if (a->num_seqs > 65535) return CLV_EUNSUPPORTED;
  if (a->num_seqs == 0 || a->num_tokens == 0) return CLV_OK;
  const int eb = elem_bytes(a->dtype);
  if (!a->out || !a->q || !a->k_cache || !a->v_cache || !a->context_lens || !a->query_start_loc)
    return CLV_EINVAL;
  if (a->max_blocks_per_seq > 0 && !a->block_tables) return CLV_EINVAL;
  if (!aligned16(a->out) || !aligned16(a->q) || !aligned16(a->k_cache) || !aligned16(a->v_cache))
    return CLV_EINVAL;
  if (!stride16(a->q_stride_token, eb) || !stride16(a->q_stride_head, eb) ||
      !stride16(a->out_stride_token, eb) || !stride16(a->out_stride_head, eb) ||
      !stride16(a->kv_stride_block, eb) || !stride16(a->kv_stride_token, eb) ||
      !stride16(a->kv_stride_head, eb))
    return CLV_EINVAL;
  clv::PrefillParams p{};
  p.out = a->out;
  p.q = a->q;
  p.k_cache = a->k_cache;
  p.v_cache = a->v_cache;
  p.block_tables = a->block_tables;
  p.context_lens = a->context_lens;
  p.query_start_loc = a->query_start_loc;
  p.q_stride_token = a->q_stride_token;
  p.q_stride_head = a->q_stride_head;
  p.out_stride_token = a->out_stride_token;
  p.out_stride_head = a->out_stride_head;
  p.kv_stride_block = a->kv_stride_block;
  p.kv_stride_token = a->kv_stride_token;
  p.kv_stride_head = a->kv_stride_head;
  p.num_seqs = a->num_seqs;
  p.num_tokens = a->num_tokens;
  p.num_heads = a->num_heads;
  p.num_kv_heads = a->num_kv_heads;
  p.head_dim = a->head_dim;
  p.group = a->num_heads / a->num_kv_heads;
  p.block_shift = log2_int(a->block_size);
  p.max_blocks_per_seq = a->max_blocks_per_seq;
  p.max_query_len = a->max_query_len;
  p.num_blocks = a->num_blocks;
  p.scale_log2 = a->scale * 1.4426950408889634f;
  p.cus_per_xcd = device_compute_units() / 8;
  const DType dt = (DType)a->dtype;
  hipError_t err;
  if (clv::prefill_mfma_supported(dt, a->head_dim, a->block_size))
    err = clv::launch_prefill_mfma(p, dt, (hipStream_t)stream);
  else
    err = clv::launch_prefill_valu(p, dt, (hipStream_t)stream);
  return err == hipSuccess ? CLV_OK : CLV_ELAUNCH;
}

}  // extern "C"
