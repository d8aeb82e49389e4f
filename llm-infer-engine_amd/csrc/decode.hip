// Split-KV single-token decode attention for gfx950: host side (plans,
// argument checks, the C entry points) and the launches of the head dims that
// are powers of two (8..256).  The kernels are in decode_kernels.hpp; the
// launches of every other head_dim are in decode_pad.hip.
#include <algorithm>
#include <mutex>

#include "decode_kernels.hpp"

// Workspace of mi_flash_decode_noalloc: the split partials (acc, m, l) of one
// call and, in its last kNoallocArriveBytes, the arrival counters of the
// in-launch combine (zero from the start -- a static array of the code object
// -- and returned to zero by every call).  Each device holds its own copy for
// the life of the process; host code reaches it only through the address
// hipGetSymbolAddress returns for the current device (scratch_base below).
static __device__ __align__(256) unsigned char scratch[MI_DECODE_NOALLOC_SCRATCH_BYTES];

// Arrival counters of the in-launch combine handed out per stream by
// mi_decode_arrive_counters: MI_DECODE_ARRIVE_SLABS slabs of
// MI_DECODE_ARRIVE_SLAB counters per device, zero from the start and returned
// to zero by every call that uses them.
static __device__ __align__(256) unsigned long long
    arrive_pool[MI_DECODE_ARRIVE_SLABS * MI_DECODE_ARRIVE_SLAB];

namespace mi {
namespace {

constexpr int64_t kNoallocArriveBytes = 64 << 10;   // 8192 groups

int elem_bytes(int32_t dtype) { return dtype == MI_DTYPE_F32 ? 4 : 2; }

// Register-layout size of a head_dim: the next power of two, at least 8.
int pad_dim(int64_t D) {
  int p = 8;
  while (p < D && p < 256) p <<= 1;
  return p;
}

// Host mirror of DecodeGeom<T, P>: lanes per row, elements per lane, rows per
// wave-load, row unroll and heads per block.
struct HostGeom {
  int lpr, e, rpw, u, gcmax;
};
HostGeom host_geom(int32_t dtype, int64_t D) {
  const int eb = elem_bytes(dtype);
  const int P = pad_dim(D);
  const int ch = P * eb / 16, epc = 16 / eb;   // >= 1: P >= 8
  HostGeom g;
  g.lpr = ch < 16 ? ch : 16;
  g.e = (ch / g.lpr) * epc;
  g.rpw = 64 / g.lpr;
  g.u = g.e <= 8 ? 4 : 2;
  g.gcmax = g.e <= 8 ? 4 : 2;
  return g;
}

int gc_max(int32_t dtype, int64_t D) { return host_geom(dtype, D).gcmax; }

bool supported_head_dim(int64_t D) { return D >= 1 && D <= 256; }

// Load mode for a head_dim and K/V layout: 0 = head_dim is the power of two
// P and rows are 16-byte aligned; 1 = head_dim fills whole 16-byte chunks of
// aligned rows (lanes past it load nothing); 2 = element loads (any head_dim,
// any element-aligned rows, row strides past 512 KB).
int load_mode(int32_t dtype, int64_t D, const void* k, const void* v, int64_t k_sb,
              int64_t k_sh, int64_t k_sl, int64_t v_sb, int64_t v_sh, int64_t v_sl) {
  const int64_t eb = elem_bytes(dtype);
  const bool aligned = ((uintptr_t)k % 16) == 0 && ((uintptr_t)v % 16) == 0 &&
                       (k_sb * eb) % 16 == 0 && (k_sh * eb) % 16 == 0 && (k_sl * eb) % 16 == 0 &&
                       (v_sb * eb) % 16 == 0 && (v_sh * eb) % 16 == 0 && (v_sl * eb) % 16 == 0;
  // MODE 0/1 address a pass's rows by 32-bit offsets from the pass's first
  // row: at most 4096 rows (16 waves x 64 rows x 4) of the larger row stride
  // stay below the out-of-range offset
  const int64_t max_rb = std::max(k_sl, v_sl) * eb;
  const bool span_ok = max_rb * 4096 + 256 * 4 < (int64_t)kOobOffset;
  if (aligned && span_ok && D == pad_dim(D)) return 0;
  if (aligned && span_ok && (D * eb) % 16 == 0) return 1;
  return 2;
}

DecodePlan make_plan(int32_t dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t L,
                     int64_t D, int64_t S, int mode) {
  DecodePlan p;
  const int64_t G = Hq / Hkv;
  const int gmax = mode == 2 ? 1 : gc_max(dtype, D);
  p.n_chunks = (int)((G + gmax - 1) / gmax);
  p.chunk_heads = (int)((G + p.n_chunks - 1) / p.n_chunks);
  p.split_len = (int)((L + S - 1) / S);
  p.n_groups = (int)(B * Hkv * p.n_chunks);
  p.n_xcc = std::max(1, device_xcc_count());
  p.P = pad_dim(D);
  p.mode = mode;
  p.fused = false;
  // A grid of at most one block per CU leaves each CU one block's waves to
  // hide the round trips: 2-byte K/V with whole-chunk rows then run the
  // software-pipelined passes (two passes of loads in flight per wave) with 8
  // waves per block up to head_dim 64 and 4 above.  B8 32/8 D64 at 4097 keys
  // (256 blocks): 21.1 vs 22.8 us per call against the single-buffered kernel,
  // then 19.77 -> 19.65 us with 8 instead of 4 waves; B1 24/8 D128 at 131072
  // keys, 16/32 splits (128/256 blocks): 86.3 vs 88.0 us, 8 waves no faster.
  // Up to two blocks per CU (pipe2) the calls without a mask run the pipelined
  // kernel too, at 4 waves: B16 24/8 D128 ragged (512 blocks) 69.0 -> 68.0 us,
  // B1 24/8 D128 131072 keys at 64 splits 87.6 -> 86.4 us; through mask= it
  // lost (72.8 -> 74.0 us), so mask calls keep the single-buffered kernel there.  With two or more blocks
  // per CU the blocks overlap each other and the single-buffered kernel is as
  // fast or faster (B16 24/8 D128, 512 blocks: 69.0 vs 72.2 us; 131072 keys at
  // 64 splits: 88.6 vs 89.6 us).  One MI355X.
  const int64_t blocks = (int64_t)p.n_groups * S;
  const int cus = device_cu_count();
  p.pipe = dtype != MI_DTYPE_F32 && mode == 0 && blocks <= cus;
  p.pipe2 = dtype != MI_DTYPE_F32 && mode == 0 && !p.pipe && blocks <= 2 * cus;
  int nw = p.pipe && D <= 64 ? 8 : 4;
  if (!p.pipe && blocks < cus)
    nw = 16;
  else if (!p.pipe && blocks < 2 * cus)
    nw = 8;
  // No more waves than the split has row-loads for.
  const HostGeom geo = host_geom(dtype, D);
  if (dtype == MI_DTYPE_F32 && p.P >= 128 && nw > 8) nw = 8;   // split_max_threads
  while (nw > 1 && (int64_t)nw * geo.rpw * geo.u > p.split_len) nw >>= 1;
  p.nw = nw;
  int nw2 = 4;
  while (nw2 > 1 && (int64_t)nw2 * geo.rpw * geo.u > p.split_len) nw2 >>= 1;
  p.nw_pipe2 = nw2;
  return p;
}

template <typename T>
hipError_t launch_split_exact(const DecodeArgs& a, const DecodePlan& p, hipStream_t stream) {
  return launch_split_mode<T, 0>(a, p, stream);
}

hipError_t launch_split_any(int32_t dtype, const DecodeArgs& a, const DecodePlan& p,
                            hipStream_t stream) {
  if (p.mode != 0) return launch_split_padded(dtype, a, p, stream);
  switch (dtype) {
    case MI_DTYPE_BF16: return launch_split_exact<bf16_t>(a, p, stream);
    case MI_DTYPE_F16: return launch_split_exact<f16_t>(a, p, stream);
    default: return launch_split_exact<float>(a, p, stream);
  }
}

int32_t check_common(const void* q, const void* k, const void* v,
                     int64_t B, int64_t Hq, int64_t Hkv, int64_t L,
                     int64_t D, int64_t S, int32_t dtype) {
  if (q == nullptr || k == nullptr || v == nullptr) {
    set_last_error("decode: null q/k/v pointer");
    return MI_ERR_INVALID;
  }
  if (dtype != MI_DTYPE_BF16 && dtype != MI_DTYPE_F16 && dtype != MI_DTYPE_F32) {
    set_last_error("decode: unknown dtype code %d", (int)dtype);
    return MI_ERR_INVALID;
  }
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || L <= 0 || D <= 0 || S <= 0) {
    set_last_error("decode: sizes must be positive (B=%lld Hq=%lld Hkv=%lld L=%lld D=%lld splits=%lld)",
                   (long long)B, (long long)Hq, (long long)Hkv, (long long)L,
                   (long long)D, (long long)S);
    return MI_ERR_INVALID;
  }
  if (Hq % Hkv != 0) {
    set_last_error("decode: query heads (%lld) must be divisible by KV heads (%lld)",
                   (long long)Hq, (long long)Hkv);
    return MI_ERR_INVALID;
  }
  if (!supported_head_dim(D)) {
    set_last_error("decode: head_dim %lld has no kernel (supported: 1 to 256)", (long long)D);
    return MI_ERR_UNSUPPORTED;
  }
  if (L > INT32_MAX / 2 || B > 65535 || Hq > 65535 || S > INT32_MAX / 2 ||
      B * Hq * S > INT32_MAX / 2) {
    set_last_error("decode: shape exceeds launch limits");
    return MI_ERR_UNSUPPORTED;
  }
  const int eb = elem_bytes(dtype);
  if (((uintptr_t)k % eb) != 0 || ((uintptr_t)v % eb) != 0 || ((uintptr_t)q % eb) != 0) {
    set_last_error("decode: q/k/v must be aligned to their element size");
    return MI_ERR_INVALID;
  }
  return MI_OK;
}

DecodeArgs fill_args(const void* q, const void* k, const void* v,
                     const uint8_t* mask, int64_t mask_sb, int64_t mask_sl,
                     const int64_t* seq_lens, int64_t B, int64_t Hq, int64_t Hkv,
                     int64_t L, int64_t D, int64_t S, int64_t q_sb, int64_t q_sh,
                     int64_t q_sd, int64_t k_sb, int64_t k_sh, int64_t k_sl,
                     int64_t v_sb, int64_t v_sh, int64_t v_sl, float sm_scale,
                     const DecodePlan& p, int dtype_bytes) {
  DecodeArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.mask = mask;
  a.mask_sb = mask_sb;
  a.mask_sl = mask_sl;
  a.seq_lens = seq_lens;
  a.q_sb = q_sb; a.q_sh = q_sh; a.q_sd = q_sd;
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_sl = k_sl;
  a.v_sb = v_sb; a.v_sh = v_sh; a.v_sl = v_sl;
  a.batch = (int32_t)B;
  a.n_heads = (int32_t)Hq;
  a.group = (int32_t)(Hq / Hkv);
  a.kv_len = (int32_t)L;
  a.head_dim = (int32_t)D;
  a.n_vchunks = (int32_t)(D * dtype_bytes / 16);
  a.split_len = p.split_len;
  a.num_splits = (int32_t)S;
  a.n_chunks = p.n_chunks;
  a.chunk_heads = p.chunk_heads;
  a.n_xcc = p.n_xcc;
  a.n_groups = p.n_groups;
  a.scale_log2 = sm_scale * kLog2e;
  const int64_t eb = dtype_bytes;
  a.q_vec = (q_sd == 1 && ((uintptr_t)q % 16) == 0 && ((q_sb * eb) % 16) == 0 &&
             ((q_sh * eb) % 16) == 0) ? 1 : 0;
  a.by_length = (seq_lens != nullptr && mask == nullptr && B >= 2 && B <= 64) ? 1 : 0;
  return a;
}

// Many rows with up to 16 splits each: one wave per (batch, head) row (no
// barriers); otherwise one workgroup per row (the splits' loads spread over
// 256 threads, which a few rows need to fill the GPU).  head_dim % 4 != 0
// takes the workgroup kernel with scalar columns.
hipError_t launch_combine_any(int32_t dtype, const CombineArgs& c, int64_t B,
                              int64_t Hq, hipStream_t stream) {
  dim3 block(256);
  const int D = c.head_dim;
  if (c.num_splits <= 16 && B * Hq >= 64 && D % 4 == 0) {
    dim3 grid((unsigned)((B * Hq + 3) / 4));
    switch (dtype) {
      case MI_DTYPE_BF16:
        hipLaunchKernelGGL(decode_combine_wave_kernel<bf16_t>, grid, block, 0, stream, c);
        break;
      case MI_DTYPE_F16:
        hipLaunchKernelGGL(decode_combine_wave_kernel<f16_t>, grid, block, 0, stream, c);
        break;
      default:
        hipLaunchKernelGGL(decode_combine_wave_kernel<float>, grid, block, 0, stream, c);
        break;
    }
    return hipGetLastError();
  }
  const int vec = D % 4 == 0 ? 4 : 1;
  int ncp = 1;
  while (ncp < D / vec) ncp <<= 1;
  const int nsp = 256 / ncp;
  const size_t shmem = ((size_t)c.num_splits + (size_t)nsp * D) * sizeof(float);
  dim3 grid((unsigned)(B * Hq));
#define MI_COMBINE_BLOCK(T)                                                                  \
  if (vec == 4)                                                                              \
    hipLaunchKernelGGL((decode_combine_block_kernel<T, 4>), grid, block, shmem, stream, c);  \
  else                                                                                       \
    hipLaunchKernelGGL((decode_combine_block_kernel<T, 1>), grid, block, shmem, stream, c);
  switch (dtype) {
    case MI_DTYPE_BF16: MI_COMBINE_BLOCK(bf16_t) break;
    case MI_DTYPE_F16: MI_COMBINE_BLOCK(f16_t) break;
    default: MI_COMBINE_BLOCK(float) break;
  }
#undef MI_COMBINE_BLOCK
  return hipGetLastError();
}

constexpr int64_t kMaxSplits = 8192;

// Device address of `scratch` on the current device, looked up once per device.
int32_t scratch_base(unsigned char** out) {
  static std::mutex mu;
  static unsigned char* base[64] = {};
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_last_error("flash_decode_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    return (int32_t)e;
  }
  if (dev < 0 || dev >= 64) {
    set_last_error("flash_decode_noalloc: device %d out of range", dev);
    return MI_ERR_UNSUPPORTED;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (base[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_last_error("flash_decode_noalloc: hipGetSymbolAddress(scratch) failed: %s",
                     hipGetErrorString(e));
      return e != hipSuccess ? (int32_t)e : MI_ERR_INVALID;
    }
    base[dev] = static_cast<unsigned char*>(p);
  }
  *out = base[dev];
  return MI_OK;
}

// Device address of arrive_pool's slab for (current device, stream): each
// stream that asks gets a slab of its own, so calls on different streams
// never share counters; calls on one stream are ordered by the stream.
int32_t arrive_slab(void* stream, uint64_t** out) {
  static std::mutex mu;
  static unsigned long long* base[64] = {};
  static void* owner[64][MI_DECODE_ARRIVE_SLABS] = {};
  static int used[64] = {};
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_last_error("decode_arrive_counters: hipGetDevice failed: %s", hipGetErrorString(e));
    return (int32_t)e;
  }
  if (dev < 0 || dev >= 64) {
    set_last_error("decode_arrive_counters: device %d out of range", dev);
    return MI_ERR_UNSUPPORTED;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (base[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(arrive_pool));
    if (e != hipSuccess || p == nullptr) {
      set_last_error("decode_arrive_counters: hipGetSymbolAddress(arrive_pool) failed: %s",
                     hipGetErrorString(e));
      return e != hipSuccess ? (int32_t)e : MI_ERR_INVALID;
    }
    base[dev] = static_cast<unsigned long long*>(p);
  }
  int slab = -1;
  for (int i = 0; i < used[dev]; ++i)
    if (owner[dev][i] == stream) slab = i;
  if (slab < 0) {
    if (used[dev] == MI_DECODE_ARRIVE_SLABS) {
      set_last_error("decode_arrive_counters: all %d counter slabs of device %d are taken",
                     MI_DECODE_ARRIVE_SLABS, dev);
      return MI_ERR_UNSUPPORTED;
    }
    slab = used[dev]++;
    owner[dev][slab] = stream;
  }
  *out = reinterpret_cast<uint64_t*>(base[dev] + (int64_t)slab * MI_DECODE_ARRIVE_SLAB);
  return MI_OK;
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int32_t mi_decode_arrive_counters(void* stream, uint64_t** counters) {
  if (counters == nullptr) {
    set_last_error("decode_arrive_counters: null output pointer");
    return MI_ERR_INVALID;
  }
  *counters = nullptr;
  return arrive_slab(stream, counters);
}

extern "C" int64_t mi_decode_default_splits(int64_t batch, int64_t n_heads,
                                            int64_t n_kv_heads, int64_t kv_len,
                                            int64_t head_dim) {
  if (batch <= 0 || n_heads <= 0 || n_kv_heads <= 0 || kv_len <= 0) return 1;
  if (!supported_head_dim(head_dim)) head_dim = 128;
  const int64_t G = n_heads / n_kv_heads;
  const int gmax = gc_max(MI_DTYPE_BF16, head_dim);
  const int64_t chunks = (G + gmax - 1) / gmax;
  const int64_t units = batch * n_kv_heads * (chunks > 0 ? chunks : 1);
  const int64_t cus = device_cu_count();
  int64_t s = (2 * cus + units - 1) / units;       // two blocks per CU
  // Splits keep >= 512 KB of K + V (at kv_len, the cache capacity in graph
  // mode) once the blocks already cover every CU: a block's merge and partial
  // write cost a few microseconds however little it streams, so past that
  // point shorter splits lose more than their parallelism gains (measured:
  // B8 Hkv8 D64 at 4097 of 8192 keys, 4 splits 22.9 us vs 8 splits 25.0 us).
  const int64_t row_bytes = 2LL * 2 * head_dim;                            // bf16 K + V
  const int64_t s_bytes = (kv_len * row_bytes + (512 << 10) - 1) / (512 << 10);
  const int64_t s_cover = (cus + units - 1) / units;                       // one block per CU
  if (s > s_bytes) s = s_bytes > s_cover ? s_bytes : s_cover;
  const int64_t s_keys = (kv_len + 63) / 64;                               // >= 64 keys a split
  if (s > s_keys) s = s_keys;
  if (s < 1) s = 1;
  if (s > kMaxSplits) s = kMaxSplits;
  return s;
}

extern "C" int64_t mi_decode_effective_splits(int64_t batch, int64_t n_heads,
                                              int64_t n_kv_heads, int64_t kv_len,
                                              int64_t head_dim, int64_t num_splits) {
  if (batch <= 0 || n_heads <= 0 || n_kv_heads <= 0 || kv_len <= 0 || num_splits <= 1)
    return num_splits < 1 ? 1 : num_splits;
  if (!supported_head_dim(head_dim)) return num_splits;   // the launch will refuse it
  const int64_t G = n_heads / n_kv_heads;
  const int gmax = gc_max(MI_DTYPE_BF16, head_dim);
  const int64_t units = batch * n_kv_heads * ((G + gmax - 1) / gmax);
  const int64_t cus = device_cu_count();
  if (units * num_splits >= cus) return num_splits;
  // each requested split becomes f key ranges until the blocks cover the CUs,
  // keeping >= 1024 keys a range (short calls keep their split count)
  int64_t f = (cus + units * num_splits - 1) / (units * num_splits);
  const int64_t f_keys = kv_len / (1024 * num_splits);
  if (f > f_keys) f = f_keys;
  if (f < 1) f = 1;
  int64_t s = num_splits * f;
  if (s > kMaxSplits) s = num_splits;
  return s;
}

namespace {

// The in-launch combine serves a call when the caller gave counters, the
// K/V rows are whole 16-byte chunks of a power-of-two head_dim (MODE 0), no
// mask is given and the split blocks are few and short: at most one block
// per CU and <= 16 splits (one round trip of partial loads per row).
// Measured on MI355X against the two-launch form: B8 32/8 D64 at 4097 keys
// (4 splits, 256 blocks) 21.7 vs 22.7 us; two blocks per CU (B16 24/8 D128
// ragged, 512 blocks) 71.7 vs 71.1 us and 32+ splits of one sequence 89-120
// vs 88-92 us, where the last block's tail (its partial stores, the arrival
// atomic, the combine loads) costs more than the separate launch.
bool use_fused(const void* arrive, const uint8_t* mask, int mode, int64_t num_splits,
               int64_t n_groups) {
  return arrive != nullptr && mask == nullptr && mode == 0 && num_splits > 1 &&
         num_splits <= 16 && n_groups * num_splits <= device_cu_count();
}

// Phase 1 (and, with arrive, the in-launch combine where use_fused chooses
// it; *fused reports whether it did).
int32_t run_split(const void* q, const void* k, const void* v, const uint8_t* mask,
                  int64_t mask_sb, int64_t mask_sl, const int64_t* seq_lens, float* part_m,
                  float* part_l, float* part_acc, void* out, float* lse,
                  unsigned long long* arrive, int64_t batch, int64_t n_heads,
                  int64_t n_kv_heads, int64_t kv_len, int64_t head_dim, int64_t num_splits,
                  int64_t q_sb, int64_t q_sh, int64_t q_sd, int64_t k_sb, int64_t k_sh,
                  int64_t k_sl, int64_t v_sb, int64_t v_sh, int64_t v_sl, int64_t o_sb,
                  int64_t o_sh, int64_t o_sd, float sm_scale, int32_t empty_rows_nan,
                  int32_t dtype, void* stream, const char* what, bool* fused) {
  const int mode = load_mode(dtype, head_dim, k, v, k_sb, k_sh, k_sl, v_sb, v_sh, v_sl);
  DecodePlan p = make_plan(dtype, batch, n_heads, n_kv_heads, kv_len, head_dim, num_splits, mode);
  p.fused = use_fused(arrive, mask, mode, num_splits, p.n_groups);
  *fused = p.fused;
  if (!p.fused) arrive = nullptr;
  DecodeArgs a = fill_args(q, k, v, mask, mask_sb, mask_sl, seq_lens, batch, n_heads,
                           n_kv_heads, kv_len, head_dim, num_splits, q_sb, q_sh, q_sd,
                           k_sb, k_sh, k_sl, v_sb, v_sh, v_sl, sm_scale, p,
                           elem_bytes(dtype));
  a.part_m = part_m;
  a.part_l = part_l;
  a.part_acc = part_acc;
  a.out = out;
  a.lse = lse;
  a.arrive = arrive;
  a.o_sb = o_sb; a.o_sh = o_sh; a.o_sd = o_sd;
  a.direct = num_splits == 1 ? 1 : 0;
  a.empty_nan = empty_rows_nan;
  hipError_t e = launch_split_any(dtype, a, p, (hipStream_t)stream);
  if (e != hipSuccess) {
    set_last_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return (int32_t)e;
  }
  return MI_OK;
}

}  // namespace

extern "C" int32_t mi_decode_split(
    const void* q, const void* k, const void* v, const uint8_t* mask,
    int64_t mask_sb, int64_t mask_sl, const int64_t* seq_lens, float* part_m,
    float* part_l, float* part_acc, int64_t batch, int64_t n_heads,
    int64_t n_kv_heads, int64_t kv_len, int64_t head_dim, int64_t num_splits,
    int64_t q_sb, int64_t q_sh, int64_t q_sd, int64_t k_sb, int64_t k_sh,
    int64_t k_sl, int64_t v_sb, int64_t v_sh, int64_t v_sl, float sm_scale,
    int32_t dtype, void* stream) {
  int32_t st = check_common(q, k, v, batch, n_heads, n_kv_heads, kv_len,
                            head_dim, num_splits, dtype);
  if (st != MI_OK) return st;
  if (part_m == nullptr || part_l == nullptr || part_acc == nullptr) {
    set_last_error("decode_split: partial buffers must not be null");
    return MI_ERR_INVALID;
  }
  if (num_splits > kMaxSplits) {
    set_last_error("decode_split: num_splits %lld exceeds %lld",
                   (long long)num_splits, (long long)kMaxSplits);
    return MI_ERR_UNSUPPORTED;
  }
  // one split writes partials too (the combine kernel normalises them)
  const int mode = load_mode(dtype, head_dim, k, v, k_sb, k_sh, k_sl, v_sb, v_sh, v_sl);
  DecodePlan p = make_plan(dtype, batch, n_heads, n_kv_heads, kv_len, head_dim, num_splits, mode);
  DecodeArgs a = fill_args(q, k, v, mask, mask_sb, mask_sl, seq_lens, batch, n_heads,
                           n_kv_heads, kv_len, head_dim, num_splits, q_sb, q_sh, q_sd,
                           k_sb, k_sh, k_sl, v_sb, v_sh, v_sl, sm_scale, p,
                           elem_bytes(dtype));
  a.part_m = part_m;
  a.part_l = part_l;
  a.part_acc = part_acc;
  a.direct = 0;
  hipError_t e = launch_split_any(dtype, a, p, (hipStream_t)stream);
  if (e != hipSuccess) {
    set_last_error("decode_split: launch failed: %s", hipGetErrorString(e));
    return (int32_t)e;
  }
  return MI_OK;
}

extern "C" int32_t mi_decode_combine(const float* part_m, const float* part_l,
                                     const float* part_acc, void* out,
                                     float* lse, int64_t batch,
                                     int64_t n_heads, int64_t head_dim,
                                     int64_t num_splits, int64_t o_sb,
                                     int64_t o_sh, int64_t o_sd,
                                     int32_t empty_rows_nan, int32_t dtype,
                                     void* stream) {
  if (part_m == nullptr || part_l == nullptr || part_acc == nullptr ||
      out == nullptr) {
    set_last_error("decode_combine: null pointer");
    return MI_ERR_INVALID;
  }
  if (batch <= 0 || n_heads <= 0 || num_splits <= 0 || head_dim <= 0) {
    set_last_error("decode_combine: sizes must be positive");
    return MI_ERR_INVALID;
  }
  if (num_splits > kMaxSplits) {
    set_last_error("decode_combine: num_splits %lld exceeds %lld",
                   (long long)num_splits, (long long)kMaxSplits);
    return MI_ERR_UNSUPPORTED;
  }
  if (!supported_head_dim(head_dim)) {
    set_last_error("decode_combine: head_dim %lld unsupported (1 to 256)", (long long)head_dim);
    return MI_ERR_UNSUPPORTED;
  }
  if (dtype != MI_DTYPE_BF16 && dtype != MI_DTYPE_F16 && dtype != MI_DTYPE_F32) {
    set_last_error("decode_combine: unknown dtype code %d", (int)dtype);
    return MI_ERR_INVALID;
  }
  CombineArgs c{};
  c.part_m = part_m;
  c.part_l = part_l;
  c.part_acc = part_acc;
  c.out = out;
  c.lse = lse;
  c.o_sb = o_sb; c.o_sh = o_sh; c.o_sd = o_sd;
  c.n_rows = batch * n_heads;
  c.n_heads = (int32_t)n_heads;
  c.head_dim = (int32_t)head_dim;
  c.num_splits = (int32_t)num_splits;
  c.empty_nan = empty_rows_nan;
  hipError_t e = launch_combine_any(dtype, c, batch, n_heads, (hipStream_t)stream);
  if (e != hipSuccess) {
    set_last_error("decode_combine: launch failed: %s", hipGetErrorString(e));
    return (int32_t)e;
  }
  return MI_OK;
}

extern "C" int32_t mi_flash_decode(
    const void* q, const void* k, const void* v, const uint8_t* mask,
    int64_t mask_sb, int64_t mask_sl, const int64_t* seq_lens, float* part_m,
    float* part_l, float* part_acc, uint64_t* arrive, void* out, float* lse,
    int64_t batch, int64_t n_heads, int64_t n_kv_heads, int64_t kv_len, int64_t head_dim,
    int64_t num_splits, int64_t q_sb, int64_t q_sh, int64_t q_sd, int64_t k_sb,
    int64_t k_sh, int64_t k_sl, int64_t v_sb, int64_t v_sh, int64_t v_sl,
    int64_t o_sb, int64_t o_sh, int64_t o_sd, float sm_scale,
    int32_t empty_rows_nan, int32_t dtype, void* stream) {
  if (out == nullptr) {
    set_last_error("flash_decode: null output pointer");
    return MI_ERR_INVALID;
  }
  int32_t st = check_common(q, k, v, batch, n_heads, n_kv_heads, kv_len, head_dim,
                            num_splits, dtype);
  if (st != MI_OK) return st;
  if (num_splits > kMaxSplits) {
    set_last_error("flash_decode: num_splits %lld exceeds %lld",
                   (long long)num_splits, (long long)kMaxSplits);
    return MI_ERR_UNSUPPORTED;
  }
  if (num_splits != 1 && (part_m == nullptr || part_l == nullptr || part_acc == nullptr)) {
    set_last_error("flash_decode: partial buffers must not be null with num_splits > 1");
    return MI_ERR_INVALID;
  }
  bool fused = false;
  st = run_split(q, k, v, mask, mask_sb, mask_sl, seq_lens, part_m, part_l, part_acc, out, lse,
                 reinterpret_cast<unsigned long long*>(arrive), batch, n_heads, n_kv_heads,
                 kv_len, head_dim, num_splits, q_sb, q_sh, q_sd, k_sb, k_sh, k_sl, v_sb, v_sh,
                 v_sl, o_sb, o_sh, o_sd, sm_scale, empty_rows_nan, dtype, stream, "flash_decode",
                 &fused);
  if (st != MI_OK || num_splits == 1 || fused) return st;
  return mi_decode_combine(part_m, part_l, part_acc, out, lse, batch, n_heads, head_dim,
                           num_splits, o_sb, o_sh, o_sd, empty_rows_nan, dtype, stream);
}

extern "C" int32_t mi_flash_decode_noalloc(
    const void* q, const void* k, const void* v, const uint8_t* mask,
    int64_t mask_sb, int64_t mask_sl, const int64_t* seq_lens, void* out, float* lse,
    int64_t batch, int64_t n_heads, int64_t n_kv_heads, int64_t kv_len, int64_t head_dim,
    int64_t num_splits, int64_t q_sb, int64_t q_sh, int64_t q_sd, int64_t k_sb,
    int64_t k_sh, int64_t k_sl, int64_t v_sb, int64_t v_sh, int64_t v_sl,
    int64_t o_sb, int64_t o_sh, int64_t o_sd, float sm_scale,
    int32_t empty_rows_nan, int32_t dtype, void* stream) {
  if (batch <= 0 || n_heads <= 0 || num_splits <= 0 || head_dim <= 0 ||
      num_splits > kMaxSplits) {
    set_last_error("flash_decode_noalloc: sizes must be positive and num_splits <= %lld",
                   (long long)kMaxSplits);
    return MI_ERR_INVALID;
  }
  if (!supported_head_dim(head_dim)) {
    set_last_error("flash_decode_noalloc: head_dim %lld has no kernel (supported: 1 to 256)",
                   (long long)head_dim);
    return MI_ERR_UNSUPPORTED;
  }
  if (num_splits == 1)  // single pass: no partials at all
    return mi_flash_decode(q, k, v, mask, mask_sb, mask_sl, seq_lens, nullptr, nullptr,
                           nullptr, nullptr, out, lse, batch, n_heads, n_kv_heads, kv_len,
                           head_dim, 1, q_sb, q_sh, q_sd, k_sb, k_sh, k_sl, v_sb, v_sh, v_sl,
                           o_sb, o_sh, o_sd, sm_scale, empty_rows_nan, dtype, stream);
  // fewer splits than fill the GPU are subdivided, as flash_decode does
  num_splits = mi_decode_effective_splits(batch, n_heads, n_kv_heads, kv_len, head_dim,
                                          num_splits);
  // layout in scratch: acc [B*Hq*S*D] fp32, then m and l [B*Hq*S] fp32 each,
  // every array starting on a 256-byte boundary; the arrival counters (one
  // per group, at most batch * n_heads) in the last kNoallocArriveBytes
  const int64_t rows = batch * n_heads * num_splits;
  auto up = [](int64_t b) { return (b + 255) & ~(int64_t)255; };
  const int64_t part_cap = (int64_t)MI_DECODE_NOALLOC_SCRATCH_BYTES - kNoallocArriveBytes;
  const int64_t acc_bytes = up(rows * head_dim * 4), ml_bytes = up(rows * 4);
  if (rows > part_cap || acc_bytes + 2 * ml_bytes > part_cap) {
    set_last_error("flash_decode_noalloc: partials of batch*n_heads*num_splits = %lld rows x "
                   "(head_dim %lld + 2) fp32 exceed the %lld-byte scratch; use fewer splits "
                   "or mi_flash_decode with a workspace",
                   (long long)rows, (long long)head_dim, (long long)part_cap);
    return MI_ERR_UNSUPPORTED;
  }
  unsigned char* base = nullptr;
  int32_t st = scratch_base(&base);
  if (st != MI_OK) return st;
  float* part_acc = reinterpret_cast<float*>(base);
  float* part_m = reinterpret_cast<float*>(base + acc_bytes);
  float* part_l = reinterpret_cast<float*>(base + acc_bytes + ml_bytes);
  uint64_t* arrive = batch * n_heads * 8 <= kNoallocArriveBytes
                         ? reinterpret_cast<uint64_t*>(base + part_cap)
                         : nullptr;
  return mi_flash_decode(q, k, v, mask, mask_sb, mask_sl, seq_lens, part_m, part_l, part_acc,
                         arrive, out, lse, batch, n_heads, n_kv_heads, kv_len, head_dim,
                         num_splits, q_sb, q_sh, q_sd, k_sb, k_sh, k_sl, v_sb, v_sh, v_sl, o_sb,
                         o_sh, o_sd, sm_scale, empty_rows_nan, dtype, stream);
}
