// Output projection of a decode step (lm_head) with the final RMSNorm fused in
// front and an optional greedy argmax fused behind, for 1 <= M <= 16 token rows.
//
// Math (the reference's  out = self.output(self.norm(h))  src/model.py:137-183,
// sampler argmax  src/sampler.py:30):
//   a        = dtype(x * rsqrt(mean(x^2) + eps) * norm_w)   (fp32 inside; skipped
//              when norm_w is NULL: a = x)                   src/rms_norm.py:32-38
//   y[m, n]  = dtype(sum_k a[m, k] * w[n, k])               fp32 accumulate
//   tok[m]   = first n with y[m, n] == max_n y[m, n]         (torch.argmax rule)
//
// Design (MI355X): the weight matrix (vocab x dim, 525 MB at Llama-3.2-1B) is
// the only large operand and is streamed once from HBM; x is tiny.  Each
// workgroup stages the normalised x once in LDS (rows padded by 16 bytes so
// the 16 B-operand rows of one MFMA read hit distinct banks, rows >= M read a
// zero row), then its four waves walk 16-row tiles of w over the full K:
// v_mfma_f32_16x16x32_{bf16,f16} with w as the A operand (each lane loads 16
// contiguous bytes = the 8 k-values of one A row) and x^T from LDS as B.  A
// wave keeps the next 512-k batch of weight loads in flight while it runs the
// MFMAs of the current one (two register buffers, loads issued unconditionally
// from clamped addresses so the in-order vmcnt waits stay exact).  The grid is
// persistent (at most two workgroups per CU) so the x prologue is paid once per
// workgroup, not once per tile.  No K split: every tile's sum lives in one
// wave, so there is no cross-wave reduction.
//
// Argmax: each lane keeps the best (value, index) of the tiles it saw for its
// x row; lanes and waves merge through shuffles / LDS into one partial per
// (row, workgroup), and a one-workgroup-per-row finalize kernel reduces the
// partials.  Ties keep the smaller index, the first occurrence.
#include <math.h>

#include "common.hpp"

namespace mi {

struct LmHeadArgs {
  const void* x;        // [M, K], row stride x_sm (elements)
  const void* norm_w;   // [K] or null
  float eps;
  const void* w;        // [N, K] activation dtype, row stride w_sn (elements)
  void* y;              // [M, N] logits, row stride y_sm (elements)
  float* part_v;        // [M][n_parts] best value per workgroup (argmax) or null
  int32_t* part_i;      // [M][n_parts] its index
  int64_t x_sm, w_sn, y_sm;
  int32_t M, K, N, n_tiles, n_parts;
  int32_t y_vec;        // y rows 8-byte aligned: 4 logits per 64-bit store
};

template <typename T> struct HMfma;
template <> struct HMfma<bf16_t> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  __device__ static inline f32x4 mma(const v8& a, const v8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct HMfma<f16_t> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  __device__ static inline f32x4 mma(const v8& a, const v8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// (value, index) order of the argmax: larger value wins, equal values keep
// the smaller index.
__device__ inline bool better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

// x from lane (lane ^ OFF) without LDS traffic: a DPP row rotate for 8, the
// gfx950 permlane swap for 32.
template <int OFF>
__device__ inline float lm_lane_xor(float x, int lane) {
  if constexpr (OFF == 8) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xF, 0xF, true));
  } else {
    static_assert(OFF == 32, "lane stride");
    auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                               false);
    return __uint_as_float((lane & 32) ? sw[0] : sw[1]);
  }
}

constexpr int kLmWaves = 4;
constexpr int kLmBatch = 16;   // 16 MFMAs (512 k) per weight batch

// DIAG (M <= 8): tiles of 8 weight rows, diagonal-packed -- A lanes of rows
// r < 8 hold weight row r over the first 32 k of a 64-k step, rows r >= 8 the
// same rows over the second 32 k; B columns c < 8 hold token row c over the
// first half, c >= 8 token row c - 8 over the second; C[r][c] + C[r+8][c+8]
// is the 64-k product.  A load instruction then reads 8 rows x 128 contiguous
// bytes (whole cache lines) instead of 16 rows x 64 bytes, and no B column is
// padding.  Otherwise (up to 16 rows): 16-row tiles, columns >= M zero.
template <typename T, bool DIAG>
__global__ __launch_bounds__(64 * kLmWaves) void lm_head_kernel(LmHeadArgs a) {
  using MM = HMfma<T>;
  typedef typename MM::v8 v8;
  extern __shared__ __align__(16) unsigned char smem[];
  const int K = a.K, M = a.M;
  const int row_b = K * 2 + 16;                 // padded LDS row (bytes)
  unsigned char* xs = smem;                     // rows 0..M-1: a; row M: zeros
  __shared__ float red_ss[kLmWaves][16];
  __shared__ float red_v[kLmWaves][16];
  __shared__ int red_i[kLmWaves][16];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);

  // ---- tiles: wave-global index gw walks tiles gw, gw + G, ...
  const int G = gridDim.x * kLmWaves;
  const int gw = blockIdx.x * kLmWaves + w;
  const int my_tiles = gw < a.n_tiles ? (a.n_tiles - 1 - gw) / G + 1 : 0;
  constexpr int TR = DIAG ? 8 : 16;             // weight rows per tile
  constexpr int KS = DIAG ? 64 : 32;            // k per MFMA
  const int KB = K / (KS * kLmBatch);           // weight batches per tile
  const int n_steps = my_tiles * KB;
  const int r = lane & 15, g = lane >> 4;       // A: tile row / k group
  const int rrow = DIAG ? (r & 7) : r;          // weight row within the tile
  const int khalf = DIAG ? 32 * (r >> 3) : 0;   // k offset of this lane's half
  const int mcol = lane & 15;                   // B: x row (>= M: zero row)
  const int xrow = DIAG ? (mcol & 7) : mcol;
  const unsigned char* xb = xs + (xrow < M ? xrow : M) * row_b + g * 16 + khalf * 2;
  const T* wbase = reinterpret_cast<const T*>(a.w);

  auto issue = [&](u32x4 (&buf)[kLmBatch], int s) {
    const int t = gw + (s / KB) * G, kb = s % KB;
    const int row = min(t * TR + rrow, a.N - 1);  // rows past N: clamped, discarded
    const T* p = wbase + (int64_t)row * a.w_sn + kb * KS * kLmBatch + khalf + 8 * g;
#pragma unroll
    for (int j = 0; j < kLmBatch; ++j) buf[j] = load16_stream(p + KS * j);
  };
  float best_v = -INFINITY;
  int best_i = 0x7fffffff;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  auto compute = [&](const u32x4 (&buf)[kLmBatch], int s) {
    const int t = gw + (s / KB) * G, kb = s % KB;
#pragma unroll
    for (int j = 0; j < kLmBatch; ++j) {
      const v8 xv = __builtin_bit_cast(
          v8, *reinterpret_cast<const u32x4*>(xb + (kb * KS * kLmBatch + KS * j) * 2));
      acc = MM::mma(__builtin_bit_cast(v8, buf[j]), xv, acc);
    }
    if (kb == KB - 1) {
      if constexpr (DIAG) {
        // fold the diagonal quadrants: lane + 40 holds C[4g + i + 8][c + 8]
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] += lm_lane_xor<8>(lm_lane_xor<32>(acc[i], lane), lane);
      }
      // acc[i] = y[mcol][t*TR + 4g + i]  (DIAG: lanes g < 2, mcol < 8)
      const int n0 = t * TR + 4 * g;
      T yv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) yv[i] = Elem<T>::from_f32(acc[i]);
      if (mcol < M && (!DIAG || g < 2)) {
        T* yp = reinterpret_cast<T*>(a.y) + (int64_t)mcol * a.y_sm + n0;
        if (a.y_vec && n0 + 3 < a.N) {
          typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
          *reinterpret_cast<u32x2*>(yp) = __builtin_bit_cast(u32x2, yv);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (n0 + i < a.N) yp[i] = yv[i];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float v = Elem<T>::to_f32(yv[i]);
          if (n0 + i < a.N && better(v, n0 + i, best_v, best_i)) {
            best_v = v;
            best_i = n0 + i;
          }
        }
      }
      acc = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };

  u32x4 ba[kLmBatch], bb[kLmBatch];

  // ---- prologue: a = rmsnorm(x) (or x) into LDS, zero row M.  The x rows and
  //      this thread's norm-weight chunks (K <= 4096: at most two) are loaded
  //      first, then the first weight batch is issued, so the batch streams
  //      during the statistics and the normalisation (which then wait on LDS
  //      only, never on a global load issued behind the batch)
  {
    const int nch = K / 8;                      // 16-byte chunks per row
    u32x4 nwr[2] = {u32x4{0, 0, 0, 0}, u32x4{0, 0, 0, 0}};
    if (a.norm_w != nullptr) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
        if (tid + i * 64 * kLmWaves < nch)
          nwr[i] = load16(reinterpret_cast<const T*>(a.norm_w) + (tid + i * 64 * kLmWaves) * 8);
    }
    float ss[16];
#pragma unroll
    for (int m = 0; m < 16; ++m) ss[m] = 0.f;
    for (int m = 0; m < M; ++m) {
      for (int c = tid; c < nch; c += 64 * kLmWaves) {
        const u32x4 v = load16(reinterpret_cast<const T*>(a.x) + (int64_t)m * a.x_sm + c * 8);
        *reinterpret_cast<u32x4*>(xs + m * row_b + c * 16) = v;
        if (a.norm_w != nullptr) {
          float f[8];
          Chunk<T>::unpack(v, f);
          float t = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) t = fmaf(f[e], f[e], t);
#pragma unroll
          for (int mm = 0; mm < 16; ++mm)
            if (mm == m) ss[mm] += t;
        }
      }
    }
    // the norm-weight registers are consumed here (an empty asm taking them),
    // before the batch is issued, so no later wait on them covers the batch
    asm volatile("" ::"v"(nwr[0]), "v"(nwr[1]) : "memory");
    if (n_steps > 0) issue(ba, 0);
    for (int c = tid; c < nch; c += 64 * kLmWaves)
      *reinterpret_cast<u32x4*>(xs + M * row_b + c * 16) = u32x4{0, 0, 0, 0};
    if (a.norm_w != nullptr) {
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        float t = ss[m];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) t += shfl_xor_f32(t, off);
        if (lane == 0) red_ss[w][m] = t;
      }
    }
    __syncthreads();
    if (a.norm_w != nullptr) {
      for (int m = 0; m < M; ++m) {
        const float tot = red_ss[0][m] + red_ss[1][m] + red_ss[2][m] + red_ss[3][m];
        const float rstd = 1.0f / sqrtf(tot / (float)K + a.eps);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int c = tid + i * 64 * kLmWaves;
          if (c >= nch) break;
          u32x4* p = reinterpret_cast<u32x4*>(xs + m * row_b + c * 16);
          float f[8];
          Chunk<T>::unpack(*p, f);
          typedef T t8 __attribute__((ext_vector_type(8)));
          t8 o;
          float wn[8];
          Chunk<T>::unpack(nwr[i], wn);
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = Elem<T>::from_f32(f[e] * rstd * wn[e]);
          *reinterpret_cast<t8*>(p) = o;
        }
      }
      __syncthreads();
    }
  }

  if (n_steps > 0) {
    for (int s = 0; s < n_steps; s += 2) {
      issue(bb, min(s + 1, n_steps - 1));
      compute(ba, s);
      issue(ba, min(s + 2, n_steps - 1));
      if (s + 1 < n_steps) compute(bb, s + 1);
    }
  }

  if (a.part_v == nullptr) return;
  // ---- argmax partials: lanes m, m+16, m+32, m+48 hold row m's candidates
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) {
    const float ov = shfl_xor_f32(best_v, off);
    const int oi = __shfl_xor(best_i, off);
    if (better(ov, oi, best_v, best_i)) {
      best_v = ov;
      best_i = oi;
    }
  }
  if (lane < 16) {
    red_v[w][lane] = best_v;
    red_i[w][lane] = best_i;
  }
  __syncthreads();
  if (tid < M) {
    float bv = red_v[0][tid];
    int bi = red_i[0][tid];
#pragma unroll
    for (int ww = 1; ww < kLmWaves; ++ww)
      if (better(red_v[ww][tid], red_i[ww][tid], bv, bi)) {
        bv = red_v[ww][tid];
        bi = red_i[ww][tid];
      }
    a.part_v[(int64_t)tid * a.n_parts + blockIdx.x] = bv;
    a.part_i[(int64_t)tid * a.n_parts + blockIdx.x] = bi;
  }
}

// One workgroup per row: argmax over the per-workgroup partials (count
// entries per row, row stride `stride`).
__global__ __launch_bounds__(256) void lm_head_argmax_kernel(const float* part_v,
                                                             const int32_t* part_i, int count,
                                                             int stride, int64_t* out) {
  __shared__ float sv[4];
  __shared__ int si[4];
  const int m = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int p = tid; p < count; p += 256) {
    const float v = part_v[(int64_t)m * stride + p];
    const int i = part_i[(int64_t)m * stride + p];
    if (better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = shfl_xor_f32(bv, off);
    const int oi = __shfl_xor(bi, off);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane == 0) {
    sv[w] = bv;
    si[w] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int ww = 1; ww < 4; ++ww)
      if (better(sv[ww], si[ww], bv, bi)) {
        bv = sv[ww];
        bi = si[ww];
      }
    out[m] = bi;
  }
}

namespace {

// Workgroups of a launch over `tiles` weight tiles (persistent: at most two per
// CU); with 8-row tiles this also bounds the 16-row tiling's grid.
int lm_head_grid_tiles(int64_t tiles) {
  const int cus = device_cu_count();
  const int64_t groups = (tiles + kLmWaves - 1) / kLmWaves;
  return (int)(groups < 2 * cus ? groups : 2 * cus);
}
int lm_head_grid(int64_t n) { return lm_head_grid_tiles((n + 7) / 8); }

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int64_t mi_lm_head_partials(int64_t m, int64_t n) {
  if (m <= 0 || n <= 0) return 0;
  return lm_head_grid(n);
}

extern "C" int32_t mi_lm_head(const void* x, int64_t x_sm, const void* norm_w, float eps,
                              const void* w, int64_t w_sn, void* y, int64_t y_sm,
                              int64_t* argmax_out, float* part_v, int32_t* part_i,
                              int64_t n_parts, int64_t m, int64_t n, int64_t k,
                              int32_t dtype, void* stream) {
  if (x == nullptr || w == nullptr || y == nullptr) {
    set_last_error("lm_head: null pointer");
    return MI_ERR_INVALID;
  }
  if (m <= 0 || n <= 0 || k <= 0) {
    set_last_error("lm_head: sizes must be positive");
    return MI_ERR_INVALID;
  }
  if (dtype != MI_DTYPE_BF16 && dtype != MI_DTYPE_F16) {
    set_last_error("lm_head: dtype code %d has no kernel (bf16, fp16 only)", (int)dtype);
    return MI_ERR_UNSUPPORTED;
  }
  if (m > 16 || k % 512 != 0 || k > 4096 || n > INT32_MAX - 16) {
    set_last_error("lm_head: shape m=%lld k=%lld n=%lld unsupported (m <= 16, k %% 512 == 0, "
                   "k <= 4096)", (long long)m, (long long)k, (long long)n);
    return MI_ERR_UNSUPPORTED;
  }
  const uintptr_t px = (uintptr_t)x, pw = (uintptr_t)w, py = (uintptr_t)y;
  if ((px | pw) % 16 != 0 || py % 2 != 0 || (x_sm * 2) % 16 != 0 || (w_sn * 2) % 16 != 0 ||
      (norm_w != nullptr && (uintptr_t)norm_w % 16 != 0) || x_sm < k || w_sn < k || y_sm < n) {
    set_last_error("lm_head: x / w / norm_w rows must be 16-byte aligned");
    return MI_ERR_INVALID;
  }
  // diagonal-packed 8-row tiles for up to 8 rows (64-k MFMA steps, 1024-k batches)
  const bool diag = m <= 8 && k % (64 * kLmBatch) == 0;
  const int grid = lm_head_grid_tiles(diag ? (n + 7) / 8 : (n + 15) / 16);
  if (argmax_out != nullptr && (part_v == nullptr || part_i == nullptr || n_parts < grid)) {
    set_last_error("lm_head: argmax needs partial buffers of >= %d entries per row", grid);
    return MI_ERR_INVALID;
  }
  LmHeadArgs a{};
  a.x = x; a.norm_w = norm_w; a.eps = eps; a.w = w; a.y = y;
  a.part_v = argmax_out != nullptr ? part_v : nullptr;
  a.part_i = argmax_out != nullptr ? part_i : nullptr;
  a.x_sm = x_sm; a.w_sn = w_sn; a.y_sm = y_sm;
  a.M = (int32_t)m; a.K = (int32_t)k; a.N = (int32_t)n;
  a.n_tiles = (int32_t)(diag ? (n + 7) / 8 : (n + 15) / 16);
  a.n_parts = (int32_t)(argmax_out != nullptr ? n_parts : 0);
  a.y_vec = (py % 8 == 0 && (y_sm * 2) % 8 == 0) ? 1 : 0;
  const size_t shmem = (size_t)(m + 1) * (size_t)(k * 2 + 16);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == MI_DTYPE_BF16) {
    if (diag)
      hipLaunchKernelGGL((lm_head_kernel<bf16_t, true>), dim3(grid), dim3(64 * kLmWaves), shmem, st, a);
    else
      hipLaunchKernelGGL((lm_head_kernel<bf16_t, false>), dim3(grid), dim3(64 * kLmWaves), shmem, st, a);
  } else {
    if (diag)
      hipLaunchKernelGGL((lm_head_kernel<f16_t, true>), dim3(grid), dim3(64 * kLmWaves), shmem, st, a);
    else
      hipLaunchKernelGGL((lm_head_kernel<f16_t, false>), dim3(grid), dim3(64 * kLmWaves), shmem, st, a);
  }
  hipError_t e = hipGetLastError();
  if (e == hipSuccess && argmax_out != nullptr) {
    hipLaunchKernelGGL(lm_head_argmax_kernel, dim3((unsigned)m), dim3(256), 0, st, part_v, part_i,
                       grid, (int)n_parts, argmax_out);
    e = hipGetLastError();
  }
  if (e != hipSuccess) {
    set_last_error("lm_head: launch failed: %s", hipGetErrorString(e));
    return (int32_t)e;
  }
  return MI_OK;
}
