// W8A16 GEMV for decode: y[m, n] = (sum_k x[m, k] * q[n, k]) * s[n], M <= 16.
//
// Math of the reference's GEMV kernel (src/quant_linear.py:7-63): fp32
// accumulation of x.f32 * q.f32 over k, the per-row scale applied once after
// the sum (:57), result rounded to x's dtype.
//
// MI355X design: the weights are the only large operand (read once from HBM),
// and M <= 8 rows of x is far too little work per weight byte for the VALU
// (8 MACs/byte at 5.6 TB/s exceeds the non-packed fp32 FMA rate), so the MACs
// run on v_mfma_f32_16x16x32_{bf16,f16}: int8 weights are converted exactly to
// the activation dtype in registers (|q| <= 128 is exact in bf16/fp16) and fed
// as the A operand (16 weight rows x 32 k); x^T is the B operand with the m
// columns beyond M zero-filled.  Each lane loads 16 contiguous int8 of a row
// (two MFMA k-steps).  A workgroup owns 16 output rows; its 4 waves split K
// and are reduced through LDS, then the scale is applied and y is written.
#include "common.hpp"

namespace mi {

struct GemvArgs {
  const void* x;
  const int8_t* w;
  const void* scales;
  void* y;
  int64_t x_sm, x_sk;
  int64_t w_sn;
  int64_t s_sn;
  int64_t y_sm, y_sn;
  int32_t M, N, K;
};

template <typename T> struct GemvMfma;
template <> struct GemvMfma<bf16_t> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  __device__ static inline f32x4 mma(const v8& a, const v8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct GemvMfma<f16_t> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  __device__ static inline f32x4 mma(const v8& a, const v8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// 8 signed bytes (two words) -> 8 activation-dtype values (exact).
template <typename T, typename V8>
__device__ inline V8 i8x8_to(uint32_t lo, uint32_t hi) {
  V8 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r[i] = (T)(float)(int8_t)(lo >> (8 * i));
    r[4 + i] = (T)(float)(int8_t)(hi >> (8 * i));
  }
  return r;
}

template <typename T, typename ST>
__global__ __launch_bounds__(256) void w8a16_gemv_kernel(GemvArgs a) {
  using MM = GemvMfma<T>;
  typedef typename MM::v8 v8;
  constexpr int kUnroll = 4;
  __shared__ f32x4 red[4][64];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int n0 = blockIdx.x * 16;
  const int r = lane & 15, g = lane >> 4;     // weight row in tile / k group
  const int n = min(n0 + r, a.N - 1);
  const int8_t* wrow = a.w + (int64_t)n * a.w_sn;
  const int m = lane & 15;                    // x row for the B operand
  const bool m_ok = m < a.M;
  const T* xrow = reinterpret_cast<const T*>(a.x) + (int64_t)(m_ok ? m : 0) * a.x_sm;
  const int n_chunks = (a.K + 63) / 64;       // 64-k chunks; waves interleave

  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int c0 = w; c0 < n_chunks; c0 += 4 * kUnroll) {
    u32x4 wq[kUnroll];
    v8 xb[kUnroll][2];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int c = c0 + 4 * u;
      const int k0 = c * 64 + 16 * g;
      const bool ok = c < n_chunks && k0 < a.K;
      wq[u] = ok ? *reinterpret_cast<const u32x4*>(wrow + k0) : u32x4{0, 0, 0, 0};
      if (ok && m_ok) {
        if (a.x_sk == 1) {
          xb[u][0] = __builtin_bit_cast(v8, load16(xrow + k0));
          xb[u][1] = __builtin_bit_cast(v8, load16(xrow + k0 + 8));
        } else {
#pragma unroll
          for (int t = 0; t < 8; ++t) {
            xb[u][0][t] = xrow[(int64_t)(k0 + t) * a.x_sk];
            xb[u][1][t] = xrow[(int64_t)(k0 + 8 + t) * a.x_sk];
          }
        }
      } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) { xb[u][0][t] = (T)0.f; xb[u][1][t] = (T)0.f; }
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const v8 w0 = i8x8_to<T, v8>(wq[u].x, wq[u].y);
      const v8 w1 = i8x8_to<T, v8>(wq[u].z, wq[u].w);
      acc = MM::mma(w0, xb[u][0], acc);
      acc = MM::mma(w1, xb[u][1], acc);
    }
  }
  red[w][lane] = acc;
  __syncthreads();
  if (w != 0) return;
  acc = red[0][lane] + red[1][lane] + red[2][lane] + red[3][lane];
  // acc[i] = C[row 4*(lane/16) + i][col lane%16] = y[m = lane%16][n0 + 4*g + i]
  if (!m_ok) return;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int nn = n0 + 4 * g + i;
    if (nn < a.N) {
      const float s = Elem<ST>::to_f32(reinterpret_cast<const ST*>(a.scales)[(int64_t)nn * a.s_sn]);
      reinterpret_cast<T*>(a.y)[(int64_t)m * a.y_sm + (int64_t)nn * a.y_sn] =
          Elem<T>::from_f32(acc[i] * s);
    }
  }
}

}  // namespace mi

using namespace mi;

extern "C" int32_t mi_w8a16_gemv(const void* x, const int8_t* w,
                                 const void* scales, void* y, int64_t m,
                                 int64_t n, int64_t k, int64_t x_sm,
                                 int64_t x_sk, int64_t w_sn, int64_t s_sn,
                                 int64_t y_sm, int64_t y_sn, int32_t dtype,
                                 int32_t sdtype, void* stream) {
  if (x == nullptr || w == nullptr || scales == nullptr || y == nullptr) {
    set_last_error("w8a16_gemv: null pointer");
    return MI_ERR_INVALID;
  }
  if (m <= 0 || m > 16 || n <= 0 || k <= 0 || n > INT32_MAX || k > INT32_MAX) {
    set_last_error("w8a16_gemv: need 1 <= M <= 16 and positive N, K (M=%lld N=%lld K=%lld)",
                   (long long)m, (long long)n, (long long)k);
    return MI_ERR_INVALID;
  }
  if (k % 16 != 0 || (uintptr_t)w % 16 != 0 || w_sn % 16 != 0) {
    set_last_error("w8a16_gemv: K and the weight row stride must be multiples of 16 bytes");
    return MI_ERR_UNSUPPORTED;
  }
  if (x_sk == 1 && (((uintptr_t)x % 16) != 0 || (x_sm * 2) % 16 != 0)) {
    set_last_error("w8a16_gemv: contiguous x rows must be 16-byte aligned");
    return MI_ERR_INVALID;
  }
  GemvArgs a{x, w, scales, y, x_sm, x_sk, w_sn, s_sn, y_sm, y_sn,
             (int32_t)m, (int32_t)n, (int32_t)k};
  dim3 grid((unsigned)((n + 15) / 16)), block(256);
  hipStream_t st = (hipStream_t)stream;
#define MI_GEMV(T, ST) hipLaunchKernelGGL((w8a16_gemv_kernel<T, ST>), grid, block, 0, st, a)
  if (dtype == MI_DTYPE_BF16 && sdtype == MI_DTYPE_BF16) MI_GEMV(bf16_t, bf16_t);
  else if (dtype == MI_DTYPE_BF16 && sdtype == MI_DTYPE_F32) MI_GEMV(bf16_t, float);
  else if (dtype == MI_DTYPE_BF16 && sdtype == MI_DTYPE_F16) MI_GEMV(bf16_t, f16_t);
  else if (dtype == MI_DTYPE_F16 && sdtype == MI_DTYPE_F16) MI_GEMV(f16_t, f16_t);
  else if (dtype == MI_DTYPE_F16 && sdtype == MI_DTYPE_F32) MI_GEMV(f16_t, float);
  else if (dtype == MI_DTYPE_F16 && sdtype == MI_DTYPE_BF16) MI_GEMV(f16_t, bf16_t);
  else {
    set_last_error("w8a16_gemv: activations must be bf16 or fp16 (dtype %d, scales %d)",
                   (int)dtype, (int)sdtype);
    return MI_ERR_UNSUPPORTED;
  }
#undef MI_GEMV
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_last_error("w8a16_gemv: launch failed: %s", hipGetErrorString(e));
    return (int32_t)e;
  }
  return MI_OK;
}
