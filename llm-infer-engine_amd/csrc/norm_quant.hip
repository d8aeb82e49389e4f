// RMSNorm and symmetric per-channel int8 weight quantisation.
//
// RMSNorm (src/rms_norm.py:18-39): y = x * rsqrt(sum(x^2)/N + eps) * w, all in
// fp32 from the stored values, rounded once to x's dtype.  One workgroup per
// row; wave shuffles + LDS for the sum of squares; 16-byte rows in registers.
//
// Quantiser (src/quant_utils.py:7-36): per output row n,
//   amax = max(max_k |w[n,k]|, 1e-12)          (fp32)
//   s    = round_to_dtype(amax / 127)            (IEEE fp32 divide, RNE)
//   q    = clamp(rne(w / s), -128, 127) -> int8  (IEEE fp32 divide)
// Bit-exact with the reference recipe: every step is a correctly rounded IEEE
// operation (no reciprocal approximations, no contraction).
#include <math.h>

#include "common.hpp"

namespace mi {

struct NormArgs {
  const void* x;
  const void* w;
  void* y;
  int64_t x_rs, y_rs;  // row strides (elements)
  int32_t M, N;
  float eps;
};

template <typename T, typename WT>
__global__ __launch_bounds__(256) void rmsnorm_kernel(NormArgs a) {
  __shared__ float red[4];
  const int row = blockIdx.x;
  const T* xr = reinterpret_cast<const T*>(a.x) + (int64_t)row * a.x_rs;
  T* yr = reinterpret_cast<T*>(a.y) + (int64_t)row * a.y_rs;
  const WT* w = reinterpret_cast<const WT*>(a.w);
  const int tid = threadIdx.x;
  float ss = 0.f;
  for (int i = tid; i < a.N; i += 256) {
    const float v = Elem<T>::to_f32(xr[i]);
    ss = fmaf(v, v, ss);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ss += shfl_xor_f32(ss, off);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  const float tot = red[0] + red[1] + red[2] + red[3];
  const float rstd = 1.0f / sqrtf(tot / (float)a.N + a.eps);
  for (int i = tid; i < a.N; i += 256) {
    const float v = Elem<T>::to_f32(xr[i]);
    yr[i] = Elem<T>::from_f32(v * rstd * Elem<WT>::to_f32(w[i]));
  }
}

// 2-byte rows of N <= 2048 * CPT elements with 16-byte aligned rows and
// weights: each thread loads its 16-byte chunks of the row once, keeps them in
// registers across the reduction and writes 16-byte chunks (one read and one
// write of the row instead of two reads with 2-byte accesses).  The same fp32
// maths as rmsnorm_kernel; the sum of squares is taken over a thread's 8
// contiguous elements first (fp32 summation order only).
template <typename T, typename WT, int CPT>
__global__ __launch_bounds__(256) void rmsnorm_vec_kernel(NormArgs a) {
  __shared__ float red[4];
  const int row = blockIdx.x, tid = threadIdx.x;
  const T* xr = reinterpret_cast<const T*>(a.x) + (int64_t)row * a.x_rs;
  T* yr = reinterpret_cast<T*>(a.y) + (int64_t)row * a.y_rs;
  const WT* w = reinterpret_cast<const WT*>(a.w);
  const int nch = a.N >> 3;
  u32x4 xv[CPT];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int idx = tid + c * 256;
    if (idx < nch) {
      xv[c] = load16(xr + 8 * idx);
      float f[8];
      Chunk<T>::unpack(xv[c], f);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(f[e], f[e], ss);
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ss += shfl_xor_f32(ss, off);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  const float tot = red[0] + red[1] + red[2] + red[3];
  const float rstd = 1.0f / sqrtf(tot / (float)a.N + a.eps);
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int idx = tid + c * 256;
    if (idx < nch) {
      float f[8], wf[8];
      Chunk<T>::unpack(xv[c], f);
      if constexpr (sizeof(WT) == 2) {
        Chunk<WT>::unpack(load16(w + 8 * idx), wf);
      } else {
        const f32x4 w0 = *reinterpret_cast<const f32x4*>(w + 8 * idx);
        const f32x4 w1 = *reinterpret_cast<const f32x4*>(w + 8 * idx + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) { wf[e] = w0[e]; wf[4 + e] = w1[e]; }
      }
      union { u32x4 u; T t[8]; } o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o.t[e] = Elem<T>::from_f32(f[e] * rstd * wf[e]);
      *reinterpret_cast<u32x4*>(yr + 8 * idx) = o.u;
    }
  }
}

struct QuantArgs {
  const void* w;
  int8_t* q;
  void* scales;
  int64_t w_rs, q_rs;
  int32_t N, K;
};

template <typename T>
__global__ __launch_bounds__(256) void quantize_kernel(QuantArgs a) {
#pragma clang fp contract(off)
  __shared__ float red[4];
  const int n = blockIdx.x;
  const T* wr = reinterpret_cast<const T*>(a.w) + (int64_t)n * a.w_rs;
  int8_t* qr = a.q + (int64_t)n * a.q_rs;
  const int tid = threadIdx.x;
  float mx = 0.f;
  for (int k = tid; k < a.K; k += 256) mx = fmaxf(mx, fabsf(Elem<T>::to_f32(wr[k])));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, shfl_xor_f32(mx, off));
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  float amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  amax = fmaxf(amax, 1e-12f);
  const T s_t = Elem<T>::from_f32(amax / 127.0f);
  const float s = Elem<T>::to_f32(s_t);
  if (tid == 0) reinterpret_cast<T*>(a.scales)[n] = s_t;
  for (int k = tid; k < a.K; k += 256) {
    const float r = rintf(Elem<T>::to_f32(wr[k]) / s);
    // 0/0 (an all-zero fp16 row whose scale underflows to 0) has no defined
    // int8 value in the reference recipe; it is written as 0.
    qr[k] = r != r ? (int8_t)0 : (int8_t)fminf(fmaxf(r, -128.0f), 127.0f);
  }
}

}  // namespace mi

using namespace mi;

extern "C" int32_t mi_rmsnorm(const void* x, const void* w, void* y,
                              int64_t rows, int64_t n, int64_t x_rs,
                              int64_t y_rs, float eps, int32_t dtype,
                              int32_t wdtype, void* stream) {
  if (x == nullptr || w == nullptr || y == nullptr) {
    set_last_error("rmsnorm: null pointer");
    return MI_ERR_INVALID;
  }
  if (rows < 0 || n <= 0 || rows > INT32_MAX || n > INT32_MAX) {
    set_last_error("rmsnorm: invalid shape");
    return MI_ERR_INVALID;
  }
  if (rows == 0) return MI_OK;
  NormArgs a{x, w, y, x_rs, y_rs, (int32_t)rows, (int32_t)n, eps};
  dim3 grid((unsigned)rows), block(256);
  hipStream_t st = (hipStream_t)stream;
  // 16-byte rows take the vector kernel (CPT chunks of 8 per thread)
  const bool vec = dtype != MI_DTYPE_F32 && n % 8 == 0 && n <= 8192 &&
                   ((uintptr_t)x | (uintptr_t)y | (uintptr_t)w) % 16 == 0 &&
                   ((x_rs | y_rs) * 2) % 16 == 0;
  const int cpt = (int)((n / 8 + 255) / 256);
#define MI_NORM(T, WT)                                                                   \
  if (!vec)                                                                              \
    hipLaunchKernelGGL((rmsnorm_kernel<T, WT>), grid, block, 0, st, a);                 \
  else if (cpt == 1)                                                                     \
    hipLaunchKernelGGL((rmsnorm_vec_kernel<T, WT, 1>), grid, block, 0, st, a);          \
  else if (cpt == 2)                                                                     \
    hipLaunchKernelGGL((rmsnorm_vec_kernel<T, WT, 2>), grid, block, 0, st, a);          \
  else                                                                                   \
    hipLaunchKernelGGL((rmsnorm_vec_kernel<T, WT, 4>), grid, block, 0, st, a)
  if (dtype == MI_DTYPE_BF16 && wdtype == MI_DTYPE_BF16) MI_NORM(bf16_t, bf16_t);
  else if (dtype == MI_DTYPE_BF16 && wdtype == MI_DTYPE_F32) MI_NORM(bf16_t, float);
  else if (dtype == MI_DTYPE_F16 && wdtype == MI_DTYPE_F16) MI_NORM(f16_t, f16_t);
  else if (dtype == MI_DTYPE_F16 && wdtype == MI_DTYPE_F32) MI_NORM(f16_t, float);
  else if (dtype == MI_DTYPE_F32 && wdtype == MI_DTYPE_F32)
    hipLaunchKernelGGL((rmsnorm_kernel<float, float>), grid, block, 0, st, a);
  else if (dtype == MI_DTYPE_F32 && wdtype == MI_DTYPE_BF16)
    hipLaunchKernelGGL((rmsnorm_kernel<float, bf16_t>), grid, block, 0, st, a);
  else {
    set_last_error("rmsnorm: unsupported dtype pair (%d, %d)", (int)dtype, (int)wdtype);
    return MI_ERR_UNSUPPORTED;
  }
#undef MI_NORM
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_last_error("rmsnorm: launch failed: %s", hipGetErrorString(e));
    return (int32_t)e;
  }
  return MI_OK;
}

extern "C" int32_t mi_quantize_int8(const void* w, int8_t* q, void* scales,
                                    int64_t n_rows, int64_t k, int64_t w_rs,
                                    int64_t q_rs, int32_t dtype, void* stream) {
  if (w == nullptr || q == nullptr || scales == nullptr) {
    set_last_error("quantize_int8: null pointer");
    return MI_ERR_INVALID;
  }
  if (n_rows < 0 || k <= 0 || n_rows > INT32_MAX || k > INT32_MAX) {
    set_last_error("quantize_int8: invalid shape");
    return MI_ERR_INVALID;
  }
  if (n_rows == 0) return MI_OK;
  QuantArgs a{w, q, scales, w_rs, q_rs, (int32_t)n_rows, (int32_t)k};
  dim3 grid((unsigned)n_rows), block(256);
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case MI_DTYPE_BF16: hipLaunchKernelGGL(quantize_kernel<bf16_t>, grid, block, 0, st, a); break;
    case MI_DTYPE_F16: hipLaunchKernelGGL(quantize_kernel<f16_t>, grid, block, 0, st, a); break;
    case MI_DTYPE_F32: hipLaunchKernelGGL(quantize_kernel<float>, grid, block, 0, st, a); break;
    default:
      set_last_error("quantize_int8: unknown dtype code %d", (int)dtype);
      return MI_ERR_INVALID;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_last_error("quantize_int8: launch failed: %s", hipGetErrorString(e));
    return (int32_t)e;
  }
  return MI_OK;
}
