// Rotary position embedding and the fused K-RoPE + KV-cache append.
//
// Math (rotate-half form, src/rope.py:85-86 / :162-163 / :230-231):
//   y[i]       = x[i]       * cos[i] - x[i + D/2] * sin[i]
//   y[i + D/2] = x[i + D/2] * cos[i] + x[i]       * sin[i]      0 <= i < D/2
// computed in fp32 from the stored values, with the products and the sum
// rounded separately (FP contraction off for this code), then rounded
// once to the output dtype.  The KV append writes RoPE(K) and a bitwise copy
// of V into cache slot ((((b*Hkv + h)*T + pos)*D + d) of the layer view
// (src/kv_cache.py:15, src/rope.py:166,216).
//
// One thread per rotation pair (i, i + D/2); consecutive threads take
// consecutive i, so loads/stores of a row coalesce when the head dim has unit
// stride.  With cos == sin == NULL the append copies K unrotated (KV write).
#include "common.hpp"

namespace mi {

struct RopeArgs {
  const void* x;
  void* out;
  const void* cos;
  const void* sin;
  const int64_t* positions;  // null: table row s; else row positions[s]
  int64_t x_sb, x_sh, x_ss, x_sd;
  int64_t o_sb, o_sh, o_ss, o_sd;
  int64_t c_ss, c_sd, s_ss, s_sd;
  int32_t B, H, S, half;
};

template <typename T, typename CT>
__device__ inline void rotate(float x1, float x2, CT cv, CT sv, T& y1, T& y2) {
  // No contraction: products and the sum are each rounded to fp32, then the
  // result is rounded to T (an fma, or a fused fma_mix f16 conversion, would
  // round once and can differ in the last bit).
#pragma clang fp contract(off)
  const float c = Elem<CT>::to_f32(cv), s = Elem<CT>::to_f32(sv);
  const float x1c = x1 * c, x2s = x2 * s, x2c = x2 * c, x1s = x1 * s;
  const float r1 = x1c - x2s, r2 = x2c + x1s;
  y1 = Elem<T>::from_f32(r1);
  y2 = Elem<T>::from_f32(r2);
}

template <typename T, typename CT>
__global__ __launch_bounds__(256) void rope_kernel(RopeArgs a) {
  const int64_t total = (int64_t)a.B * a.H * a.S * a.half;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    int64_t r = idx;
    const int i = (int)(r % a.half); r /= a.half;
    const int s = (int)(r % a.S); r /= a.S;
    const int h = (int)(r % a.H);
    const int b = (int)(r / a.H);
    const T* xp = reinterpret_cast<const T*>(a.x) + b * a.x_sb + h * a.x_sh + s * a.x_ss;
    T* op = reinterpret_cast<T*>(a.out) + b * a.o_sb + h * a.o_sh + s * a.o_ss;
    const int64_t crow = a.positions != nullptr ? a.positions[s] : s;
    const CT* cp = reinterpret_cast<const CT*>(a.cos) + crow * a.c_ss + i * a.c_sd;
    const CT* sp = reinterpret_cast<const CT*>(a.sin) + crow * a.s_ss + i * a.s_sd;
    const float x1 = Elem<T>::to_f32(xp[i * a.x_sd]);
    const float x2 = Elem<T>::to_f32(xp[(i + a.half) * a.x_sd]);
    T y1, y2;
    rotate<T, CT>(x1, x2, *cp, *sp, y1, y2);
    op[i * a.o_sd] = y1;
    op[(i + a.half) * a.o_sd] = y2;
  }
}

struct KvAppendArgs {
  const void* xk;
  const void* xv;
  const void* cos;
  const void* sin;
  void* ck;
  void* cv;
  const int64_t* positions;  // null: pos = start_pos + s
  int64_t start_pos;
  int64_t xk_sb, xk_sh, xk_ss, xk_sd;
  int64_t xv_sb, xv_sh, xv_ss, xv_sd;
  int64_t ck_sb, ck_sh, ck_st, ck_sd;
  int64_t cv_sb, cv_sh, cv_st, cv_sd;
  int64_t c_ss, c_sd, s_ss, s_sd;
  int64_t capacity;  // T: slots outside [0, T) are never written
  int32_t B, H, S, half;
  int32_t cos_by_pos;  // cos/sin rows indexed by absolute position, not s
};

template <typename T, typename CT>
__global__ __launch_bounds__(256) void rope_kv_append_kernel(KvAppendArgs a) {
  const int64_t total = (int64_t)a.B * a.H * a.S * a.half;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    int64_t r = idx;
    const int i = (int)(r % a.half); r /= a.half;
    const int s = (int)(r % a.S); r /= a.S;
    const int h = (int)(r % a.H);
    const int b = (int)(r / a.H);
    const int64_t pos = a.positions != nullptr ? a.positions[s] : a.start_pos + s;
    if (pos < 0 || pos >= a.capacity) continue;
    const int64_t crow = a.cos_by_pos ? pos : s;
    const T* kp = reinterpret_cast<const T*>(a.xk) + b * a.xk_sb + h * a.xk_sh + s * a.xk_ss;
    const T* vp = reinterpret_cast<const T*>(a.xv) + b * a.xv_sb + h * a.xv_sh + s * a.xv_ss;
    T* kc = reinterpret_cast<T*>(a.ck) + b * a.ck_sb + h * a.ck_sh + pos * a.ck_st;
    T* vc = reinterpret_cast<T*>(a.cv) + b * a.cv_sb + h * a.cv_sh + pos * a.cv_st;
    const CT* cp = reinterpret_cast<const CT*>(a.cos) + crow * a.c_ss + i * a.c_sd;
    const CT* sp = reinterpret_cast<const CT*>(a.sin) + crow * a.s_ss + i * a.s_sd;
    if (a.cos != nullptr) {
      const float x1 = Elem<T>::to_f32(kp[i * a.xk_sd]);
      const float x2 = Elem<T>::to_f32(kp[(i + a.half) * a.xk_sd]);
      T y1, y2;
      rotate<T, CT>(x1, x2, *cp, *sp, y1, y2);
      kc[i * a.ck_sd] = y1;
      kc[(i + a.half) * a.ck_sd] = y2;
    } else {  // plain KV write (KVCache.update): K copied bitwise too
      kc[i * a.ck_sd] = kp[i * a.xk_sd];
      kc[(i + a.half) * a.ck_sd] = kp[(i + a.half) * a.xk_sd];
    }
    vc[i * a.cv_sd] = vp[i * a.xv_sd];
    vc[(i + a.half) * a.cv_sd] = vp[(i + a.half) * a.xv_sd];
  }
}

namespace {

bool valid_dtype(int32_t d) {
  return d == MI_DTYPE_BF16 || d == MI_DTYPE_F16 || d == MI_DTYPE_F32;
}

unsigned grid_for(int64_t total) {
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  return (unsigned)blocks;
}

}  // namespace
}  // namespace mi

using namespace mi;

#define MI_ROPE_DISPATCH(KERNEL, ARGS, TOTAL, STREAM)                            \
  do {                                                                        \
    dim3 grid_(grid_for(TOTAL)), block_(256);                                 \
    if (dtype == MI_DTYPE_BF16 && cdtype == MI_DTYPE_BF16)                    \
      hipLaunchKernelGGL((KERNEL<bf16_t, bf16_t>), grid_, block_, 0, STREAM, ARGS); \
    else if (dtype == MI_DTYPE_BF16 && cdtype == MI_DTYPE_F32)                \
      hipLaunchKernelGGL((KERNEL<bf16_t, float>), grid_, block_, 0, STREAM, ARGS);  \
    else if (dtype == MI_DTYPE_F16 && cdtype == MI_DTYPE_F16)                 \
      hipLaunchKernelGGL((KERNEL<f16_t, f16_t>), grid_, block_, 0, STREAM, ARGS);   \
    else if (dtype == MI_DTYPE_F16 && cdtype == MI_DTYPE_F32)                 \
      hipLaunchKernelGGL((KERNEL<f16_t, float>), grid_, block_, 0, STREAM, ARGS);   \
    else if (dtype == MI_DTYPE_F32 && cdtype == MI_DTYPE_F32)                 \
      hipLaunchKernelGGL((KERNEL<float, float>), grid_, block_, 0, STREAM, ARGS);   \
    else if (dtype == MI_DTYPE_F32 && cdtype == MI_DTYPE_BF16)                \
      hipLaunchKernelGGL((KERNEL<float, bf16_t>), grid_, block_, 0, STREAM, ARGS);  \
    else if (dtype == MI_DTYPE_F32 && cdtype == MI_DTYPE_F16)                 \
      hipLaunchKernelGGL((KERNEL<float, f16_t>), grid_, block_, 0, STREAM, ARGS);   \
    else if (dtype == MI_DTYPE_BF16 && cdtype == MI_DTYPE_F16)                \
      hipLaunchKernelGGL((KERNEL<bf16_t, f16_t>), grid_, block_, 0, STREAM, ARGS);  \
    else                                                                      \
      hipLaunchKernelGGL((KERNEL<f16_t, bf16_t>), grid_, block_, 0, STREAM, ARGS);  \
  } while (0)

extern "C" int32_t mi_rope(const void* x, void* out, const void* cos,
                           const void* sin, const int64_t* positions,
                           int64_t batch, int64_t n_heads,
                           int64_t seq_len, int64_t head_dim, int64_t x_sb,
                           int64_t x_sh, int64_t x_ss, int64_t x_sd,
                           int64_t o_sb, int64_t o_sh, int64_t o_ss,
                           int64_t o_sd, int64_t c_ss, int64_t c_sd,
                           int64_t s_ss, int64_t s_sd, int32_t dtype,
                           int32_t cdtype, void* stream) {
  if (x == nullptr || out == nullptr || cos == nullptr || sin == nullptr) {
    set_last_error("rope: null pointer");
    return MI_ERR_INVALID;
  }
  if (!valid_dtype(dtype) || !valid_dtype(cdtype)) {
    set_last_error("rope: unknown dtype code");
    return MI_ERR_INVALID;
  }
  if (batch < 0 || n_heads < 0 || seq_len < 0 || head_dim <= 0 || head_dim % 2 != 0) {
    set_last_error("rope: invalid shape (head_dim must be even)");
    return MI_ERR_INVALID;
  }
  const int64_t total = batch * n_heads * seq_len * (head_dim / 2);
  if (total == 0) return MI_OK;
  RopeArgs a{};
  a.x = x; a.out = out; a.cos = cos; a.sin = sin; a.positions = positions;
  a.x_sb = x_sb; a.x_sh = x_sh; a.x_ss = x_ss; a.x_sd = x_sd;
  a.o_sb = o_sb; a.o_sh = o_sh; a.o_ss = o_ss; a.o_sd = o_sd;
  a.c_ss = c_ss; a.c_sd = c_sd; a.s_ss = s_ss; a.s_sd = s_sd;
  a.B = (int32_t)batch; a.H = (int32_t)n_heads; a.S = (int32_t)seq_len;
  a.half = (int32_t)(head_dim / 2);
  MI_ROPE_DISPATCH(rope_kernel, a, total, (hipStream_t)stream);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_last_error("rope: launch failed: %s", hipGetErrorString(e));
    return (int32_t)e;
  }
  return MI_OK;
}

extern "C" int32_t mi_rope_kv_append(
    const void* xk, const void* xv, const void* cos, const void* sin,
    void* cache_k, void* cache_v, int64_t start_pos, const int64_t* positions,
    int64_t batch, int64_t n_kv_heads, int64_t seq_len, int64_t head_dim,
    int64_t capacity, int64_t xk_sb, int64_t xk_sh, int64_t xk_ss,
    int64_t xk_sd, int64_t xv_sb, int64_t xv_sh, int64_t xv_ss, int64_t xv_sd,
    int64_t ck_sb, int64_t ck_sh, int64_t ck_st, int64_t ck_sd, int64_t cv_sb,
    int64_t cv_sh, int64_t cv_st, int64_t cv_sd, int64_t c_ss, int64_t c_sd,
    int64_t s_ss, int64_t s_sd, int32_t cos_by_position, int32_t dtype,
    int32_t cdtype, void* stream) {
  if (xk == nullptr || xv == nullptr || cache_k == nullptr || cache_v == nullptr ||
      ((cos == nullptr) != (sin == nullptr))) {
    set_last_error("rope_kv_append: null pointer");
    return MI_ERR_INVALID;
  }
  if (!valid_dtype(dtype) || !valid_dtype(cdtype)) {
    set_last_error("rope_kv_append: unknown dtype code");
    return MI_ERR_INVALID;
  }
  if (batch < 0 || n_kv_heads < 0 || seq_len < 0 || head_dim <= 0 ||
      head_dim % 2 != 0 || capacity <= 0) {
    set_last_error("rope_kv_append: invalid shape");
    return MI_ERR_INVALID;
  }
  if (positions == nullptr && (start_pos < 0 || start_pos + seq_len > capacity)) {
    set_last_error("rope_kv_append: positions [%lld, %lld) exceed cache capacity %lld",
                   (long long)start_pos, (long long)(start_pos + seq_len),
                   (long long)capacity);
    return MI_ERR_INVALID;
  }
  const int64_t total = batch * n_kv_heads * seq_len * (head_dim / 2);
  if (total == 0) return MI_OK;
  KvAppendArgs a{};
  a.xk = xk; a.xv = xv; a.cos = cos; a.sin = sin; a.ck = cache_k; a.cv = cache_v;
  a.positions = positions;
  a.start_pos = start_pos;
  a.xk_sb = xk_sb; a.xk_sh = xk_sh; a.xk_ss = xk_ss; a.xk_sd = xk_sd;
  a.xv_sb = xv_sb; a.xv_sh = xv_sh; a.xv_ss = xv_ss; a.xv_sd = xv_sd;
  a.ck_sb = ck_sb; a.ck_sh = ck_sh; a.ck_st = ck_st; a.ck_sd = ck_sd;
  a.cv_sb = cv_sb; a.cv_sh = cv_sh; a.cv_st = cv_st; a.cv_sd = cv_sd;
  a.c_ss = c_ss; a.c_sd = c_sd; a.s_ss = s_ss; a.s_sd = s_sd;
  a.capacity = capacity;
  a.B = (int32_t)batch; a.H = (int32_t)n_kv_heads; a.S = (int32_t)seq_len;
  a.half = (int32_t)(head_dim / 2);
  a.cos_by_pos = cos_by_position;
  MI_ROPE_DISPATCH(rope_kv_append_kernel, a, total, (hipStream_t)stream);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_last_error("rope_kv_append: launch failed: %s", hipGetErrorString(e));
    return (int32_t)e;
  }
  return MI_OK;
}
