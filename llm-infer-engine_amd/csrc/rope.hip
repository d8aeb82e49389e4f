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
#include <initializer_list>

#include "common.hpp"

namespace mi {

struct RopeArgs {
  const void* x;
  void* out;
  const void* cos;
  const void* sin;
  const int64_t* positions;  // null: table row s; else row positions[s]
  int64_t rows;              // table rows: positions are clamped into [0, rows)
  int64_t x_sb, x_sh, x_ss, x_sd;
  int64_t o_sb, o_sh, o_ss, o_sd;
  int64_t c_ss, c_sd, s_ss, s_sd;
  int32_t B, H, S, half;
};

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
    const int64_t crow =
        a.positions != nullptr ? min(max(a.positions[s], (int64_t)0), a.rows - 1) : s;
    const CT* cp = reinterpret_cast<const CT*>(a.cos) + crow * a.c_ss + i * a.c_sd;
    const CT* sp = reinterpret_cast<const CT*>(a.sin) + crow * a.s_ss + i * a.s_sd;
    const float x1 = Elem<T>::to_f32(xp[i * a.x_sd]);
    const float x2 = Elem<T>::to_f32(xp[(i + a.half) * a.x_sd]);
    T y1, y2;
    rope_rotate<T, CT>(x1, x2, *cp, *sp, y1, y2);
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
  int64_t rows;      // table rows: a position past them uses the last row
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
    const int64_t crow = a.cos_by_pos ? min(pos, a.rows - 1) : s;
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
      rope_rotate<T, CT>(x1, x2, *cp, *sp, y1, y2);
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

// 16-byte forms of the two kernels above for 2-byte data with tables in the
// same dtype, unit head-dim strides and 16-byte aligned rows: a thread rotates
// 8 consecutive pairs (i0 .. i0+7 with their partners i0+D/2 ..), one 16-byte
// load or store per 8 elements.  Same per-pair arithmetic (rope_rotate), so the
// same bits.
template <typename T>
__device__ inline void rotate8(const u32x4& xa, const u32x4& xb, const u32x4& cw,
                               const u32x4& sw, u32x4& ya, u32x4& yb) {
  typedef T t8 __attribute__((ext_vector_type(8)));
  const t8 x1 = __builtin_bit_cast(t8, xa), x2 = __builtin_bit_cast(t8, xb);
  const t8 c = __builtin_bit_cast(t8, cw), sn = __builtin_bit_cast(t8, sw);
  t8 y1, y2;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    T r1, r2;
    rope_rotate<T, T>(Elem<T>::to_f32(x1[e]), Elem<T>::to_f32(x2[e]), c[e], sn[e], r1, r2);
    y1[e] = r1;
    y2[e] = r2;
  }
  ya = __builtin_bit_cast(u32x4, y1);
  yb = __builtin_bit_cast(u32x4, y2);
}

// Grid: x over (token, 8-pair group) of one (batch, head) row, y over
// (batch, head); 32-bit index arithmetic (the host checks the sizes).
template <typename T>
__global__ __launch_bounds__(256) void rope_vec_kernel(RopeArgs a) {
  const uint32_t nj = (uint32_t)a.half >> 3, per_row = (uint32_t)a.S * nj;
  for (uint32_t bh = blockIdx.y; bh < (uint32_t)(a.B * a.H); bh += gridDim.y) {
    const int b = (int)(bh / (uint32_t)a.H), h = (int)(bh % (uint32_t)a.H);
    for (uint32_t t = blockIdx.x * blockDim.x + threadIdx.x; t < per_row;
         t += gridDim.x * blockDim.x) {
      const int s = (int)(t / nj), i0 = 8 * (int)(t % nj);
      const T* xp = reinterpret_cast<const T*>(a.x) + b * a.x_sb + h * a.x_sh + s * a.x_ss + i0;
      T* op = reinterpret_cast<T*>(a.out) + b * a.o_sb + h * a.o_sh + s * a.o_ss + i0;
      const int64_t crow =
          a.positions != nullptr ? min(max(a.positions[s], (int64_t)0), a.rows - 1) : s;
      const T* cp = reinterpret_cast<const T*>(a.cos) + crow * a.c_ss + i0;
      const T* sp = reinterpret_cast<const T*>(a.sin) + crow * a.s_ss + i0;
      u32x4 ya, yb;
      rotate8<T>(load16(xp), load16(xp + a.half), load16(cp), load16(sp), ya, yb);
      *reinterpret_cast<u32x4*>(op) = ya;
      *reinterpret_cast<u32x4*>(op + a.half) = yb;
    }
  }
}

// The cache rows are written with non-temporal stores (streamed to memory
// rather than kept in L2): at config 2's model-layout prefill (33.5 MB moved)
// 7.5 -> 7.0 us per call, and the attention block that then reads the cache
// 88.7 -> 87.4 us (one MI355X).  The inputs keep temporal loads: they are the
// projection outputs just written, and non-temporal loads of them cost 11 us.
template <typename T>
__global__ __launch_bounds__(256) void rope_kv_append_vec_kernel(KvAppendArgs a) {
  const uint32_t nj = (uint32_t)a.half >> 3, per_row = (uint32_t)a.S * nj;
  for (uint32_t bh = blockIdx.y; bh < (uint32_t)(a.B * a.H); bh += gridDim.y) {
    const int b = (int)(bh / (uint32_t)a.H), h = (int)(bh % (uint32_t)a.H);
    for (uint32_t t = blockIdx.x * blockDim.x + threadIdx.x; t < per_row;
         t += gridDim.x * blockDim.x) {
      const int s = (int)(t / nj), i0 = 8 * (int)(t % nj);
      const int64_t pos = a.positions != nullptr ? a.positions[s] : a.start_pos + s;
      if (pos < 0 || pos >= a.capacity) continue;
      const T* kp = reinterpret_cast<const T*>(a.xk) + b * a.xk_sb + h * a.xk_sh + s * a.xk_ss + i0;
      const T* vp = reinterpret_cast<const T*>(a.xv) + b * a.xv_sb + h * a.xv_sh + s * a.xv_ss + i0;
      T* kc = reinterpret_cast<T*>(a.ck) + b * a.ck_sb + h * a.ck_sh + pos * a.ck_st + i0;
      T* vc = reinterpret_cast<T*>(a.cv) + b * a.cv_sb + h * a.cv_sh + pos * a.cv_st + i0;
      const u32x4 k1 = load16(kp), k2 = load16(kp + a.half);
      const u32x4 v1 = load16(vp), v2 = load16(vp + a.half);
      if (a.cos != nullptr) {
        const int64_t crow = a.cos_by_pos ? min(pos, a.rows - 1) : s;
        const T* cp = reinterpret_cast<const T*>(a.cos) + crow * a.c_ss + i0;
        const T* sp = reinterpret_cast<const T*>(a.sin) + crow * a.s_ss + i0;
        u32x4 ya, yb;
        rotate8<T>(k1, k2, load16(cp), load16(sp), ya, yb);
        __builtin_nontemporal_store(ya, reinterpret_cast<u32x4*>(kc));
        __builtin_nontemporal_store(yb, reinterpret_cast<u32x4*>(kc + a.half));
      } else {  // plain KV write: K copied bitwise too
        __builtin_nontemporal_store(k1, reinterpret_cast<u32x4*>(kc));
        __builtin_nontemporal_store(k2, reinterpret_cast<u32x4*>(kc + a.half));
      }
      __builtin_nontemporal_store(v1, reinterpret_cast<u32x4*>(vc));
      __builtin_nontemporal_store(v2, reinterpret_cast<u32x4*>(vc + a.half));
    }
  }
}

namespace {

bool valid_dtype(int32_t d) {
  return d == MI_DTYPE_BF16 || d == MI_DTYPE_F16 || d == MI_DTYPE_F32;
}

// The 16-byte kernels apply: 2-byte data with tables of the same dtype, head_dim
// a multiple of 16, unit head-dim strides, 16-byte aligned bases and rows.
bool vec_ok(int32_t dtype, int32_t cdtype, int64_t head_dim, int64_t n_rows, int64_t seq_len,
            std::initializer_list<const void*> ptrs,
            std::initializer_list<int64_t> unit, std::initializer_list<int64_t> strides) {
  if (dtype != cdtype || (dtype != MI_DTYPE_BF16 && dtype != MI_DTYPE_F16)) return false;
  if (head_dim % 16 != 0) return false;
  if (n_rows > INT32_MAX || seq_len * (head_dim / 16) > INT32_MAX) return false;
  for (const void* p : ptrs)
    if (p != nullptr && (uintptr_t)p % 16 != 0) return false;
  for (int64_t u : unit)
    if (u != 1) return false;
  for (int64_t r : strides)
    if ((r * 2) % 16 != 0) return false;
  return true;
}

// (x, y) grid of the 16-byte kernels: y over the batch x head rows, x over a
// row's tokens x 8-pair groups, both capped (the kernels loop over the rest).
dim3 vec_grid(int64_t rows, int64_t per_row) {
  int64_t gx = (per_row + 255) / 256, gy = rows;
  if (gx > 4096) gx = 4096;
  if (gy > 65535) gy = 65535;
  return dim3((unsigned)(gx < 1 ? 1 : gx), (unsigned)(gy < 1 ? 1 : gy));
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
                           int64_t table_rows, int64_t batch, int64_t n_heads,
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
  if (table_rows < (positions != nullptr ? 1 : seq_len)) {
    set_last_error("rope: cos/sin have %lld rows, need %lld", (long long)table_rows,
                   (long long)(positions != nullptr ? 1 : seq_len));
    return MI_ERR_INVALID;
  }
  RopeArgs a{};
  a.x = x; a.out = out; a.cos = cos; a.sin = sin; a.positions = positions;
  a.rows = table_rows;
  a.x_sb = x_sb; a.x_sh = x_sh; a.x_ss = x_ss; a.x_sd = x_sd;
  a.o_sb = o_sb; a.o_sh = o_sh; a.o_ss = o_ss; a.o_sd = o_sd;
  a.c_ss = c_ss; a.c_sd = c_sd; a.s_ss = s_ss; a.s_sd = s_sd;
  a.B = (int32_t)batch; a.H = (int32_t)n_heads; a.S = (int32_t)seq_len;
  a.half = (int32_t)(head_dim / 2);
  if (vec_ok(dtype, cdtype, head_dim, batch * n_heads, seq_len, {x, out, cos, sin}, {x_sd, o_sd, c_sd, s_sd},
             {x_sb, x_sh, x_ss, o_sb, o_sh, o_ss, c_ss, s_ss})) {
    const dim3 grid = vec_grid(batch * n_heads, seq_len * (head_dim / 16)), block(256);
    if (dtype == MI_DTYPE_BF16)
      hipLaunchKernelGGL(rope_vec_kernel<bf16_t>, grid, block, 0, (hipStream_t)stream, a);
    else
      hipLaunchKernelGGL(rope_vec_kernel<f16_t>, grid, block, 0, (hipStream_t)stream, a);
  } else {
    MI_ROPE_DISPATCH(rope_kernel, a, total, (hipStream_t)stream);
  }
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
    int64_t table_rows, int64_t batch, int64_t n_kv_heads, int64_t seq_len, int64_t head_dim,
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
  if (cos != nullptr && table_rows < (cos_by_position ? 1 : seq_len)) {
    set_last_error("rope_kv_append: cos/sin have %lld rows, need %lld", (long long)table_rows,
                   (long long)(cos_by_position ? 1 : seq_len));
    return MI_ERR_INVALID;
  }
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
  a.rows = table_rows;
  a.B = (int32_t)batch; a.H = (int32_t)n_kv_heads; a.S = (int32_t)seq_len;
  a.half = (int32_t)(head_dim / 2);
  a.cos_by_pos = cos_by_position;
  if (vec_ok(dtype, cos == nullptr ? dtype : cdtype, head_dim, batch * n_kv_heads, seq_len,
             {xk, xv, cache_k, cache_v, cos, sin},
             {xk_sd, xv_sd, ck_sd, cv_sd, cos == nullptr ? 1 : c_sd, cos == nullptr ? 1 : s_sd},
             {xk_sb, xk_sh, xk_ss, xv_sb, xv_sh, xv_ss, ck_sb, ck_sh, ck_st, cv_sb, cv_sh, cv_st,
              cos == nullptr ? 0 : c_ss, cos == nullptr ? 0 : s_ss})) {
    const dim3 grid = vec_grid(batch * n_kv_heads, seq_len * (head_dim / 16)), block(256);
    if (dtype == MI_DTYPE_BF16)
      hipLaunchKernelGGL(rope_kv_append_vec_kernel<bf16_t>, grid, block, 0, (hipStream_t)stream, a);
    else
      hipLaunchKernelGGL(rope_kv_append_vec_kernel<f16_t>, grid, block, 0, (hipStream_t)stream, a);
  } else {
    MI_ROPE_DISPATCH(rope_kv_append_kernel, a, total, (hipStream_t)stream);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_last_error("rope_kv_append: launch failed: %s", hipGetErrorString(e));
    return (int32_t)e;
  }
  return MI_OK;
}
