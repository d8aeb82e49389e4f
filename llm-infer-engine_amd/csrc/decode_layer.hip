// Fused W8A16 kernels of one decode step (M <= 16 token rows).
//
// A decode step of the W8A16 Llama block (src/model_quantized.py:42-93 with
// src/model.py:39-127) is a chain of small matrix-vector products; run one
// launch per reference op, the step is dominated by launch gaps and by
// kernels too small to reach HBM bandwidth.  These kernels fold every
// elementwise neighbour of a projection into it:
//
//   rmsnorm -> wq | wk | wv -> RoPE(q), RoPE(k) + KV-cache append, v append
//   wo -> + residual
//   rmsnorm -> w1 | w3 -> silu(w1 x) * (w3 x)
//   w2 -> + residual
//
// Arithmetic follows the reference op by op: RMSNorm in fp32 rounded once to
// the activation dtype (src/rms_norm.py:32-38); each projection accumulates
// x.f32 * q.f32 in fp32 and applies the row scale after the sum
// (src/quant_linear.py:37-57), rounded to the activation dtype; RoPE,
// residual adds and silu/mul then act on those rounded values exactly as the
// reference's separate ops do (src/rope.py:85-86, src/model.py:23, :113-127).
//
// GEMV design (MI355X): the int8 weights are the only large operand and are
// read once.  A workgroup owns a tile of RPB (8 or 16) output rows of one (or,
// for SwiGLU, two) weight matrices; its NW waves split K.  The products run on
// v_mfma_f32_16x16x32_{bf16,f16}: the A operand is 16 weight rows x 32 k
// (int8 converted exactly in registers), the B operand is x^T with the
// columns beyond M zero.  Each lane loads 16 contiguous int8 of one row; a
// wave issues every weight load of its K slice before its first MFMA, so the
// whole matrix is in flight at once (these GEMVs are latency-bound: a few MB
// each).  With the RMSNorm prologue the normalised rows are staged in LDS and
// the B operands are read from there; otherwise straight from global memory.
#include <math.h>
#include <type_traits>

#include "common.hpp"

namespace mi {

enum : int32_t {
  kEpiStore = 0,     // y = round(acc * s)
  kEpiResidual = 1,  // y = round(res + round(acc * s))
  kEpiSwiglu = 2,    // y = round(round(silu(a)) * b), a/b = rounded w1/w3 outputs
  kEpiQkvRope = 3,   // q -> RoPE -> q_out; k -> RoPE -> cache_k[pos]; v -> cache_v[pos]
};

struct LayerGemvArgs {
  const void* x;        // [M, K], unit k stride, row stride x_sm
  const void* norm_w;   // [K] RMSNorm weight (prologue) or null
  float eps;
  const int8_t* w0;     // first matrix [N0, K] (QKV: wq; SwiGLU: w1)
  const int8_t* w1;     // second matrix (QKV: wk; SwiGLU: w3) or null
  const int8_t* w2;     // third matrix (QKV: wv) or null
  const void* s0;       // row scales of w0 / w1 / w2
  const void* s1;
  const void* s2;
  int64_t w_sn0, w_sn1, w_sn2;  // weight row strides (bytes)
  void* y;              // output [M, N] (store / residual / swiglu) or q_out
  const void* res;      // residual [M, N]
  int64_t x_sm, y_sm, res_sm;
  int32_t M, K, N;      // N: output rows (QKV: Hq*D)
  int32_t n_tiles0;     // QKV: tiles of wq (the rest are wk then wv)
  int32_t n_tiles1;
  int32_t pair_kv;      // QKV with two tiles per block: wk / wv tiles paired too
  // QKV + RoPE + append
  const void* cos;      // [rows, D/2] tables, row stride c_ss (elements); position
  const void* sin;      //   p uses row p - rope_row0
  int64_t c_ss, rope_row0, rope_rows;
  const int64_t* pos;   // device position (one for all rows)
  void* ck;             // cache views of this layer: element (m, h, p, d) at
  void* cv;             //   m*c_sb + h*c_sh + p*c_st + d
  int64_t c_sb, c_sh, c_st;
  int64_t capacity;     // T
  int32_t Hq, Hkv, D;
};

template <typename T> struct LMfma;
template <> struct LMfma<bf16_t> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  __device__ static inline f32x4 mma(const v8& a, const v8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct LMfma<f16_t> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  __device__ static inline f32x4 mma(const v8& a, const v8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// 8 signed bytes (two words) -> 8 activation-dtype values (exact).
template <typename T, typename V8>
__device__ inline V8 i8x8_cvt(uint32_t lo, uint32_t hi) {
  if constexpr (std::is_same<T, bf16_t>::value) {
    // integers of magnitude <= 128 have 8 significant bits: the fp32 upper
    // halves are the bf16 values, so pair them with one byte permute
    auto hi2 = [](float a, float b) {
      return __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x07060302u);
    };
    u32x4 r;
    r.x = hi2((float)(int8_t)lo, (float)(int8_t)(lo >> 8));
    r.y = hi2((float)(int8_t)(lo >> 16), (float)(int8_t)(lo >> 24));
    r.z = hi2((float)(int8_t)hi, (float)(int8_t)(hi >> 8));
    r.w = hi2((float)(int8_t)(hi >> 16), (float)(int8_t)(hi >> 24));
    return __builtin_bit_cast(V8, r);
  } else {
    V8 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      r[i] = (T)(float)(int8_t)(lo >> (8 * i));
      r[4 + i] = (T)(float)(int8_t)(hi >> (8 * i));
    }
    return r;
  }
}


// x from lane (lane ^ OFF) without LDS traffic: a DPP row rotate for 8 (a
// 16-lane row rotated by 8 is the xor), the gfx950 permlane swaps for 16 and 32.
template <int OFF>
__device__ inline float dl_lane_xor(float x, int lane) {
  if constexpr (OFF == 8) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xF, 0xF, true));
  } else if constexpr (OFF == 16) {
    auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                               false);
    return __uint_as_float((lane & 16) ? sw[0] : sw[1]);
  } else {
    static_assert(OFF == 32, "lane stride");
    auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                               false);
    return __uint_as_float((lane & 32) ? sw[0] : sw[1]);
  }
}

// Weight row of tile row r (0..15) for tile `tile`: rows 0..RPB-1 of the tile;
// for the RoPE epilogue a tile holds 8 rotation pairs: rows i and i+8 are head
// dims d and d + D/2.
template <int EPI, int RPB>
__device__ inline int tile_row(int tile_in_mat, int r, int D) {
  if constexpr (EPI == kEpiQkvRope) {
    const int half = D >> 1, tiles_per_head = half >> 3;
    const int head = tile_in_mat / tiles_per_head, j = tile_in_mat % tiles_per_head;
    return head * D + 8 * j + (r & 7) + ((r >> 3) ? half : 0);
  } else {
    return tile_in_mat * RPB + r;
  }
}

template <typename T, int NW, bool NORM, int EPI, int RPB, int MR>
__global__ __launch_bounds__(64 * NW) void layer_gemv_kernel(LayerGemvArgs a) {
  using MM = LMfma<T>;
  typedef typename MM::v8 v8;
  constexpr int NMAT = EPI == kEpiSwiglu ? 2 : 1;      // A streams per tile
  constexpr int MAXC = 8;          // 64-k chunks per wave: K = 512 * NW (host-checked)
  // MR: rows of x the RMSNorm prologue holds (>= M)
  extern __shared__ __align__(16) unsigned char smem[];
  T* xs = reinterpret_cast<T*>(smem);                   // NORM: [M][K] normalised x
  float* red_ss = reinterpret_cast<float*>(smem + (NORM ? (size_t)a.M * a.K * sizeof(T) : 0));
  f32x4* red = reinterpret_cast<f32x4*>(smem + (NORM ? (size_t)a.M * a.K * sizeof(T) +
                                                           (size_t)NW * MR * sizeof(float)
                                                     : 0));

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;    // A: weight row in tile / k group
  const int m = lane & 15;                   // B: x row
  const bool m_ok = m < a.M;

  // ---- RMSNorm prologue, part 1: this thread's 16-byte column chunk of every
  //      x row (and of the norm weight), requested before any weight load so
  //      the statistics do not wait behind the weight stream (vmcnt retires
  //      in order).  K = 8 * 64 * NW: one chunk per thread per row.
  //      Every load in this kernel is unconditional (rows beyond M or N read
  //      a clamped row and are discarded by the epilogue): a load under a
  //      branch forces the compiler's vmcnt waits to assume it was skipped,
  //      which would make the first wait cover the whole weight stream.
  u32x4 xv[NORM ? MR : 1], nwv = {0, 0, 0, 0};
  if constexpr (NORM) {
#pragma unroll
    for (int row = 0; row < MR; ++row)
      xv[row] = load16(reinterpret_cast<const T*>(a.x) + (int64_t)min(row, a.M - 1) * a.x_sm +
                       tid * 8);
    nwv = load16(reinterpret_cast<const T*>(a.norm_w) + tid * 8);
  }

  // device position of the QKV epilogue (a scalar load, needed for the
  // RoPE table addresses below)
  const int64_t pos = EPI == kEpiQkvRope ? *a.pos : 0;

  // ---- which matrix / tile this block owns
  int tile = blockIdx.x;
  int mat = 0;
  if constexpr (EPI == kEpiQkvRope) {
    if (tile >= a.n_tiles0) {
      tile -= a.n_tiles0;
      mat = 1;
      if (tile >= a.n_tiles1) { tile -= a.n_tiles1; mat = 2; }
    }
  }
  const int8_t* wm = mat == 0 ? a.w0 : (mat == 1 ? a.w1 : a.w2);
  const int64_t w_sn = mat == 0 ? a.w_sn0 : (mat == 1 ? a.w_sn1 : a.w_sn2);
  const int n_in_mat = tile_row<EPI, RPB>(tile, r, a.D);   // this lane's weight row
  const int n_valid = EPI == kEpiQkvRope ? (mat == 0 ? a.Hq : a.Hkv) * a.D : a.N;
  const bool row_ok = r < RPB && n_in_mat < n_valid;
  // weight rows through buffer resources (host-checked: the matrix spans < 2^31 bytes):
  // lanes of padding rows (r >= RPB, n >= N) get an out-of-range offset and
  // load zeros without a memory access
  const buf_rsrc wr0 = make_rsrc(wm, (uint32_t)((int64_t)(n_valid - 1) * w_sn + a.K));
  const uint32_t wo0 = row_ok ? (uint32_t)((int64_t)n_in_mat * w_sn) : kOobOffset;
  const buf_rsrc wr1 = make_rsrc(NMAT == 2 ? a.w1 : wm,
                                 NMAT == 2 ? (uint32_t)((int64_t)(a.N - 1) * a.w_sn1 + a.K) : 0u);
  const uint32_t wo1 = NMAT == 2 && row_ok ? (uint32_t)((int64_t)n_in_mat * a.w_sn1) : kOobOffset;

  // ---- without the prologue the B operands come straight from global memory:
  //      request them all first (L2 hits, they retire ahead of the weights)
  const int c_lo = w * MAXC;
  const int mc = min(m, a.M - 1);             // columns m >= M are discarded
  u32x4 xr[NORM ? 1 : MAXC][2];
  if constexpr (!NORM) {
    // x through a buffer resource (host-checked: ((M-1)*x_sm + K)*2 < 2^31):
    // the B-operand columns m >= M load zeros without a memory access
    const buf_rsrc xrs = make_rsrc(a.x, (uint32_t)(((int64_t)(a.M - 1) * a.x_sm + a.K) * sizeof(T)));
    const uint32_t xo = m_ok ? (uint32_t)((int64_t)m * a.x_sm * sizeof(T)) : kOobOffset;
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
      const int k0 = (c_lo + i) * 64 + 16 * g;
      xr[i][0] = buf_load16(xrs, xo + (uint32_t)(k0 * sizeof(T)));
      xr[i][1] = buf_load16(xrs, xo + (uint32_t)((k0 + 8) * sizeof(T)));
    }
  }

  // ---- issue every weight load of this wave's K slice (MAXC chunks of 64)
  u32x4 wq[NMAT][MAXC];
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int k0 = (c_lo + i) * 64 + 16 * g;
    wq[0][i] = buf_load16_nt(wr0, wo0 + (uint32_t)k0);
    if constexpr (NMAT == 2) wq[1][i] = buf_load16_nt(wr1, wo1 + (uint32_t)k0);
  }
  // ---- epilogue operands (row scales, residual, RoPE table entries), issued
  //      behind the weights so the epilogue does not start with a round trip;
  //      unconditional, from clamped indices (lanes beyond M / N discard them)
  T e_s0[4], e_s1[4], e_res[4], e_cos[4], e_sin[4];
  auto load_epilogue = [&]() {
  if constexpr (EPI == kEpiQkvRope) {
    const T* sc = reinterpret_cast<const T*>(mat == 0 ? a.s0 : (mat == 1 ? a.s1 : a.s2));
    const int half = a.D >> 1, tph = half >> 3;
    const int head = tile / tph, j8 = tile % tph;
    // rows outside the table are clamped (callers keep positions in range)
    const int64_t crow = min(max(pos - a.rope_row0, (int64_t)0), a.rope_rows - 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rr = 4 * g + i;
      e_s0[i] = sc[head * a.D + 8 * j8 + (rr & 7) + ((rr >> 3) ? half : 0)];
      const int ii = 8 * j8 + 4 * (g & 1) + i;
      e_cos[i] = reinterpret_cast<const T*>(a.cos)[crow * a.c_ss + ii];
      e_sin[i] = reinterpret_cast<const T*>(a.sin)[crow * a.c_ss + ii];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int nc = min(tile * RPB + 4 * g + i, a.N - 1);
      e_s0[i] = reinterpret_cast<const T*>(a.s0)[nc];
      if constexpr (EPI == kEpiSwiglu) e_s1[i] = reinterpret_cast<const T*>(a.s1)[nc];
      if constexpr (EPI == kEpiResidual)
        e_res[i] = reinterpret_cast<const T*>(a.res)[(int64_t)mc * a.res_sm + nc];
    }
  }
  };
  // 1024-thread blocks (128 VGPRs) with a prologue or two weight streams have
  // no registers to spare: they load these at the epilogue instead
  constexpr bool kPrefetchEpi = !(NW >= 16 && (NORM || NMAT == 2));
  if constexpr (kPrefetchEpi) load_epilogue();
  // keep the whole load stream issued before the prologue's first wait
  __builtin_amdgcn_sched_barrier(0);

  // ---- RMSNorm prologue, part 2: per-row sum of squares (wave shuffles, then
  //      LDS across waves), normalised rows into LDS, rounded to T
  if constexpr (NORM) {
    float ss[MR];
#pragma unroll
    for (int row = 0; row < MR; ++row) {
      float v[8];
      Chunk<T>::unpack(xv[row], v);
      float t = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) t = fmaf(v[e], v[e], t);
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) t += shfl_xor_f32(t, off);
      ss[row] = t;
    }
    if (lane == 0) {
#pragma unroll
      for (int row = 0; row < MR; ++row) red_ss[w * MR + row] = ss[row];
    }
    __syncthreads();
    float wn[8];
    Chunk<T>::unpack(nwv, wn);
#pragma unroll
    for (int row = 0; row < MR; ++row) {
      if (row < a.M) {
        float tot = 0.f;
  #pragma unroll
        for (int ww = 0; ww < NW; ++ww) tot += red_ss[ww * MR + row];
        const float rstd = 1.0f / sqrtf(tot / (float)a.K + a.eps);
        float v[8];
        Chunk<T>::unpack(xv[row], v);
        typedef T t8 __attribute__((ext_vector_type(8)));
        t8 o;
  #pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = Elem<T>::from_f32(v[e] * rstd * wn[e]);
        *reinterpret_cast<t8*>(xs + (int64_t)row * a.K + tid * 8) = o;
      }
    }
    __syncthreads();
  }

  // ---- MFMAs over the slice
  f32x4 acc[NMAT];
#pragma unroll
  for (int t = 0; t < NMAT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int k0 = (c_lo + i) * 64 + 16 * g;
    v8 xb0, xb1;
    if constexpr (NORM) {
      const T* xp = xs + (int64_t)mc * a.K + k0;
      xb0 = __builtin_bit_cast(v8, load16(xp));
      xb1 = __builtin_bit_cast(v8, load16(xp + 8));
    } else {
      xb0 = __builtin_bit_cast(v8, xr[i][0]);
      xb1 = __builtin_bit_cast(v8, xr[i][1]);
    }
#pragma unroll
    for (int t = 0; t < NMAT; ++t) {
      acc[t] = MM::mma(i8x8_cvt<T, v8>(wq[t][i].x, wq[t][i].y), xb0, acc[t]);
      acc[t] = MM::mma(i8x8_cvt<T, v8>(wq[t][i].z, wq[t][i].w), xb1, acc[t]);
    }
  }

  // ---- reduce the NW waves' partial sums
  if (w != 0) {
#pragma unroll
    for (int t = 0; t < NMAT; ++t) red[((w - 1) * NMAT + t) * 64 + lane] = acc[t];
  }
  __syncthreads();
  if (w != 0) return;
#pragma unroll
  for (int ww = 1; ww < NW; ++ww)
#pragma unroll
    for (int t = 0; t < NMAT; ++t) acc[t] += red[((ww - 1) * NMAT + t) * 64 + lane];

  if constexpr (!kPrefetchEpi) load_epilogue();
  // acc[t][i] = C[tile row 4*g + i][x row m]
  auto f32_of = [](T v) { return Elem<T>::to_f32(v); };
  if constexpr (EPI == kEpiQkvRope) {
    // rows 4g+i (g < 2) are dims d = 8j + 4g + i, their partners (rows +8) sit
    // in lane + 32: swap the rounded projections across the lane halves
    const int half = a.D >> 1, tph = half >> 3;
    const int head = tile / tph, j8 = tile % tph;
    float yv[4], yp[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      yv[i] = Elem<T>::to_f32(Elem<T>::from_f32(acc[0][i] * f32_of(e_s0[i])));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(yv[i]), __float_as_uint(yv[i]),
                                                 false, false);
      yp[i] = __uint_as_float(lane < 32 ? sw[1] : sw[0]);
    }
    if (!m_ok) return;
    const int64_t p = pos;
    const bool hi = g >= 2;                       // rows 8..15: second half of the pair
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ii = 8 * j8 + 4 * (g & 1) + i;    // rotation index, 0 <= ii < half
      const int d = ii + (hi ? half : 0);
      T out;
      if (mat == 2) {
        out = Elem<T>::from_f32(yv[i]);           // v: appended unrotated (bitwise)
      } else {
        const float cs = f32_of(e_cos[i]), sn = f32_of(e_sin[i]);
        const float x1 = hi ? yp[i] : yv[i], x2 = hi ? yv[i] : yp[i];
        T y1, y2;
        {
#pragma clang fp contract(off)
          const float x1c = x1 * cs, x2s = x2 * sn, x2c = x2 * cs, x1s = x1 * sn;
          y1 = Elem<T>::from_f32(x1c - x2s);
          y2 = Elem<T>::from_f32(x2c + x1s);
        }
        out = hi ? y2 : y1;
      }
      if (mat == 0) {
        reinterpret_cast<T*>(a.y)[((int64_t)m * a.Hq + head) * a.D + d] = out;
      } else if (p >= 0 && p < a.capacity) {
        T* c = reinterpret_cast<T*>(mat == 1 ? a.ck : a.cv);
        c[(int64_t)m * a.c_sb + (int64_t)head * a.c_sh + p * a.c_st + d] = out;
      }
    }
  } else {
    if (!m_ok) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rr = 4 * g + i;
      const int n = tile * RPB + rr;
      if (rr >= RPB || n >= a.N) continue;
      float v = Elem<T>::to_f32(Elem<T>::from_f32(acc[0][i] * f32_of(e_s0[i])));
      if constexpr (EPI == kEpiResidual) {
        v = Elem<T>::to_f32(Elem<T>::from_f32(f32_of(e_res[i]) + v));
      } else if constexpr (EPI == kEpiSwiglu) {
        const float b = Elem<T>::to_f32(Elem<T>::from_f32(acc[1][i] * f32_of(e_s1[i])));
        const float sa = Elem<T>::to_f32(Elem<T>::from_f32(silu_f32(v)));
        v = sa * b;
      }
      reinterpret_cast<T*>(a.y)[(int64_t)m * a.y_sm + n] = Elem<T>::from_f32(v);
    }
  }
}

// ---------------------------------------------------------------------------
// Diagonal-packed GEMV for M <= 8 token rows.
//
// One v_mfma_f32_16x16x32 multiplies a 16 x 32 A tile by a 32 x 16 B tile.
// With at most 8 token rows half of B's columns would be padding, and an
// 8-row weight tile half of A's rows; padding lanes still cost the CU's
// vector-memory issue (about 64 bytes per clock per CU, the limit of these
// small GEMVs once the weight stream is in flight).  Here both halves carry
// data: A lanes of rows r < 8 hold weight row n(r) over the first 64 k of a
// 128-k superchunk, rows r >= 8 the same weight rows over the second 64 k; B
// columns c < 8 hold token row c over the first 64 k, columns c >= 8 token row
// c - 8 over the second.  C[r][c] + C[r + 8][c + 8] (r, c < 8) is then the
// 128-k dot product and the off-diagonal quadrants are discarded: every byte
// loaded is used.
//
// A block has NW waves splitting K (SC consecutive superchunks each, K =
// 128 * NW * SC) and owns TPB 8-row tiles of each of its NMAT matrices.  With
// the RMSNorm prologue each wave normalises its own x slice in registers (the
// row statistics meet once in LDS).  Each wave folds its diagonal quadrants
// in registers, the waves' sums meet in LDS, and one thread per (token row,
// output row) sums them and runs the epilogue.
template <typename T, int NW, int SC, bool NORM, int EPI, int TPB>
__global__ __launch_bounds__(64 * NW) void dgemv_kernel(LayerGemvArgs a) {
  using MM = LMfma<T>;
  typedef typename MM::v8 v8;
  constexpr int NMAT = EPI == kEpiSwiglu ? 2 : 1;
  constexpr int NT = NMAT * TPB;                       // 8-row A tiles per block
  constexpr int RB = 8 * TPB;                          // output rows per block (per matrix)
  constexpr int NOUT = EPI == kEpiQkvRope ? 64 * TPB : 8 * RB;  // epilogue threads
  static_assert(NOUT <= 64 * NW, "too few threads for the epilogue");
  __shared__ __align__(16) float red[NT][8][8][NW];    // [tile][row][token][wave]
  __shared__ float ssq[NORM ? NW : 1][8];              // per-wave sums of squares

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int rr = r16 & 7;                // A: tile row / B: token row
  const int kofs = (r16 >> 3) * 64 + 16 * g;
  const bool m_ok = rr < a.M;
  // K slice of this wave, rotated by block so that concurrent blocks do not all
  // read the same x lines at the same time
  const int ks = (w + (int)blockIdx.x) % NW;
  const int kw = ks * SC * 128;

  // ---- which matrix / tiles this block owns.  QKV: one tile per block, or
  //      (TPB = 2) tiles 2b and 2b + 1 of wq for the first ceil(n_tiles0 / 2)
  //      blocks, then the wk and the wv tiles one per block (or in pairs with
  //      pair_kv).  A CU that runs two blocks streams x twice and sets the
  //      launch's time, so grids with more tiles than CUs pair them (ntv: the
  //      tiles this block really has; a missing second tile loads zeros)
  int mat0 = 0, tile0 = blockIdx.x * TPB, ntv = TPB;
  if constexpr (EPI == kEpiQkvRope) {
    int b = blockIdx.x;
    const int per0 = TPB == 2 ? (a.n_tiles0 + 1) >> 1 : a.n_tiles0;
    const bool pkv = TPB == 2 && a.pair_kv != 0;
    const int per1 = pkv ? (a.n_tiles1 + 1) >> 1 : a.n_tiles1;
    int nt = a.n_tiles0;
    if (b >= per0) {
      b -= per0;
      mat0 = 1;
      if (b >= per1) { b -= per1; mat0 = 2; }
      nt = a.n_tiles1;
    }
    const bool paired = TPB == 2 && (mat0 == 0 || pkv);
    tile0 = paired ? 2 * b : b;
    ntv = paired ? min(2, nt - tile0) : 1;
  }
  const int half = a.D >> 1, tph = EPI == kEpiQkvRope ? half >> 2 : 1;
  // weight row of tile row `row` of tile `tim` of the matrix: the QKV tiles hold
  // 4 rotation pairs (rows 0..3 dims d, rows 4..7 dims d + D/2)
  auto w_row = [&](int tim, int row) -> int {
    if constexpr (EPI == kEpiQkvRope) {
      const int head = tim / tph, j = tim - head * tph;
      return head * a.D + 4 * j + (row & 3) + ((row >> 2) ? half : 0);
    } else {
      return tim * 8 + row;
    }
  };
  const int8_t* wm0 = mat0 == 0 ? a.w0 : (mat0 == 1 ? a.w1 : a.w2);
  const int64_t wsn0 = mat0 == 0 ? a.w_sn0 : (mat0 == 1 ? a.w_sn1 : a.w_sn2);
  const int nvalid = EPI == kEpiQkvRope ? (mat0 == 0 ? a.Hq : a.Hkv) * a.D : a.N;
  // weight rows through buffer resources (host-checked: each matrix spans
  // < 2^31 bytes); rows past N get an out-of-range offset and load zeros
  buf_rsrc wr[NMAT];
  wr[0] = make_rsrc(wm0, (uint32_t)((int64_t)(nvalid - 1) * wsn0 + a.K));
  if constexpr (NMAT == 2) wr[1] = make_rsrc(a.w1, (uint32_t)((int64_t)(a.N - 1) * a.w_sn1 + a.K));
  uint32_t woff[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int n = w_row(tile0 + (t % TPB), rr);
    const int64_t sn = t / TPB == 0 ? wsn0 : a.w_sn1;
    woff[t] = (n < nvalid && (t % TPB) < ntv) ? (uint32_t)((int64_t)n * sn) : kOobOffset;
  }

  // ---- B operand (token rows through a buffer resource: rows >= M read zeros
  //      without a memory access), then the norm weights, then every weight
  //      load of this wave; all issued before the first wait
  const buf_rsrc xrs =
      make_rsrc(a.x, (uint32_t)(((int64_t)(a.M - 1) * a.x_sm + a.K) * sizeof(T)));
  const uint32_t xo = m_ok ? (uint32_t)((int64_t)rr * a.x_sm * sizeof(T)) : kOobOffset;
  u32x4 xr[SC][2];
#pragma unroll
  for (int s = 0; s < SC; ++s) {
    const int k0 = kw + s * 128 + kofs;
    xr[s][0] = buf_load16(xrs, xo + (uint32_t)(k0 * sizeof(T)));
    xr[s][1] = buf_load16(xrs, xo + (uint32_t)((k0 + 8) * sizeof(T)));
  }
  u32x4 nr[NORM ? SC : 1][2];
  if constexpr (NORM) {
#pragma unroll
    for (int s = 0; s < SC; ++s) {
      const T* np = reinterpret_cast<const T*>(a.norm_w) + kw + s * 128 + kofs;
      nr[s][0] = load16(np);
      nr[s][1] = load16(np + 8);
    }
  }
  u32x4 wq[NT][SC];
#pragma unroll
  for (int s = 0; s < SC; ++s)
#pragma unroll
    for (int t = 0; t < NT; ++t)
      wq[t][s] = buf_load16_nt(wr[t / TPB], woff[t] + (uint32_t)(kw + s * 128 + kofs));

  // ---- epilogue operands, behind the weights (every thread loads from
  //      clamped indices; only threads < NOUT use them)
  const int et = tid % NOUT;
  T e_s0, e_s1, e_res, e_cos, e_sin;
  int64_t pos = 0;
  if constexpr (EPI == kEpiQkvRope) {
    pos = *a.pos;
    const T* sc = reinterpret_cast<const T*>(mat0 == 0 ? a.s0 : (mat0 == 1 ? a.s1 : a.s2));
    const int tt = tile0 + min(et >> 6, ntv - 1);   // this epilogue thread's tile
    const int row = et & 7, j = tt % tph;
    e_s0 = sc[w_row(tt, row)];
    e_s1 = sc[w_row(tt, row ^ 4)];
    const int64_t crow = min(max(pos - a.rope_row0, (int64_t)0), a.rope_rows - 1);
    const int ii = 4 * j + (row & 3);
    e_cos = reinterpret_cast<const T*>(a.cos)[crow * a.c_ss + ii];
    e_sin = reinterpret_cast<const T*>(a.sin)[crow * a.c_ss + ii];
  } else {
    const int em = min(et / RB, a.M - 1);
    const int en = min(blockIdx.x * RB + et % RB, a.N - 1);
    e_s0 = reinterpret_cast<const T*>(a.s0)[en];
    if constexpr (EPI == kEpiSwiglu) e_s1 = reinterpret_cast<const T*>(a.s1)[en];
    if constexpr (EPI == kEpiResidual)
      e_res = reinterpret_cast<const T*>(a.res)[(int64_t)em * a.res_sm + en];
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- RMSNorm: per-token-row sum of squares over this lane's k (lanes c,
  //      c ^ 8 and every k group share a token row), over waves in LDS; then
  //      x * rstd * w rounded once to T, in place
  if constexpr (NORM) {
    float ss = 0.f;
#pragma unroll
    for (int s = 0; s < SC; ++s)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float v[8];
        Chunk<T>::unpack(xr[s][h], v);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(v[e], v[e], ss);
      }
    ss += dl_lane_xor<8>(ss, lane);
    ss += dl_lane_xor<16>(ss, lane);
    ss += dl_lane_xor<32>(ss, lane);
    if (lane < 8) ssq[w][lane] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) tot += ssq[ww][rr];
    const float rstd = 1.0f / sqrtf(tot / (float)a.K + a.eps);
#pragma unroll
    for (int s = 0; s < SC; ++s)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float v[8], wn[8];
        Chunk<T>::unpack(xr[s][h], v);
        Chunk<T>::unpack(nr[s][h], wn);
        typedef T t8 __attribute__((ext_vector_type(8)));
        t8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = Elem<T>::from_f32(v[e] * rstd * wn[e]);
        xr[s][h] = __builtin_bit_cast(u32x4, o);
      }
  }

  // ---- MFMAs over the wave's superchunks
  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < SC; ++s) {
    const v8 xb0 = __builtin_bit_cast(v8, xr[s][0]);
    const v8 xb1 = __builtin_bit_cast(v8, xr[s][1]);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      acc[t] = MM::mma(i8x8_cvt<T, v8>(wq[t][s].x, wq[t][s].y), xb0, acc[t]);
      acc[t] = MM::mma(i8x8_cvt<T, v8>(wq[t][s].z, wq[t][s].w), xb1, acc[t]);
    }
  }

  // ---- fold the diagonal quadrants: lane c + 16 g (g < 2, c < 8) holds
  //      C[4g + i][c], lane + 40 holds C[4g + i + 8][c + 8]
#pragma unroll
  for (int t = 0; t < NT; ++t) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v = acc[t][i] + dl_lane_xor<8>(dl_lane_xor<32>(acc[t][i], lane), lane);
      if (g < 2 && r16 < 8) red[t][4 * g + i][r16][w] = v;
    }
  }
  __syncthreads();
  if (tid >= NOUT) return;

  // sum over waves of tile t, row `row`, token row `mm`
  auto wsum = [&](int t, int row, int mm) -> float {
    const f32x4* p = reinterpret_cast<const f32x4*>(&red[t][row][mm][0]);
    float acc_s = 0.f;
#pragma unroll
    for (int q = 0; q < NW / 4; ++q) {
      const f32x4 v = p[q];
      acc_s += v[0] + v[1] + v[2] + v[3];
    }
    return acc_s;
  };
  auto f32_of = [](T v) { return Elem<T>::to_f32(v); };
  auto rnd = [](float v) { return Elem<T>::to_f32(Elem<T>::from_f32(v)); };

  if constexpr (EPI == kEpiQkvRope) {
    const int te = tid >> 6, mm = (tid >> 3) & 7, row = tid & 7;
    if (mm >= a.M || te >= ntv) return;
    const int tt = tile0 + te;
    const float yv = rnd(wsum(te, row, mm) * f32_of(e_s0));
    const float yp = rnd(wsum(te, row ^ 4, mm) * f32_of(e_s1));
    const bool hi = row >= 4;
    const int head = tt / tph;
    const int d = w_row(tt, row) - head * a.D;
    T out;
    if (mat0 == 2) {
      out = Elem<T>::from_f32(yv);                  // v: appended unrotated (bitwise)
    } else {
      const float cs = f32_of(e_cos), sn = f32_of(e_sin);
      const float x1 = hi ? yp : yv, x2 = hi ? yv : yp;
      T y1, y2;
      {
#pragma clang fp contract(off)
        const float x1c = x1 * cs, x2s = x2 * sn, x2c = x2 * cs, x1s = x1 * sn;
        y1 = Elem<T>::from_f32(x1c - x2s);
        y2 = Elem<T>::from_f32(x2c + x1s);
      }
      out = hi ? y2 : y1;
    }
    if (mat0 == 0) {
      reinterpret_cast<T*>(a.y)[((int64_t)mm * a.Hq + head) * a.D + d] = out;
    } else if (pos >= 0 && pos < a.capacity) {
      T* c = reinterpret_cast<T*>(mat0 == 1 ? a.ck : a.cv);
      c[(int64_t)mm * a.c_sb + (int64_t)head * a.c_sh + pos * a.c_st + d] = out;
    }
  } else {
    const int mm = tid / RB, j = tid - mm * RB;
    const int n = blockIdx.x * RB + j;
    if (mm >= a.M || n >= a.N) return;
    float v = rnd(wsum(j >> 3, j & 7, mm) * f32_of(e_s0));
    if constexpr (EPI == kEpiResidual) {
      v = rnd(f32_of(e_res) + v);
    } else if constexpr (EPI == kEpiSwiglu) {
      const float b = rnd(wsum(TPB + (j >> 3), j & 7, mm) * f32_of(e_s1));
      v = rnd(silu_f32(v)) * b;
    }
    reinterpret_cast<T*>(a.y)[(int64_t)mm * a.y_sm + n] = Elem<T>::from_f32(v);
  }
}

namespace {

template <typename T, int NW, bool NORM, int EPI, int RPB, int MR>
hipError_t launch_layer_gemv(const LayerGemvArgs& a, int n_blocks, hipStream_t st) {
  size_t smem = (size_t)(NW - 1) * (EPI == kEpiSwiglu ? 2 : 1) * 64 * sizeof(f32x4);
  if (NORM) smem += (size_t)a.M * a.K * sizeof(T) + (size_t)NW * MR * sizeof(float);
  hipLaunchKernelGGL((layer_gemv_kernel<T, NW, NORM, EPI, RPB, MR>), dim3((unsigned)n_blocks),
                     dim3(64 * NW), smem, st, a);
  return hipGetLastError();
}

// Waves per block: K = 512 * NW (each wave owns 8 chunks of 64 k).  The
// RMSNorm prologue keeps MR (8 or 16 >= M) rows of one column chunk per thread.
template <typename T, bool NORM, int EPI, int RPB>
hipError_t dispatch_nw(const LayerGemvArgs& a, int n_blocks, hipStream_t st) {
  constexpr int MR = 8;
  if (NORM && a.M > MR) {
    switch (a.K) {
      case 512: return launch_layer_gemv<T, 1, NORM, EPI, RPB, 16>(a, n_blocks, st);
      case 1024: return launch_layer_gemv<T, 2, NORM, EPI, RPB, 16>(a, n_blocks, st);
      case 2048: return launch_layer_gemv<T, 4, NORM, EPI, RPB, 16>(a, n_blocks, st);
      default: return hipErrorInvalidValue;  // host checks exclude the rest
    }
  }
  switch (a.K) {
    case 512: return launch_layer_gemv<T, 1, NORM, EPI, RPB, MR>(a, n_blocks, st);
    case 1024: return launch_layer_gemv<T, 2, NORM, EPI, RPB, MR>(a, n_blocks, st);
    case 1536: return launch_layer_gemv<T, 3, NORM, EPI, RPB, MR>(a, n_blocks, st);
    case 2048: return launch_layer_gemv<T, 4, NORM, EPI, RPB, MR>(a, n_blocks, st);
    case 3072: return launch_layer_gemv<T, 6, NORM, EPI, RPB, MR>(a, n_blocks, st);
    case 4096: return launch_layer_gemv<T, 8, NORM, EPI, RPB, MR>(a, n_blocks, st);
    default: break;
  }
  if constexpr (EPI != kEpiSwiglu) {  // two weight streams: K <= 4096 (host-checked)
    switch (a.K) {
      case 6144: return launch_layer_gemv<T, 12, NORM, EPI, RPB, MR>(a, n_blocks, st);
      case 8192: return launch_layer_gemv<T, 16, NORM, EPI, RPB, MR>(a, n_blocks, st);
      default: break;
    }
  }
  return hipErrorInvalidValue;
}

template <typename T, int EPI, int RPB>
hipError_t dispatch_norm(const LayerGemvArgs& a, int n_blocks, hipStream_t st) {
  return a.norm_w != nullptr ? dispatch_nw<T, true, EPI, RPB>(a, n_blocks, st)
                             : dispatch_nw<T, false, EPI, RPB>(a, n_blocks, st);
}

// Row tiles of 16 when that already makes a few hundred blocks, else of 8
// (the A rows beyond 8 are zero) so that small-N projections use every CU.
template <typename T, int EPI>
hipError_t dispatch_tile(const LayerGemvArgs& a, hipStream_t st) {
  if (a.N / 16 >= 240) return dispatch_norm<T, EPI, 16>(a, (a.N + 15) / 16, st);
  return dispatch_norm<T, EPI, 8>(a, (a.N + 7) / 8, st);
}

// Diagonal-packed kernel (M <= 8): waves and superchunks per wave from K =
// 128 * NW * SC, at most 16 waves.
template <typename T, bool NORM, int EPI, int TPB, int NW, int SC>
hipError_t launch_dg(const LayerGemvArgs& a, int n_blocks, hipStream_t st) {
  hipLaunchKernelGGL((dgemv_kernel<T, NW, SC, NORM, EPI, TPB>), dim3((unsigned)n_blocks),
                     dim3(64 * NW), 0, st, a);
  return hipGetLastError();
}

template <typename T, bool NORM, int EPI, int TPB>
hipError_t dispatch_dg_k(const LayerGemvArgs& a, int n_blocks, hipStream_t st) {
  switch (a.K) {
    case 512: return launch_dg<T, NORM, EPI, TPB, 4, 1>(a, n_blocks, st);
    case 1024: return launch_dg<T, NORM, EPI, TPB, 8, 1>(a, n_blocks, st);
    case 1536: return launch_dg<T, NORM, EPI, TPB, 12, 1>(a, n_blocks, st);
    // K = 2048 (the 1B model's projections from the residual stream): fewer,
    // longer waves pay the per-wave set-up, RMSNorm statistics and cross-wave
    // reduction less often.  One MI355X, M = 8, per call in a 16-layer graph:
    // wo + residual 4.03 -> 3.75 us (16 x 1 -> 4 x 4), w1|w3 + SwiGLU 11.2 ->
    // 9.9 us (8 x 2), RMSNorm + QKV + RoPE + append about 0.85 us less (4 x 4).
    case 2048:
      if constexpr (EPI == kEpiSwiglu) return launch_dg<T, NORM, EPI, TPB, 8, 2>(a, n_blocks, st);
      else return launch_dg<T, NORM, EPI, TPB, 4, 4>(a, n_blocks, st);
    case 3072: return launch_dg<T, NORM, EPI, TPB, 12, 2>(a, n_blocks, st);
    case 4096: return launch_dg<T, NORM, EPI, TPB, 16, 2>(a, n_blocks, st);
    default: break;
  }
  if constexpr (EPI != kEpiSwiglu) {  // two weight streams: K <= 4096 (host-checked)
    switch (a.K) {
      case 6144: return launch_dg<T, NORM, EPI, TPB, 16, 3>(a, n_blocks, st);
      case 8192: return launch_dg<T, NORM, EPI, TPB, 16, 4>(a, n_blocks, st);
      default: break;
    }
  }
  return hipErrorInvalidValue;
}

template <typename T, int EPI, int TPB>
hipError_t dispatch_dg(const LayerGemvArgs& a, int n_blocks, hipStream_t st) {
  return a.norm_w != nullptr ? dispatch_dg_k<T, true, EPI, TPB>(a, n_blocks, st)
                             : dispatch_dg_k<T, false, EPI, TPB>(a, n_blocks, st);
}

// Store / residual / SwiGLU projections: the diagonal-packed kernel for M <= 8
// (one 8-row tile per block; SwiGLU two tiles of each matrix), else the
// 16-column kernel above.
template <typename T, int EPI>
hipError_t dispatch_linear(const LayerGemvArgs& a, hipStream_t st) {
  if (a.M <= 8) {
    constexpr int TPB = EPI == kEpiSwiglu ? 2 : 1;
    return dispatch_dg<T, EPI, TPB>(a, (a.N + 8 * TPB - 1) / (8 * TPB), st);
  }
  return dispatch_tile<T, EPI>(a, st);
}

bool k_supported(int64_t K) {
  return K == 512 || K == 1024 || K == 1536 || K == 2048 || K == 3072 || K == 4096 ||
         K == 6144 || K == 8192;
}

int32_t check_x(const void* x, int64_t M, int64_t K, int64_t x_sm, const void* norm_w,
                int32_t dtype, const char* what) {
  if (x == nullptr) {
    set_last_error("%s: null x", what);
    return MI_ERR_INVALID;
  }
  if (dtype != MI_DTYPE_BF16 && dtype != MI_DTYPE_F16) {
    set_last_error("%s: activations must be bf16 or fp16 (dtype %d)", what, (int)dtype);
    return MI_ERR_UNSUPPORTED;
  }
  if (M < 1 || M > 16 || !k_supported(K)) {
    set_last_error("%s: need 1 <= M <= 16 and K in {512, 1024, 1536, 2048, 3072, 4096, 6144, "
                   "8192} (M=%lld K=%lld)", what, (long long)M, (long long)K);
    return MI_ERR_UNSUPPORTED;
  }
  if ((uintptr_t)x % 16 != 0 || (x_sm * 2) % 16 != 0) {
    set_last_error("%s: x rows must be 16-byte aligned", what);
    return MI_ERR_INVALID;
  }
  if (x_sm < 0 || ((M - 1) * x_sm + K) * 2 >= ((int64_t)1 << 31)) {
    set_last_error("%s: x row stride %lld out of range (x must span < 2 GB)", what,
                   (long long)x_sm);
    return MI_ERR_UNSUPPORTED;
  }
  if (norm_w != nullptr && ((uintptr_t)norm_w % 16 != 0 || M * K * 2 > 64 * 1024 ||
                            (M > 8 && K > 2048))) {
    set_last_error("%s: RMSNorm prologue needs a 16-byte aligned weight, M*K*2 <= 64 KB and "
                   "K <= 2048 for M > 8", what);
    return MI_ERR_UNSUPPORTED;
  }
  return MI_OK;
}

int32_t check_w(const int8_t* w, const void* s, int64_t w_sn, int64_t rows, int64_t K,
                const char* what) {
  if (w == nullptr || s == nullptr) {
    set_last_error("%s: null weight or scales", what);
    return MI_ERR_INVALID;
  }
  if ((uintptr_t)w % 16 != 0 || w_sn % 16 != 0) {
    set_last_error("%s: weight rows must be 16-byte aligned", what);
    return MI_ERR_UNSUPPORTED;
  }
  // weight loads use 32-bit byte offsets into the matrix
  if (w_sn < 0 || (rows - 1) * w_sn + K >= ((int64_t)1 << 31)) {
    set_last_error("%s: weight matrix out of range (%lld rows x %lld-byte stride must span "
                   "< 2 GB)", what, (long long)rows, (long long)w_sn);
    return MI_ERR_UNSUPPORTED;
  }
  return MI_OK;
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int32_t mi_w8a16_linear_fused(
    const void* x, int64_t x_sm, const void* norm_w, float eps, const int8_t* w_a,
    const void* s_a, int64_t w_sn_a, const int8_t* w_b, const void* s_b, int64_t w_sn_b,
    const void* res, int64_t res_sm, void* y, int64_t y_sm, int64_t M, int64_t N, int64_t K,
    int32_t epilogue, int32_t dtype, void* stream) {
  const char* what = "w8a16_linear_fused";
  int32_t st = check_x(x, M, K, x_sm, norm_w, dtype, what);
  if (st != MI_OK) return st;
  if ((st = check_w(w_a, s_a, w_sn_a, N, K, what)) != MI_OK) return st;
  if (y == nullptr || N < 1 || N > INT32_MAX - 16) {
    set_last_error("%s: null output or bad N (%lld)", what, (long long)N);
    return MI_ERR_INVALID;
  }
  if (epilogue == kEpiResidual && res == nullptr) {
    set_last_error("%s: residual epilogue needs res", what);
    return MI_ERR_INVALID;
  }
  if (epilogue == kEpiSwiglu && (st = check_w(w_b, s_b, w_sn_b, N, K, what)) != MI_OK) return st;
  if (epilogue == kEpiSwiglu && K > 4096) {
    set_last_error("%s: the SwiGLU epilogue supports K <= 4096 (K=%lld)", what,
                   (long long)K);
    return MI_ERR_UNSUPPORTED;
  }
  if (epilogue != kEpiStore && epilogue != kEpiResidual && epilogue != kEpiSwiglu) {
    set_last_error("%s: unknown epilogue %d", what, (int)epilogue);
    return MI_ERR_INVALID;
  }
  LayerGemvArgs a{};
  a.x = x; a.norm_w = norm_w; a.eps = eps;
  a.w0 = w_a; a.s0 = s_a; a.w_sn0 = w_sn_a;
  a.w1 = w_b; a.s1 = s_b; a.w_sn1 = w_sn_b;
  a.y = y; a.res = res; a.x_sm = x_sm; a.y_sm = y_sm; a.res_sm = res_sm;
  a.M = (int32_t)M; a.K = (int32_t)K; a.N = (int32_t)N;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  if (dtype == MI_DTYPE_BF16) {
    e = epilogue == kEpiStore ? dispatch_linear<bf16_t, kEpiStore>(a, s)
        : epilogue == kEpiResidual ? dispatch_linear<bf16_t, kEpiResidual>(a, s)
                                   : dispatch_linear<bf16_t, kEpiSwiglu>(a, s);
  } else {
    e = epilogue == kEpiStore ? dispatch_linear<f16_t, kEpiStore>(a, s)
        : epilogue == kEpiResidual ? dispatch_linear<f16_t, kEpiResidual>(a, s)
                                   : dispatch_linear<f16_t, kEpiSwiglu>(a, s);
  }
  if (e != hipSuccess) {
    set_last_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return (int32_t)e;
  }
  return MI_OK;
}

extern "C" int32_t mi_w8a16_qkv_rope_append(
    const void* x, int64_t x_sm, const void* norm_w, float eps, const int8_t* wq,
    const void* sq, int64_t wq_sn, const int8_t* wk, const void* sk, int64_t wk_sn,
    const int8_t* wv, const void* sv, int64_t wv_sn, const void* cos, const void* sin,
    int64_t c_ss, int64_t rope_row0, int64_t rope_rows, const int64_t* pos, void* q_out,
    void* cache_k, void* cache_v,
    int64_t c_sb, int64_t c_sh, int64_t c_st, int64_t capacity, int64_t M, int64_t K,
    int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, int32_t dtype, void* stream) {
  const char* what = "w8a16_qkv_rope_append";
  int32_t st = check_x(x, M, K, x_sm, norm_w, dtype, what);
  if (st != MI_OK) return st;
  if ((st = check_w(wq, sq, wq_sn, n_heads * head_dim, K, what)) != MI_OK) return st;
  if ((st = check_w(wk, sk, wk_sn, n_kv_heads * head_dim, K, what)) != MI_OK) return st;
  if ((st = check_w(wv, sv, wv_sn, n_kv_heads * head_dim, K, what)) != MI_OK) return st;
  if (cos == nullptr || sin == nullptr || pos == nullptr || q_out == nullptr ||
      cache_k == nullptr || cache_v == nullptr || rope_rows < 1 || c_ss < head_dim / 2) {
    set_last_error("%s: null rope table, position, output or cache pointer", what);
    return MI_ERR_INVALID;
  }
  if (head_dim < 16 || head_dim % 16 != 0 || n_heads < 1 || n_kv_heads < 1 ||
      n_heads % n_kv_heads != 0 || capacity < 1 || n_heads * head_dim > INT32_MAX / 2) {
    set_last_error("%s: unsupported heads (%lld/%lld) or head_dim %lld", what,
                   (long long)n_heads, (long long)n_kv_heads, (long long)head_dim);
    return MI_ERR_UNSUPPORTED;
  }
  LayerGemvArgs a{};
  a.x = x; a.norm_w = norm_w; a.eps = eps;
  a.w0 = wq; a.s0 = sq; a.w_sn0 = wq_sn;
  a.w1 = wk; a.s1 = sk; a.w_sn1 = wk_sn;
  a.w2 = wv; a.s2 = sv; a.w_sn2 = wv_sn;
  a.y = q_out; a.x_sm = x_sm;
  a.M = (int32_t)M; a.K = (int32_t)K; a.N = (int32_t)(n_heads * head_dim);
  a.cos = cos; a.sin = sin; a.c_ss = c_ss; a.rope_row0 = rope_row0; a.rope_rows = rope_rows;
  a.pos = pos;
  a.ck = cache_k; a.cv = cache_v; a.c_sb = c_sb; a.c_sh = c_sh; a.c_st = c_st;
  a.capacity = capacity;
  a.Hq = (int32_t)n_heads; a.Hkv = (int32_t)n_kv_heads; a.D = (int32_t)head_dim;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  if (M <= 8) {
    // diagonal-packed kernel: 8-row tiles of 4 rotation pairs
    const int tph = (int)(head_dim / 8);
    a.n_tiles0 = (int32_t)(n_heads * tph);
    a.n_tiles1 = (int32_t)(n_kv_heads * tph);
    const int n_tiles = a.n_tiles0 + 2 * a.n_tiles1, cus = device_cu_count();
    if (n_tiles > cus) {
      // tiles in pairs (see dgemv_kernel): wq's first, and wk's / wv's as well
      // when that alone leaves more blocks than CUs.  One MI355X, M = 8, K =
      // 2048, 16-call graph: Llama-3.2-1B (384 tiles -> 256 blocks) 6.34 ->
      // 5.29 us per call
      const int per0 = (a.n_tiles0 + 1) / 2;
      a.pair_kv = per0 + 2 * a.n_tiles1 > cus ? 1 : 0;
      const int n_blocks = per0 + 2 * (a.pair_kv ? (a.n_tiles1 + 1) / 2 : a.n_tiles1);
      e = dtype == MI_DTYPE_BF16 ? dispatch_dg<bf16_t, kEpiQkvRope, 2>(a, n_blocks, s)
                                 : dispatch_dg<f16_t, kEpiQkvRope, 2>(a, n_blocks, s);
    } else {
      e = dtype == MI_DTYPE_BF16 ? dispatch_dg<bf16_t, kEpiQkvRope, 1>(a, n_tiles, s)
                                 : dispatch_dg<f16_t, kEpiQkvRope, 1>(a, n_tiles, s);
    }
  } else {
    const int tph = (int)(head_dim / 16);   // tiles (8 rotation pairs each) per head
    a.n_tiles0 = (int32_t)(n_heads * tph);
    a.n_tiles1 = (int32_t)(n_kv_heads * tph);
    const int n_blocks = a.n_tiles0 + 2 * a.n_tiles1;
    e = dtype == MI_DTYPE_BF16 ? dispatch_norm<bf16_t, kEpiQkvRope, 16>(a, n_blocks, s)
                               : dispatch_norm<f16_t, kEpiQkvRope, 16>(a, n_blocks, s);
  }
  if (e != hipSuccess) {
    set_last_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return (int32_t)e;
  }
  return MI_OK;
}
