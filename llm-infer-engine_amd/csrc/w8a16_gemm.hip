// W8A16 GEMM for prefill: y[m, n] = (sum_k x[m, k] * q[n, k]) * s[n], any M.
//
// Math of the reference's GEMM kernel (src/quant_linear.py:123-188): the int8
// weight is converted to the activation dtype (exact, |q| <= 128), products are
// accumulated in fp32, the per-row scale is applied once to the finished sum
// (:180-183) and the result is rounded to x's dtype.  The reference dispatches
// to it when the flattened input has more than 8 rows (:273).
//
// MI355X design.  At prefill sizes (M in the thousands) the product is
// MFMA-bound: a 128 x 256 (m x n) output tile per workgroup of 4 waves, 64-deep
// k stages, v_mfma_f32_32x32x16_{bf16,f16} with fp32 accumulators, two
// workgroups per CU (two waves per SIMD, so one wave's VALU and LDS work issues
// under the other's MFMAs).
//  * Each wave owns 64 output columns (n) and all 128 rows (m).  The activation
//    tile is shared by the 4 waves and copied global->LDS by DMA
//    (global_load_lds_dwordx4: no VGPRs, no VALU); the int8 weight fragments
//    are private to a wave and go straight from global memory to registers
//    (a wave's 64 rows x 64 k = 4 KB per stage).  Both are fetched one stage
//    ahead.
//  * The weight is widened to the activation dtype in registers right before
//    the MFMAs; every widened fragment feeds 4 MFMAs: 1.5 VALU ops per element
//    = 3 per 32x32x16 MFMA.
//  * The weight rows are the MFMA A operand and the activation rows the B
//    operand, so each lane's accumulators hold 4 consecutive output columns
//    of one row (8-byte stores).
//  * The k order inside a 64-deep stage is permuted identically for both
//    operands: the lane of half h feeds k = 32h + 8j .. 32h + 8j + 7 to MFMA
//    step j, so it reads 32 contiguous k of a row (two 16-byte loads of the
//    weight row, four 16-byte LDS reads of the activation row).  The sum is
//    over the same k.
//  * Activation rows are XOR-swizzled by 16-byte chunk in LDS so those reads
//    are free of bank conflicts; the DMA realises the swizzle by choosing which
//    chunk each lane fetches (a DMA wave instruction writes 1 KB contiguously).
//  * The 256 column scales are staged in LDS at the start, so the epilogue has
//    no dependent global loads.
//  * Tiles are ordered so that concurrently resident workgroups of one XCD
//    (blocks are dealt to the 8 XCDs round-robin) cover a patch of 8 m-tiles
//    and share their operand rows in that XCD's L2.
#include "common.hpp"

namespace mi {

struct GemmArgs {
  const unsigned char* x;  // [M, K] activations (unit k stride), rows x_sm elements apart
  const unsigned char* w;  // [N, K] int8, rows w_sn bytes apart
  const void* scales;      // [N] (element stride s_sn)
  void* y;                 // [M, N] (unit n stride), rows y_sm elements apart
  int64_t x_sm, w_sn, s_sn, y_sm;
  int32_t M, N, K;
  int32_t tiles_m, tiles_n;
  int32_t y_vec;           // rows of y allow 8-byte stores of 4 columns
  // split-K: workgroup (tile, split) sums stages [split * split_stages, +split_stages)
  // into part[split][m][n] (fp32, rows of N); one split = the whole K
  float* part;
  int32_t split_stages;
  int32_t part_vec;        // part rows allow 16-byte stores of 4 columns
  int32_t y_line;          // y and its rows are 16-byte aligned (whole-line epilogue)
  // SwiGLU form: y = silu(x w^T * s) * (x w3^T * s3), each product rounded to
  // the activation dtype first (w3 / scales3 / strides as w / scales)
  const unsigned char* w3;
  const void* scales3;
  int64_t w3_sn, s3_sn;
  // residual form (res != nullptr): y = round(res + round(x w^T * s)), res [M, N]
  // in the activation dtype with unit column stride, rows res_sm elements apart
  const void* res;
  int64_t res_sm;
  int32_t res_line;        // res and its rows are 16-byte aligned
};

// 8 activation-dtype values a and b (16 bytes each): round(a + b) per element
template <typename T>
__device__ inline u32x4 add8(const u32x4& a, const u32x4& b) {
  float fa[8], fb[8];
  Chunk<T>::unpack(a, fa);
  Chunk<T>::unpack(b, fb);
  typedef T t8 __attribute__((ext_vector_type(8)));
  t8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = Elem<T>::from_f32(fa[e] + fb[e]);
  return __builtin_bit_cast(u32x4, o);
}

constexpr int kGmBM = 128;                      // output rows (m) per workgroup
constexpr int kGmBN = 256;                      // output columns (n) per workgroup
constexpr int kGmBK = 64;                       // k per stage
constexpr int kGmXBytes = kGmBM * kGmBK * 2;    // activation tile per stage, 16 KB
constexpr int kGmXDma = kGmXBytes / 1024 / 4;   // 1 KB DMA instructions per wave and stage
constexpr int kGmGroupM = 8;                    // m-tiles per tile group
// LDS: two activation stages, then the workgroup's column scales (fp32)
constexpr size_t kGmLdsBytes = 2 * kGmXBytes + kGmBN * sizeof(float);

// silu(x) = x / (1 + e^-x) with the hardware exp2 and reciprocal (a few ulp
// of fp32; the SwiGLU epilogue rounds it to the activation dtype right after)
__device__ inline float silu_fast(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * 1.44269504f));
}

// chunk swizzle of activation row r (8 chunks of 16 bytes per row)
__device__ inline int gm_xswz(int r) { return ((r >> 1) ^ (r << 2)) & 7; }

template <typename T> struct GemmOps;
template <> struct GemmOps<bf16_t> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  __device__ static inline f32x16 mma(const v8& a, const v8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  // upper halves of two fp32 values whose low 16 bits are zero
  __device__ static inline uint32_t hi2(float lo, float hi) {
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
  }
  // 8 int8 (two words) -> 8 bf16, exact: each byte is sign-extended and
  // converted to fp32 (one SDWA op); integers of magnitude <= 128 have 8
  // significant bits, so the fp32 upper halves are the bf16 values.
  __device__ static inline v8 widen(uint32_t lo, uint32_t hi) {
    u32x4 r;
    r.x = hi2((float)(int8_t)lo, (float)(int8_t)(lo >> 8));
    r.y = hi2((float)(int8_t)(lo >> 16), (float)(int8_t)(lo >> 24));
    r.z = hi2((float)(int8_t)hi, (float)(int8_t)(hi >> 8));
    r.w = hi2((float)(int8_t)(hi >> 16), (float)(int8_t)(hi >> 24));
    return __builtin_bit_cast(v8, r);
  }
};
template <> struct GemmOps<f16_t> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  __device__ static inline f32x16 mma(const v8& a, const v8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  // two bytes of u (= q ^ 0x80 = q + 128) -> fp16 pair 1024 + u (bit pattern
  // 0x6400 | u), minus 1152 -> q exactly (fp16 spacing is 1 in [1024, 2048)).
  __device__ static inline uint32_t pair(uint32_t u, uint32_t sel) {
    const h2 v = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, u, sel));
    return __builtin_bit_cast(uint32_t, v - h2{(_Float16)1152.f, (_Float16)1152.f});
  }
  __device__ static inline v8 widen(uint32_t lo, uint32_t hi) {
    lo ^= 0x80808080u;
    hi ^= 0x80808080u;
    u32x4 r;
    r.x = pair(lo, 0x04010400u);
    r.y = pair(lo, 0x04030402u);
    r.z = pair(hi, 0x04010400u);
    r.w = pair(hi, 0x04030402u);
    return __builtin_bit_cast(v8, r);
  }
};

// Tile of a linear workgroup id: ids dealt round-robin to the 8 XCDs are first
// regrouped so that each XCD's ids are consecutive, then consecutive ids walk
// groups of kGmGroupM m-tiles, m fastest.
__device__ inline void gm_tile(int tiles_m, int tiles_n, int b, int& tm, int& tn) {
  const int G = tiles_m * tiles_n;
  if ((G & 7) == 0) b = (b & 7) * (G >> 3) + (b >> 3);
  const int group = kGmGroupM * tiles_n;
  const int g = b / group, first = g * kGmGroupM;
  const int gm = min(tiles_m - first, kGmGroupM);
  const int in = b - g * group;
  tm = first + in % gm;
  tn = in / gm;
}

// One workgroup's 128 x 256 output tile (tm, tn) of the GEMM described by a
// (split-K: the k stages of `split`).  SWIGLU: the tile is 128 columns of the
// gated product, its 256 weight rows the 128 matching rows of w and of w3
// (each wave: 32 rows of each), combined in the epilogue.
template <typename T, typename ST, bool PARTIAL, bool SWIGLU = false>
__device__ __forceinline__ void gemm_tile_body(const GemmArgs& a, int tm, int tn, int split) {
  static_assert(!(PARTIAL && SWIGLU), "the SwiGLU epilogue needs the whole K");
  using OP = GemmOps<T>;
  typedef typename OP::v8 v8;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // the wave's 64 columns
  const int r = lane & 31, h = lane >> 5;
  const int m0 = tm * kGmBM, n0 = tn * (SWIGLU ? kGmBN / 2 : kGmBN);

  // the workgroup's 256 column scales as fp32, staged in LDS after the first
  // stage's copies are issued (read by the epilogue; published by the main
  // loop's first barrier)
  ST sc_raw;
  if constexpr (SWIGLU) {   // [0, 128): w's scales, [128, 256): w3's
    const bool hi = threadIdx.x >= kGmBN / 2;
    const int c = min(n0 + (int)(threadIdx.x & (kGmBN / 2 - 1)), a.N - 1);
    sc_raw = hi ? reinterpret_cast<const ST*>(a.scales3)[(int64_t)c * a.s3_sn]
                : reinterpret_cast<const ST*>(a.scales)[(int64_t)c * a.s_sn];
  } else {
    sc_raw = reinterpret_cast<const ST*>(a.scales)[(int64_t)min(n0 + (int)threadIdx.x, a.N - 1) * a.s_sn];
  }
  float* const sc_lds = reinterpret_cast<float*>(smem_raw + 2 * kGmXBytes);

  // ---- activation DMA: instruction i of wave wv copies tile rows
  // 8 (4 wv + i) .. + 8; lane t fetches logical chunk (t % 8) ^ swz(row) of
  // row t / 8 (byte offsets relative to the stage's first column).
  uint32_t x_off[kGmXDma];
#pragma unroll
  for (int i = 0; i < kGmXDma; ++i) {
    const int row = 8 * (kGmXDma * wv + i) + (lane >> 3);
    const int c = (lane & 7) ^ gm_xswz(row);
    const int gm = min(m0 + row, a.M - 1);                 // rows past M: clamped, never stored
    x_off[i] = (uint32_t)((int64_t)(gm - m0) * a.x_sm * 2 + c * 16);
  }
  const unsigned char* x_base = a.x + (int64_t)m0 * a.x_sm * 2;
  const uint32_t lds0 = lds_addr(smem_raw);
  const int s_begin = PARTIAL ? split * a.split_stages : 0;
  const int nk = PARTIAL ? min(s_begin + a.split_stages, a.K / kGmBK) : a.K / kGmBK;
  auto issue_x = [&](int s) {
    const uint32_t xl = lds0 + (s & 1) * kGmXBytes;
    const unsigned char* xb = x_base + (int64_t)s * kGmBK * 2;
#pragma unroll
    for (int i = 0; i < kGmXDma; ++i) lds_dma16(xb, x_off[i], xl + (kGmXDma * wv + i) * 1024);
  };

  // ---- weight fragments: lane (r, h) of fragment nf loads the 32 k
  // 32h .. 32h + 31 of the stage from weight row n0 + 64 wv + 32 nf + r (rows
  // past N clamped, never stored).
  const unsigned char* w_row[2];
#pragma unroll
  for (int nf = 0; nf < 2; ++nf) {
    if constexpr (SWIGLU)   // fragment 0 from w, 1 from w3: the same 32 output columns
      w_row[nf] = (nf ? a.w3 : a.w) + (int64_t)min(n0 + 32 * wv + r, a.N - 1) * (nf ? a.w3_sn : a.w_sn) + 32 * h;
    else
      w_row[nf] = a.w + (int64_t)min(n0 + 64 * wv + 32 * nf + r, a.N - 1) * a.w_sn + 32 * h;
  }
  auto load_w = [&](int s, u32x4 (&q)[2][2]) {
#pragma unroll
    for (int nf = 0; nf < 2; ++nf)
#pragma unroll
      for (int e = 0; e < 2; ++e) q[nf][e] = load16(w_row[nf] + (int64_t)s * kGmBK + 16 * e);
  };

  // ---- activation fragment mf: LDS row 32 mf + r, chunks 4h + j (j = MFMA k step)
  int x_rd[4][4];
#pragma unroll
  for (int mf = 0; mf < 4; ++mf) {
    const int row = 32 * mf + r;
#pragma unroll
    for (int j = 0; j < 4; ++j) x_rd[mf][j] = row * 128 + 16 * ((4 * h + j) ^ gm_xswz(row));
  }

  f32x16 acc[4][2];
#pragma unroll
  for (int mf = 0; mf < 4; ++mf)
#pragma unroll
    for (int nf = 0; nf < 2; ++nf)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[mf][nf][i] = 0.f;

  // One stage: stage s's activation tile is in LDS slot s % 2 and its weight
  // fragments in wc; the copies of stage s + 1 (activation DMA, weight loads
  // into wn) are issued before its MFMAs so that they land under them.
  auto step = [&](int s, u32x4 (&wc)[2][2], u32x4 (&wn)[2][2]) {
    dma_wait_all();                          // this wave's copies of stage s landed
    // wc is read here, after the wait, so the compiler's own wait for the
    // weight loads also falls here and not after the next stage's copies
    __asm__ volatile("" ::"v"(wc[0][0]), "v"(wc[0][1]), "v"(wc[1][0]), "v"(wc[1][1]));
    // every wave's part of stage s is in LDS, and every wave is done reading
    // the slot that the next copy overwrites (stage s - 1's)
    block_sync_lds();
    if (s + 1 < nk) {
      issue_x(s + 1);
      load_w(s + 1, wn);
    }
    // keep the next stage's loads ahead of this stage's MFMAs
    __builtin_amdgcn_sched_barrier(0);
    const unsigned char* st = smem_raw + (s & 1) * kGmXBytes;
    v8 xa[4][4];
#pragma unroll
    for (int mf = 0; mf < 4; ++mf)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        xa[mf][j] = __builtin_bit_cast(v8, *reinterpret_cast<const u32x4*>(st + x_rd[mf][j]));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int nf = 0; nf < 2; ++nf) {
        const u32x4& q = wc[nf][j >> 1];
        const v8 wb = (j & 1) ? OP::widen(q.z, q.w) : OP::widen(q.x, q.y);
#pragma unroll
        for (int mf = 0; mf < 4; ++mf) acc[mf][nf] = OP::mma(wb, xa[mf][j], acc[mf][nf]);
      }
    }
  };

  // two register sets for the weight fragments, alternating by stage
  u32x4 wa[2][2], wb[2][2];
  issue_x(s_begin);
  load_w(s_begin, wa);
  sc_lds[threadIdx.x] = Elem<ST>::to_f32(sc_raw);
  int s = s_begin;
  for (; s + 1 < nk; s += 2) {
    step(s, wa, wb);
    step(s + 1, wb, wa);
  }
  if (s < nk) step(s, wa, wb);

  // ---- epilogue: acc[mf][nf][4 g + i] = C[n][m] with
  // n = n0 + 64 wv + 32 nf + 8 g + 4 h + i, m = m0 + 32 mf + r
  if constexpr (PARTIAL) {
    // unscaled fp32 sums of this split's k range
    float* pp = a.part + (int64_t)split * a.M * a.N;
#pragma unroll
    for (int nf = 0; nf < 2; ++nf)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int nb = n0 + 64 * wv + 32 * nf + 8 * g + 4 * h;
#pragma unroll
        for (int mf = 0; mf < 4; ++mf) {
          const int m = m0 + 32 * mf + r;
          if (m >= a.M) continue;
          float* q = pp + (int64_t)m * a.N + nb;
          if (a.part_vec && nb + 3 < a.N) {
            *reinterpret_cast<f32x4*>(q) = f32x4{acc[mf][nf][4 * g], acc[mf][nf][4 * g + 1],
                                                 acc[mf][nf][4 * g + 2], acc[mf][nf][4 * g + 3]};
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (nb + i < a.N) q[i] = acc[mf][nf][4 * g + i];
          }
        }
      }
    return;
  }
  T* y = reinterpret_cast<T*>(a.y);
  if constexpr (SWIGLU) {
    // acc[mf][0] / acc[mf][1]: w / w3 products of the same 4 columns per g,
    // rounded where the unfused chain rounds: y1, y3, silu(y1), the product
    // (silu with the hardware exp2 and reciprocal: within an ulp of the
    // chain's bits)
    auto rnd = [](float v) { return Elem<T>::to_f32(Elem<T>::from_f32(v)); };
    typedef T t4 __attribute__((ext_vector_type(4)));
    auto gate4 = [&](int mf, int g, const f32x4& s1, const f32x4& s3) {
      t4 v;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float y1 = rnd(acc[mf][0][4 * g + i] * s1[i]);
        const float y3 = rnd(acc[mf][1][4 * g + i] * s3[i]);
        v[i] = Elem<T>::from_f32(rnd(silu_fast(y1)) * y3);
      }
      return v;
    };
    if (a.y_line && n0 + kGmBN / 2 <= a.N) {
      // whole-line stores as below: each wave stages its 32 columns of 32
      // rows at a time and writes a row's 64 bytes with 4 lanes x 16 bytes
      constexpr int RS = 80;                 // staged row stride (bytes, padded)
      block_sync_lds();
      unsigned char* const stg = smem_raw + wv * 32 * RS;
      f32x4 s1[4], s3[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        s1[g] = *reinterpret_cast<const f32x4*>(sc_lds + 32 * wv + 8 * g + 4 * h);
        s3[g] = *reinterpret_cast<const f32x4*>(sc_lds + kGmBN / 2 + 32 * wv + 8 * g + 4 * h);
      }
#pragma unroll
      for (int mf = 0; mf < 4; ++mf) {
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<t4*>(stg + r * RS + (8 * g + 4 * h) * 2) = gate4(mf, g, s1[g], s3[g]);
        __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the wave's own rows are staged
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int rr = 16 * i + (lane >> 2), cc = lane & 3;
          const u32x4 v = *reinterpret_cast<const u32x4*>(stg + rr * RS + cc * 16);
          const int m = m0 + 32 * mf + rr;
          if (m < a.M)
            *reinterpret_cast<u32x4*>(y + (int64_t)m * a.y_sm + n0 + 32 * wv + 8 * cc) = v;
        }
      }
      return;
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int nl = 32 * wv + 8 * g + 4 * h, nb = n0 + nl;
      const f32x4 s1 = *reinterpret_cast<const f32x4*>(sc_lds + nl);
      const f32x4 s3 = *reinterpret_cast<const f32x4*>(sc_lds + kGmBN / 2 + nl);
#pragma unroll
      for (int mf = 0; mf < 4; ++mf) {
        const int m = m0 + 32 * mf + r;
        if (m >= a.M) continue;
        const t4 v = gate4(mf, g, s1, s3);
        T* yp = y + (int64_t)m * a.y_sm + nb;
        if (a.y_vec && nb + 3 < a.N) {
          *reinterpret_cast<t4*>(yp) = v;
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (nb + i < a.N) yp[i] = v[i];
        }
      }
    }
    return;
  }
  if (a.y_line && (a.res == nullptr || a.res_line) && n0 + kGmBN <= a.N) {
    // Whole-line stores: each wave stages its 64 columns of 32 rows at a time
    // in LDS (the activation stages, free once every wave has read the last
    // one) and writes each row's 128 bytes with 8 lanes x 16 bytes of one
    // instruction, instead of 16-byte pieces of 32 rows from 8 instructions.
    constexpr int RS = 136;                  // staged row stride (bytes, padded)
    block_sync_lds();
    unsigned char* const stg = smem_raw + wv * 32 * RS;
    typedef T t4 __attribute__((ext_vector_type(4)));
    f32x4 s4[2][4];
#pragma unroll
    for (int nf = 0; nf < 2; ++nf)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        s4[nf][g] = *reinterpret_cast<const f32x4*>(sc_lds + 64 * wv + 32 * nf + 8 * g + 4 * h);
#pragma unroll
    for (int mf = 0; mf < 4; ++mf) {
#pragma unroll
      for (int nf = 0; nf < 2; ++nf)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          t4 v;
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = Elem<T>::from_f32(acc[mf][nf][4 * g + i] * s4[nf][g][i]);
          *reinterpret_cast<t4*>(stg + r * RS + (32 * nf + 8 * g + 4 * h) * 2) = v;
        }
      __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the wave's own rows are staged
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rr = 8 * i + (lane >> 3), cc = lane & 7;
        u32x4 v = *reinterpret_cast<const u32x4*>(stg + rr * RS + cc * 16);
        const int m = m0 + 32 * mf + rr;
        if (m < a.M) {
          const int64_t col = n0 + 64 * wv + 8 * cc;
          if (a.res != nullptr)
            v = add8<T>(v, load16(reinterpret_cast<const T*>(a.res) + (int64_t)m * a.res_sm + col));
          *reinterpret_cast<u32x4*>(y + (int64_t)m * a.y_sm + col) = v;
        }
      }
    }
    return;
  }
#pragma unroll
  for (int nf = 0; nf < 2; ++nf) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int nl = 64 * wv + 32 * nf + 8 * g + 4 * h, nb = n0 + nl;
      const f32x4 s4 = *reinterpret_cast<const f32x4*>(sc_lds + nl);
#pragma unroll
      for (int mf = 0; mf < 4; ++mf) {
        const int m = m0 + 32 * mf + r;
        if (m >= a.M) continue;
        T* yp = y + (int64_t)m * a.y_sm + nb;
        const T* rp = a.res != nullptr
                          ? reinterpret_cast<const T*>(a.res) + (int64_t)m * a.res_sm + nb
                          : nullptr;
        auto outv = [&](int i) {
          const T v = Elem<T>::from_f32(acc[mf][nf][4 * g + i] * s4[i]);
          return a.res != nullptr ? Elem<T>::from_f32(Elem<T>::to_f32(rp[i]) + Elem<T>::to_f32(v)) : v;
        };
        if (a.y_vec && nb + 3 < a.N) {
          typedef T t4 __attribute__((ext_vector_type(4)));
          t4 v;
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = outv(i);
          *reinterpret_cast<t4*>(yp) = v;
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (nb + i < a.N) yp[i] = outv(i);
        }
      }
    }
  }
}

template <typename T, typename ST, bool PARTIAL>
__global__ __launch_bounds__(256, 2) void w8a16_gemm_kernel(GemmArgs a) {
  // split-K: workgroup ids run over all tiles of split 0, then of split 1, ...
  const int n_tiles = a.tiles_m * a.tiles_n;
  const int split = PARTIAL ? (int)blockIdx.x / n_tiles : 0;
  int tm, tn;
  gm_tile(a.tiles_m, a.tiles_n, (int)blockIdx.x - split * n_tiles, tm, tn);
  gemm_tile_body<T, ST, PARTIAL>(a, tm, tn, split);
}

// The gated feed-forward input projection silu(x w1^T) * (x w3^T) in one
// GEMM: 128-column tiles of the product, each reading the matching rows of w1
// and w3, so neither projection is written out.
template <typename T, typename ST>
__global__ __launch_bounds__(256, 2) void w8a16_gemm_swiglu_kernel(GemmArgs a) {
  int tm, tn;
  gm_tile(a.tiles_m, a.tiles_n, (int)blockIdx.x, tm, tn);
  gemm_tile_body<T, ST, false, true>(a, tm, tn, 0);
}

// Several GEMMs of one activation x (e.g. the q, k and v projections) in one
// launch: the 128 x 256 tiles of all matrices form one grid, matrix i owning
// tile columns [col0[i], col0[i + 1]); the grid is walked in the single-GEMM
// order (XCD regrouping, groups of m-tiles), so each XCD's resident tiles
// share activation rows across the matrices.  Each tile is computed exactly
// as by w8a16_gemm_kernel on its own matrix.
constexpr int kGmMaxMats = 4;
struct GemmMultiArgs {
  GemmArgs mat[kGmMaxMats];
  int32_t col0[kGmMaxMats + 1];
  int32_t n_mats, tiles_m;
};

template <typename T, typename ST>
__global__ __launch_bounds__(256, 2) void w8a16_gemm_multi_kernel(GemmMultiArgs ma) {
  int tm, tn;
  gm_tile(ma.tiles_m, ma.col0[ma.n_mats], (int)blockIdx.x, tm, tn);
  int i = 0;
#pragma unroll
  for (int j = 1; j < kGmMaxMats; ++j)
    if (j < ma.n_mats && tn >= ma.col0[j]) i = j;
  gemm_tile_body<T, ST, false>(ma.mat[i], tm, tn - ma.col0[i], 0);
}

// Split-K finish: y[m, n] = round((sum over splits, in split order, of
// part[s][m][n]) * scale[n]); one thread per 4 consecutive columns of a row.
template <typename T, typename ST>
__global__ __launch_bounds__(256) void w8a16_splitk_reduce_kernel(GemmArgs a, int32_t splits) {
  const int64_t q4 = (a.N + 3) / 4;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)a.M * q4) return;
  const int m = (int)(idx / q4), nb = (int)(idx - (int64_t)m * q4) * 4;
  const ST* sc = reinterpret_cast<const ST*>(a.scales);
  const int64_t plane = (int64_t)a.M * a.N;
  const float* pp = a.part + (int64_t)m * a.N + nb;
  T* yp = reinterpret_cast<T*>(a.y) + (int64_t)m * a.y_sm + nb;
  if (a.part_vec && nb + 3 < a.N) {
    f32x4 t = *reinterpret_cast<const f32x4*>(pp);
    for (int sp = 1; sp < splits; ++sp) t += *reinterpret_cast<const f32x4*>(pp + sp * plane);
    typedef T t4 __attribute__((ext_vector_type(4)));
    t4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = Elem<T>::from_f32(t[i] * Elem<ST>::to_f32(sc[(int64_t)(nb + i) * a.s_sn]));
      if (a.res != nullptr)
        v[i] = Elem<T>::from_f32(
            Elem<T>::to_f32(reinterpret_cast<const T*>(a.res)[(int64_t)m * a.res_sm + nb + i]) +
            Elem<T>::to_f32(v[i]));
    }
    if (a.y_vec) {
      *reinterpret_cast<t4*>(yp) = v;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) yp[i] = v[i];
    }
  } else {
    for (int i = 0; i < 4 && nb + i < a.N; ++i) {
      float t = pp[i];
      for (int sp = 1; sp < splits; ++sp) t += pp[i + sp * plane];
      T v = Elem<T>::from_f32(t * Elem<ST>::to_f32(sc[(int64_t)(nb + i) * a.s_sn]));
      if (a.res != nullptr)
        v = Elem<T>::from_f32(
            Elem<T>::to_f32(reinterpret_cast<const T*>(a.res)[(int64_t)m * a.res_sm + nb + i]) +
            Elem<T>::to_f32(v));
      yp[i] = v;
    }
  }
}

}  // namespace mi

using namespace mi;

namespace {

// Argument checks shared by both entry points; fills `a` (no split).
int32_t gemm_setup(const char* what, const void* x, const int8_t* w, const void* scales,
                   void* y, int64_t m, int64_t n, int64_t k, int64_t x_sm, int64_t w_sn,
                   int64_t s_sn, int64_t y_sm, GemmArgs& a) {
  if (x == nullptr || w == nullptr || scales == nullptr || y == nullptr) {
    set_last_error("%s: null pointer", what);
    return MI_ERR_INVALID;
  }
  if (m <= 0 || n <= 0 || k <= 0 || m > INT32_MAX || n > INT32_MAX || k > INT32_MAX) {
    set_last_error("%s: need positive M, N, K below 2^31 (M=%lld N=%lld K=%lld)", what,
                   (long long)m, (long long)n, (long long)k);
    return MI_ERR_INVALID;
  }
  if (k % kGmBK != 0) {
    set_last_error("%s: K must be a multiple of %d (K=%lld)", what, kGmBK, (long long)k);
    return MI_ERR_UNSUPPORTED;
  }
  // tile-relative DMA offsets are 32-bit: 128 activation rows of x_sm elements
  if (x_sm < k || w_sn < k || y_sm < n || x_sm > (1LL << 23) || w_sn > (1LL << 23)) {
    set_last_error("%s: row strides must cover a row and be below 2^23 elements", what);
    return MI_ERR_INVALID;
  }
  if ((uintptr_t)x % 16 != 0 || (x_sm * 2) % 16 != 0 || (uintptr_t)w % 16 != 0 || w_sn % 16 != 0) {
    set_last_error("%s: x and weight rows must be 16-byte aligned", what);
    return MI_ERR_INVALID;
  }
  const int64_t tiles_m = (m + kGmBM - 1) / kGmBM, tiles_n = (n + kGmBN - 1) / kGmBN;
  if (tiles_m * tiles_n > INT32_MAX / 64) {
    set_last_error("%s: too many tiles", what);
    return MI_ERR_INVALID;
  }
  a = GemmArgs{static_cast<const unsigned char*>(x), reinterpret_cast<const unsigned char*>(w),
               scales, y, x_sm, w_sn, s_sn, y_sm, (int32_t)m, (int32_t)n, (int32_t)k,
               (int32_t)tiles_m, (int32_t)tiles_n,
               ((uintptr_t)y % 8 == 0 && y_sm % 4 == 0) ? 1 : 0,
               nullptr, (int32_t)(k / kGmBK), 0,
               ((uintptr_t)y % 16 == 0 && y_sm % 8 == 0) ? 1 : 0};
  return MI_OK;
}

bool dtypes_ok(int32_t dtype, int32_t sdtype) {
  return (dtype == MI_DTYPE_BF16 || dtype == MI_DTYPE_F16) &&
         (sdtype == MI_DTYPE_BF16 || sdtype == MI_DTYPE_F16 || sdtype == MI_DTYPE_F32);
}

template <bool PARTIAL>
void launch_gemm(const GemmArgs& a, int32_t splits, int32_t dtype, int32_t sdtype, hipStream_t st) {
  dim3 grid((unsigned)((int64_t)a.tiles_m * a.tiles_n * splits)), block(256);
#define MI_GEMM(T, ST) \
  hipLaunchKernelGGL((w8a16_gemm_kernel<T, ST, PARTIAL>), grid, block, kGmLdsBytes, st, a)
  if (dtype == MI_DTYPE_BF16 && sdtype == MI_DTYPE_BF16) MI_GEMM(bf16_t, bf16_t);
  else if (dtype == MI_DTYPE_BF16 && sdtype == MI_DTYPE_F32) MI_GEMM(bf16_t, float);
  else if (dtype == MI_DTYPE_BF16 && sdtype == MI_DTYPE_F16) MI_GEMM(bf16_t, f16_t);
  else if (dtype == MI_DTYPE_F16 && sdtype == MI_DTYPE_F16) MI_GEMM(f16_t, f16_t);
  else if (dtype == MI_DTYPE_F16 && sdtype == MI_DTYPE_F32) MI_GEMM(f16_t, float);
  else MI_GEMM(f16_t, bf16_t);
#undef MI_GEMM
}

void launch_multi(const GemmMultiArgs& ma, int32_t dtype, int32_t sdtype, hipStream_t st) {
  dim3 grid((unsigned)((int64_t)ma.tiles_m * ma.col0[ma.n_mats])), block(256);
#define MI_GEMM(T, ST) \
  hipLaunchKernelGGL((w8a16_gemm_multi_kernel<T, ST>), grid, block, kGmLdsBytes, st, ma)
  if (dtype == MI_DTYPE_BF16 && sdtype == MI_DTYPE_BF16) MI_GEMM(bf16_t, bf16_t);
  else if (dtype == MI_DTYPE_BF16 && sdtype == MI_DTYPE_F32) MI_GEMM(bf16_t, float);
  else if (dtype == MI_DTYPE_BF16 && sdtype == MI_DTYPE_F16) MI_GEMM(bf16_t, f16_t);
  else if (dtype == MI_DTYPE_F16 && sdtype == MI_DTYPE_F16) MI_GEMM(f16_t, f16_t);
  else if (dtype == MI_DTYPE_F16 && sdtype == MI_DTYPE_F32) MI_GEMM(f16_t, float);
  else MI_GEMM(f16_t, bf16_t);
#undef MI_GEMM
}

void launch_swiglu(const GemmArgs& a, int32_t dtype, int32_t sdtype, hipStream_t st) {
  dim3 grid((unsigned)((int64_t)a.tiles_m * a.tiles_n)), block(256);
#define MI_GEMM(T, ST) \
  hipLaunchKernelGGL((w8a16_gemm_swiglu_kernel<T, ST>), grid, block, kGmLdsBytes, st, a)
  if (dtype == MI_DTYPE_BF16 && sdtype == MI_DTYPE_BF16) MI_GEMM(bf16_t, bf16_t);
  else if (dtype == MI_DTYPE_BF16 && sdtype == MI_DTYPE_F32) MI_GEMM(bf16_t, float);
  else if (dtype == MI_DTYPE_BF16 && sdtype == MI_DTYPE_F16) MI_GEMM(bf16_t, f16_t);
  else if (dtype == MI_DTYPE_F16 && sdtype == MI_DTYPE_F16) MI_GEMM(f16_t, f16_t);
  else if (dtype == MI_DTYPE_F16 && sdtype == MI_DTYPE_F32) MI_GEMM(f16_t, float);
  else MI_GEMM(f16_t, bf16_t);
#undef MI_GEMM
}

void launch_reduce(const GemmArgs& a, int32_t splits, int32_t dtype, int32_t sdtype,
                   hipStream_t st) {
  const int64_t threads = (int64_t)a.M * ((a.N + 3) / 4);
  dim3 grid((unsigned)((threads + 255) / 256)), block(256);
#define MI_RED(T, ST) \
  hipLaunchKernelGGL((w8a16_splitk_reduce_kernel<T, ST>), grid, block, 0, st, a, splits)
  if (dtype == MI_DTYPE_BF16 && sdtype == MI_DTYPE_BF16) MI_RED(bf16_t, bf16_t);
  else if (dtype == MI_DTYPE_BF16 && sdtype == MI_DTYPE_F32) MI_RED(bf16_t, float);
  else if (dtype == MI_DTYPE_BF16 && sdtype == MI_DTYPE_F16) MI_RED(bf16_t, f16_t);
  else if (dtype == MI_DTYPE_F16 && sdtype == MI_DTYPE_F16) MI_RED(f16_t, f16_t);
  else if (dtype == MI_DTYPE_F16 && sdtype == MI_DTYPE_F32) MI_RED(f16_t, float);
  else MI_RED(f16_t, bf16_t);
#undef MI_RED
}

int32_t launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_last_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return (int32_t)e;
  }
  return MI_OK;
}

}  // namespace

extern "C" int32_t mi_w8a16_gemm(const void* x, const int8_t* w, const void* scales, void* y,
                                 int64_t m, int64_t n, int64_t k, int64_t x_sm, int64_t w_sn,
                                 int64_t s_sn, int64_t y_sm, int32_t dtype, int32_t sdtype,
                                 void* stream) {
  GemmArgs a;
  int32_t rc = gemm_setup("w8a16_gemm", x, w, scales, y, m, n, k, x_sm, w_sn, s_sn, y_sm, a);
  if (rc != MI_OK) return rc;
  if (!dtypes_ok(dtype, sdtype)) {
    set_last_error("w8a16_gemm: activations must be bf16 or fp16 (dtype %d, scales %d)",
                   (int)dtype, (int)sdtype);
    return MI_ERR_UNSUPPORTED;
  }
  launch_gemm<false>(a, 1, dtype, sdtype, (hipStream_t)stream);
  return launch_status("w8a16_gemm");
}

// Split count for mi_w8a16_gemm_splitk (measured on MI355X): 1 (no split) once
// the 128 x 256 tiles give every CU a workgroup; otherwise about one workgroup
// per CU (at one tile per two CUs the split still gains a little: wk / wv at
// M = 8192, 37.0 -> 36.1 us), each split at least 8 stages (512 k)
// deep, at most 8 splits, and the fp32 partials (written and read once) at
// most 64 MiB.
extern "C" int64_t mi_w8a16_gemm_splits(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0 || k % kGmBK != 0) return 1;
  const int64_t tiles = ((m + kGmBM - 1) / kGmBM) * ((n + kGmBN - 1) / kGmBN);
  const int64_t cus = device_cu_count();
  if (tiles >= cus) return 1;
  int64_t s = cus / tiles;
  const int64_t nk = k / kGmBK;
  if (s > nk / 8) s = nk / 8;
  if (s > 8) s = 8;
  while (s > 1 && s * m * n * 4 > (64LL << 20)) --s;
  // splits actually used: every split gets ceil(nk / s) stages
  if (s > 1) {
    const int64_t per = (nk + s - 1) / s;
    s = (nk + per - 1) / per;
  }
  return s < 1 ? 1 : s;
}

extern "C" int32_t mi_w8a16_gemm_splitk(const void* x, const int8_t* w, const void* scales,
                                        void* y, int64_t m, int64_t n, int64_t k,
                                        int64_t x_sm, int64_t w_sn, int64_t s_sn, int64_t y_sm,
                                        float* part, int64_t part_elems, int64_t splits,
                                        int32_t dtype, int32_t sdtype, void* stream) {
  GemmArgs a;
  int32_t rc = gemm_setup("w8a16_gemm_splitk", x, w, scales, y, m, n, k, x_sm, w_sn, s_sn, y_sm, a);
  if (rc != MI_OK) return rc;
  if (!dtypes_ok(dtype, sdtype)) {
    set_last_error("w8a16_gemm_splitk: activations must be bf16 or fp16 (dtype %d, scales %d)",
                   (int)dtype, (int)sdtype);
    return MI_ERR_UNSUPPORTED;
  }
  const int64_t nk = k / kGmBK;
  if (splits < 2 || splits > nk || splits > 64) {
    set_last_error("w8a16_gemm_splitk: need 2 <= splits <= min(K / %d, 64) (splits=%lld)", kGmBK,
                   (long long)splits);
    return MI_ERR_INVALID;
  }
  const int64_t per = (nk + splits - 1) / splits;
  const int64_t used = (nk + per - 1) / per;   // splits that own at least one stage
  if (part == nullptr || part_elems < used * m * n) {
    set_last_error("w8a16_gemm_splitk: workspace needs %lld fp32 elements (given %lld)",
                   (long long)(used * m * n), (long long)part_elems);
    return MI_ERR_INVALID;
  }
  a.part = part;
  a.split_stages = (int32_t)per;
  a.part_vec = ((uintptr_t)part % 16 == 0 && n % 4 == 0) ? 1 : 0;
  hipStream_t st = (hipStream_t)stream;
  launch_gemm<true>(a, (int32_t)used, dtype, sdtype, st);
  rc = launch_status("w8a16_gemm_splitk");
  if (rc != MI_OK) return rc;
  launch_reduce(a, (int32_t)used, dtype, sdtype, st);
  return launch_status("w8a16_gemm_splitk");
}

extern "C" int32_t mi_w8a16_gemm_multi(const void* x, int64_t m, int64_t k, int64_t x_sm,
                                       int32_t n_mats, const int8_t* const* w,
                                       const void* const* scales, void* const* y,
                                       const int64_t* n, const int64_t* w_sn,
                                       const int64_t* s_sn, const int64_t* y_sm,
                                       int32_t dtype, int32_t sdtype, void* stream) {
  const char* what = "w8a16_gemm_multi";
  if (n_mats < 1 || n_mats > kGmMaxMats || w == nullptr || scales == nullptr || y == nullptr ||
      n == nullptr || w_sn == nullptr || s_sn == nullptr || y_sm == nullptr) {
    set_last_error("%s: need 1..%d matrices and non-null argument arrays (n_mats=%d)", what,
                   kGmMaxMats, (int)n_mats);
    return MI_ERR_INVALID;
  }
  if (!dtypes_ok(dtype, sdtype)) {
    set_last_error("%s: activations must be bf16 or fp16 (dtype %d, scales %d)", what,
                   (int)dtype, (int)sdtype);
    return MI_ERR_UNSUPPORTED;
  }
  GemmMultiArgs ma{};
  int64_t cols = 0;
  for (int i = 0; i < n_mats; ++i) {
    int32_t rc = gemm_setup(what, x, w[i], scales[i], y[i], m, n[i], k, x_sm, w_sn[i], s_sn[i],
                            y_sm[i], ma.mat[i]);
    if (rc != MI_OK) return rc;
    ma.col0[i] = (int32_t)cols;
    cols += ma.mat[i].tiles_n;
  }
  ma.tiles_m = ma.mat[0].tiles_m;
  if (ma.tiles_m * cols > INT32_MAX / 64) {
    set_last_error("%s: too many tiles", what);
    return MI_ERR_INVALID;
  }
  ma.col0[n_mats] = (int32_t)cols;
  ma.n_mats = n_mats;
  launch_multi(ma, dtype, sdtype, (hipStream_t)stream);
  return launch_status(what);
}

extern "C" int32_t mi_w8a16_gemm_swiglu(const void* x, const int8_t* w1, const void* scales1,
                                        const int8_t* w3, const void* scales3, void* y,
                                        int64_t m, int64_t n, int64_t k, int64_t x_sm,
                                        int64_t w1_sn, int64_t s1_sn, int64_t w3_sn,
                                        int64_t s3_sn, int64_t y_sm, int32_t dtype,
                                        int32_t sdtype, void* stream) {
  const char* what = "w8a16_gemm_swiglu";
  GemmArgs a;
  int32_t rc = gemm_setup(what, x, w1, scales1, y, m, n, k, x_sm, w1_sn, s1_sn, y_sm, a);
  if (rc != MI_OK) return rc;
  if (w3 == nullptr || scales3 == nullptr) {
    set_last_error("%s: null pointer", what);
    return MI_ERR_INVALID;
  }
  if (w3_sn < k || w3_sn > (1LL << 23) || (uintptr_t)w3 % 16 != 0 || w3_sn % 16 != 0) {
    set_last_error("%s: w3 rows must cover K, be 16-byte aligned and below 2^23 bytes apart",
                   what);
    return MI_ERR_INVALID;
  }
  if (!dtypes_ok(dtype, sdtype)) {
    set_last_error("%s: activations must be bf16 or fp16 (dtype %d, scales %d)", what,
                   (int)dtype, (int)sdtype);
    return MI_ERR_UNSUPPORTED;
  }
  a.tiles_n = (int32_t)((n + kGmBN / 2 - 1) / (kGmBN / 2));
  if ((int64_t)a.tiles_m * a.tiles_n > INT32_MAX / 64) {
    set_last_error("%s: too many tiles", what);
    return MI_ERR_INVALID;
  }
  a.w3 = reinterpret_cast<const unsigned char*>(w3);
  a.scales3 = scales3;
  a.w3_sn = w3_sn;
  a.s3_sn = s3_sn;
  launch_swiglu(a, dtype, sdtype, (hipStream_t)stream);
  return launch_status(what);
}

extern "C" int32_t mi_w8a16_gemm_residual(const void* x, const int8_t* w, const void* scales,
                                          const void* res, void* y, int64_t m, int64_t n,
                                          int64_t k, int64_t x_sm, int64_t w_sn, int64_t s_sn,
                                          int64_t res_sm, int64_t y_sm, float* part,
                                          int64_t part_elems, int64_t splits, int32_t dtype,
                                          int32_t sdtype, void* stream) {
  const char* what = "w8a16_gemm_residual";
  GemmArgs a;
  int32_t rc = gemm_setup(what, x, w, scales, y, m, n, k, x_sm, w_sn, s_sn, y_sm, a);
  if (rc != MI_OK) return rc;
  if (res == nullptr || res_sm < n) {
    set_last_error("%s: null residual or residual rows shorter than N", what);
    return MI_ERR_INVALID;
  }
  if (!dtypes_ok(dtype, sdtype)) {
    set_last_error("%s: activations must be bf16 or fp16 (dtype %d, scales %d)", what,
                   (int)dtype, (int)sdtype);
    return MI_ERR_UNSUPPORTED;
  }
  a.res = res;
  a.res_sm = res_sm;
  a.res_line = ((uintptr_t)res % 16 == 0 && res_sm % 8 == 0) ? 1 : 0;
  hipStream_t st = (hipStream_t)stream;
  if (splits <= 1) {
    launch_gemm<false>(a, 1, dtype, sdtype, st);
    return launch_status(what);
  }
  const int64_t nk = k / kGmBK;
  if (splits > nk || splits > 64) {
    set_last_error("%s: need splits <= min(K / %d, 64) (splits=%lld)", what, kGmBK,
                   (long long)splits);
    return MI_ERR_INVALID;
  }
  const int64_t per = (nk + splits - 1) / splits;
  const int64_t used = (nk + per - 1) / per;
  if (part == nullptr || part_elems < used * m * n) {
    set_last_error("%s: workspace needs %lld fp32 elements (given %lld)", what,
                   (long long)(used * m * n), (long long)part_elems);
    return MI_ERR_INVALID;
  }
  a.part = part;
  a.split_stages = (int32_t)per;
  a.part_vec = ((uintptr_t)part % 16 == 0 && n % 4 == 0) ? 1 : 0;
  launch_gemm<true>(a, (int32_t)used, dtype, sdtype, st);
  rc = launch_status(what);
  if (rc != MI_OK) return rc;
  launch_reduce(a, (int32_t)used, dtype, sdtype, st);
  return launch_status(what);
}
