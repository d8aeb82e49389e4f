// Split-KV single-token decode attention for gfx950 (bandwidth-bound path):
// device code shared by decode.hip (exact head dims) and decode_pad.hip
// (every other head_dim <= 256).
//
// Math follows the reference's split/combine decode
// (src/flash_decode.py:8-137 per-split partials, :140-212 LSE combine), but the
// work decomposition is MI355X-first:
//   * one workgroup per (batch, kv-head, split) computes the partial state of
//     ALL query heads that share the kv-head (GQA), so every K/V byte is read
//     from HBM exactly once (the reference re-reads it once per query head);
//   * each lane owns one 16-byte chunk of a K/V row per load (coalesced
//     128-bit global loads; a row of P elements spans LPR = P*sizeof(T)/16
//     lanes, capped at 16 = one DPP row);
//   * q.k row sums use DPP row reductions (no LDS round trip), the softmax is
//     kept per row group in registers (log2 domain, v_exp_f32); the row
//     groups of a wave merge through DPP / permlane swaps and the waves once
//     through LDS;
//   * P.V on 2-byte K/V folds two rows per instruction: the rows' elements
//     are paired by a byte permute and their p rounded to the storage type
//     (as the prefill feeds P to its MFMAs), one v_dot2 per element and head
//     with fp32 accumulate -- half the VALU multiply-adds of fp32 P and no
//     unpacking of V (the row sum l keeps the unrounded p);
//   * no MFMA: at one query token per head there is nothing to amortise a
//     matrix tile over, and the loop is HBM-bound;
//   * grids of at most one block per CU (2-byte K/V, whole-chunk rows) run a
//     software pipeline over two register sets: the next pass's K/V loads are
//     in flight while the current pass is folded in (PIPE: 8 waves up to
//     head_dim 64, 4 above, 512-thread register budget; a last pass whose rows
//     fit in its first one or two row slots folds only those); larger grids
//     overlap their blocks instead;
//   * all splits of one (batch, kv-head) group run on one XCD (the hardware
//     deals workgroup i to XCD i mod n_xcc), so with an arrival counter the
//     last split of a group can combine the group's partials from that XCD's
//     L2 inside the same launch (no combine kernel, no kernel boundary).
// Head dims: P (a power of two, 8..256) fixes the register layout; MODE 0 runs
// head_dim == P, MODE 1 any head_dim that fills whole 16-byte chunks (the
// lanes past it load nothing), MODE 2 any head_dim with element loads.
// Keys beyond seq_lens[b] are never loaded.  The grid is static (sized for
// the capacity, so the launch is hipGraph-safe) and with seq_lens the splits
// divide each sequence's own length, so a replay at any length keeps every
// split busy.
#pragma once

#include <math.h>

#include <type_traits>

#include "common.hpp"

namespace mi {

struct DecodeArgs {
  const void* q;
  const void* k;
  const void* v;
  const uint8_t* mask;
  int64_t mask_sb, mask_sl;
  const int64_t* seq_lens;
  float* part_m;
  float* part_l;
  float* part_acc;
  void* out;
  float* lse;
  // arrival counters of the in-launch combine, one per group (nullptr: the
  // partials are combined by a separate launch)
  unsigned long long* arrive;
  int64_t q_sb, q_sh, q_sd;
  int64_t k_sb, k_sh, k_sl;
  int64_t v_sb, v_sh, v_sl;
  int64_t o_sb, o_sh, o_sd;
  int32_t batch, n_heads, group, kv_len;
  int32_t head_dim;   // D <= P
  int32_t n_vchunks;  // 16-byte chunks that hold row elements (MODE 1)
  int32_t split_len, num_splits, n_chunks, chunk_heads;
  int32_t n_xcc, n_groups;  // XCDs blocks are dealt over; B * Hkv * n_chunks
  float scale_log2;
  int32_t direct;     // num_splits == 1: normalise and write out/lse here
  int32_t empty_nan;  // empty rows -> NaN instead of 0
  int32_t q_vec;      // q rows are 16-byte aligned with unit d-stride
  int32_t by_length;  // seq_lens given, 2 <= B <= 64: grid rows dealt by length
};

struct CombineArgs {
  const float* part_m;
  const float* part_l;
  const float* part_acc;
  void* out;
  float* lse;
  int64_t o_sb, o_sh, o_sd;
  int64_t n_rows;          // batch * n_heads
  int32_t n_heads, head_dim, num_splits;
  int32_t empty_nan;
};

// Batch row served by grid row z when the sequences are dealt by length (a
// bijection of [0, B)): the first ceil(B/2) grid rows take the sequences in
// decreasing length, the others in increasing length.  The blocks of one
// dispatch round fill the CUs in grid order, so the two blocks a CU receives
// (grid rows z and z + ceil(B/2)) then pair a long sequence with a short one
// instead of two arbitrary ones, and the CUs stream similar numbers of keys.
// One lane per sequence (B <= 64); ties are broken by index.  Returns the
// batch row and stores its seq_lens entry in *len.
__device__ inline int length_ranked_batch(const int64_t* seq_lens, int B, int z, int lane,
                                          int64_t* len) {
  const int64_t my = lane < B ? seq_lens[lane] : 0;
  int rank = 0;
  for (int t = 0; t < B; ++t) {
    const int64_t o = ((int64_t)__builtin_amdgcn_readlane((int)(my >> 32), t) << 32) |
                      (uint32_t)__builtin_amdgcn_readlane((int)my, t);
    rank += (o > my || (o == my && t < lane)) ? 1 : 0;
  }
  const int first = B - B / 2;
  const int r = z < first ? z : B - 1 - (z - first);
  const uint64_t hit = __builtin_amdgcn_ballot_w64(lane < B && rank == r);
  const int b = (int)__builtin_ctzll(hit);
  *len = ((int64_t)__builtin_amdgcn_readlane((int)(my >> 32), b) << 32) |
         (uint32_t)__builtin_amdgcn_readlane((int)my, b);
  return b;
}

// q.k over one 16-byte chunk, fp32 accumulate.
template <typename T>
__device__ inline float dot_chunk(const u32x4& q, const u32x4& k, float acc);

template <>
__device__ inline float dot_chunk<bf16_t>(const u32x4& q, const u32x4& k,
                                          float acc) {
  const uint32_t qa[4] = {q.x, q.y, q.z, q.w};
  const uint32_t ka[4] = {k.x, k.y, k.z, k.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    bf16x2 a = __builtin_bit_cast(bf16x2, qa[i]);
    bf16x2 b = __builtin_bit_cast(bf16x2, ka[i]);
    acc = __builtin_amdgcn_fdot2_f32_bf16(a, b, acc, false);
  }
  return acc;
}

template <>
__device__ inline float dot_chunk<f16_t>(const u32x4& q, const u32x4& k,
                                         float acc) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const uint32_t qa[4] = {q.x, q.y, q.z, q.w};
  const uint32_t ka[4] = {k.x, k.y, k.z, k.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    h2 a = __builtin_bit_cast(h2, qa[i]);
    h2 b = __builtin_bit_cast(h2, ka[i]);
    acc = __builtin_amdgcn_fdot2(a, b, acc, false);
  }
  return acc;
}

template <>
__device__ inline float dot_chunk<float>(const u32x4& q, const u32x4& k,
                                         float acc) {
  acc = fmaf(__uint_as_float(q.x), __uint_as_float(k.x), acc);
  acc = fmaf(__uint_as_float(q.y), __uint_as_float(k.y), acc);
  acc = fmaf(__uint_as_float(q.z), __uint_as_float(k.z), acc);
  acc = fmaf(__uint_as_float(q.w), __uint_as_float(k.w), acc);
  return acc;
}

// acc + x.lo * y.lo + x.hi * y.hi over 2-byte pairs, fp32 accumulate.
template <typename T>
__device__ inline float dot2_pair(uint32_t x, uint32_t y, float acc);
template <>
__device__ inline float dot2_pair<bf16_t>(uint32_t x, uint32_t y, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x), __builtin_bit_cast(bf16x2, y),
                                         acc, false);
}
template <>
__device__ inline float dot2_pair<f16_t>(uint32_t x, uint32_t y, float acc) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, x), __builtin_bit_cast(h2, y), acc, false);
}
// Two fp32 values packed as a 2-byte pair (round to nearest even).
template <typename T>
__device__ inline uint32_t pack_pair(float x, float y);
template <>
__device__ inline uint32_t pack_pair<bf16_t>(float x, float y) {
  return __builtin_bit_cast(uint32_t, bf16x2{(__bf16)x, (__bf16)y});
}
template <>
__device__ inline uint32_t pack_pair<f16_t>(float x, float y) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, h2{(_Float16)x, (_Float16)y});
}

// x from lane (lane ^ OFF): a DPP row rotate for 8, the permlane swaps for 16
// and 32 (no LDS traffic); a ds_bpermute for the small strides.
template <int OFF>
__device__ inline float lane_xor(float x, int lane) {
  if constexpr (OFF == 8) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xF, 0xF, true));
  } else if constexpr (OFF == 16) {
    auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(x),
                                               __float_as_uint(x), false, false);
    return __uint_as_float((lane & 16) ? sw[0] : sw[1]);
  } else if constexpr (OFF == 32) {
    auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x),
                                               __float_as_uint(x), false, false);
    return __uint_as_float((lane & 32) ? sw[0] : sw[1]);
  } else {
    return shfl_xor_f32(x, OFF);
  }
}

// Register layout of a row of P elements (P a power of two, 8..256).
template <typename T, int P>
struct DecodeGeom {
  static constexpr int kEPC = 16 / Elem<T>::kBytes;       // elems per chunk
  static constexpr int kCH = P / kEPC;                     // chunks per row
  static constexpr int kLPR = kCH < 16 ? kCH : 16;         // lanes per row
  static constexpr int kCPL = kCH / kLPR;                  // chunks per lane
  static constexpr int kE = kCPL * kEPC;                   // elems per lane
  static constexpr int kRPW = 64 / kLPR;                   // rows per wave-load
  static constexpr int kU = kE <= 8 ? 4 : 2;               // row unroll
  static constexpr int kGCMax = kE <= 8 ? 4 : 2;           // heads per block
  static_assert(kCH * kEPC == P, "P must fill whole 16-byte chunks");
  static_assert(kCH % kLPR == 0, "chunks must split evenly across lanes");
};

// Mask bytes staged in LDS per window of rows (a longer split is processed in
// windows of this many rows).
constexpr int kMaskWin = 4096;

// fp32 K/V at P >= 128 hold twice the registers per row chunk; the 2-byte
// kernels with 4 heads per block at P = 8 (a row per lane) or with a mask
// (the row selection), and the masked ones at P = 256, hold the largest
// score tiles: those kernels run at most 8 waves (512 threads, 256 VGPRs),
// the others up to 16 (128 VGPRs).
template <typename T, int P, int GC, bool MASK>
constexpr int split_max_threads() {
  return ((sizeof(T) == 4 && P >= 128) || (sizeof(T) == 2 && (MASK || P == 8) && GC >= 4) ||
          (sizeof(T) == 2 && MASK && P == 256))
             ? 512
             : 1024;
}

// XCD (XCC) this wave runs on.
__device__ inline uint32_t xcc_id() {
  uint32_t x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  return x & 0xf;
}

__device__ inline int next_pow2_int(int n) {
  return n <= 1 ? 1 : 1 << (32 - __builtin_clz((unsigned)(n - 1)));
}

// The LSE combine of one (batch, head) row by one wave: weights exp2(m_s - M)
// for splits with l_s > 0 (src/flash_decode.py:182-192), numerator over
// splits in float4 columns, out = num / max(den, 1) or 0 / NaN for empty rows
// (src/flash_decode.py:203-205).  Latency-bound (a few KB per row): every
// load of the first pass is issued before any reduction (one round trip to
// the partials), and the reductions stay in registers -- no barrier.
//   lanes: 64 = NSG split groups x NCP column slots (NCP = next power of two
//   of D / 4; slots past D / 4 load column 0 and store nothing)
// head_dim % 4 == 0.  poison: write NaN (out and lse) instead of the result.
template <typename T>
__device__ inline void combine_row_wave(const CombineArgs& a, int64_t bh, int lane, bool poison) {
  constexpr int kUnroll = 8;
  const int S = a.num_splits, D = a.head_dim;
  const int b = (int)(bh / a.n_heads), h = (int)(bh % a.n_heads);
  const float* pm = a.part_m + bh * S;
  const float* pl = a.part_l + bh * S;
  const float* pacc = a.part_acc + bh * S * D;
  const int ncol = D >> 2;                   // float4 columns (<= 64)
  const int ncp = next_pow2_int(ncol);
  const int nsg = 64 / ncp;                  // split groups
  const int c = lane & (ncp - 1), sg = lane / ncp;
  const int cc = c < ncol ? c : 0;

  // first pass: (m, l) of split `lane`, and this lane's numerator columns of
  // splits sg, sg + nsg, ... with their own (m, l)
  const bool own = lane < S;
  const float my_m = own ? pm[lane] : kNegBig;
  const float my_l = own ? pl[lane] : 0.f;
  f32x4 pv[kUnroll];
  float pvm[kUnroll], pvl[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int sp = sg + u * nsg;
    const bool ok = sp < S;
    const int si = ok ? sp : 0;
    pv[u] = *reinterpret_cast<const f32x4*>(pacc + (int64_t)si * D + 4 * cc);
    pvm[u] = pm[si];
    pvl[u] = ok ? pl[si] : 0.f;
  }

  // max over non-empty splits, then the denominator
  float mx = my_l > 0.f ? my_m : kNegBig;
  for (int sp = lane + 64; sp < S; sp += 64)
    if (pl[sp] > 0.f) mx = fmaxf(mx, pm[sp]);
  float M = group_max<16>(mx);
  M = fmaxf(M, lane_xor<16>(M, lane));
  M = fmaxf(M, lane_xor<32>(M, lane));
  float den = my_l > 0.f ? fast_exp2(my_m - M) * my_l : 0.f;
  for (int sp = lane + 64; sp < S; sp += 64) {
    const float ls = pl[sp];
    if (ls > 0.f) den += fast_exp2(pm[sp] - M) * ls;
  }
  den = group_sum<16>(den);
  den += lane_xor<16>(den, lane);
  den += lane_xor<32>(den, lane);

  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < kUnroll; ++u)
    if (pvl[u] > 0.f) acc += fast_exp2(pvm[u] - M) * pv[u];
  for (int s0 = sg + nsg * kUnroll; s0 < S; s0 += nsg * kUnroll) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int sp = s0 + u * nsg;
      const bool ok = sp < S;
      const int si = ok ? sp : 0;
      pv[u] = *reinterpret_cast<const f32x4*>(pacc + (int64_t)si * D + 4 * cc);
      pvm[u] = pm[si];
      pvl[u] = ok ? pl[si] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (pvl[u] > 0.f) acc += fast_exp2(pvm[u] - M) * pv[u];
  }
  // sum the split groups: lanes c, c + ncp, c + 2 ncp, ... hold the same columns
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float x = acc[i];
    if (ncp <= 1) x += lane_xor<1>(x, lane);
    if (ncp <= 2) x += lane_xor<2>(x, lane);
    if (ncp <= 4) x += lane_xor<4>(x, lane);
    if (ncp <= 8) x += lane_xor<8>(x, lane);
    if (ncp <= 16) x += lane_xor<16>(x, lane);
    if (ncp <= 32) x += lane_xor<32>(x, lane);
    acc[i] = x;
  }
  if (sg == 0 && c < ncol) {
    T ov[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float o;
      if (poison)
        o = __builtin_nanf("");
      else if (den > 0.f)
        o = acc[i] / fmaxf(den, 1.0f);
      else
        o = a.empty_nan ? __builtin_nanf("") : 0.f;
      ov[i] = Elem<T>::from_f32(o);
    }
    T* op = reinterpret_cast<T*>(a.out) + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh +
            (int64_t)(4 * c) * a.o_sd;
    if (a.o_sd == 1 && ((uintptr_t)op % (4 * sizeof(T))) == 0) {   // the 4 columns in one store
      typedef T t4 __attribute__((ext_vector_type(4)));
      *reinterpret_cast<t4*>(op) = t4{ov[0], ov[1], ov[2], ov[3]};
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) op[(int64_t)i * a.o_sd] = ov[i];
    }
  }
  if (lane == 0 && a.lse != nullptr)
    a.lse[bh] = poison ? __builtin_nanf("")
                       : (den > 0.f ? (M + __log2f(den)) * kLn2 : -INFINITY);
}

// MASK: a.mask is set (rows are staged per window and the mask-excluded ones
// are not streamed); the no-mask instantiation is a single window.
// Block id -> work: group g = z * (Hkv * n_chunks) + kv-head chunk, z the grid
// row of the batch (dealt by length with seq_lens), split s.  Without FUSED,
// block L = g * S + s (splits of a group are consecutive blocks).  With FUSED
// (the in-launch combine), block L runs on XCD x = L mod n_xcc (the hardware's
// round-robin dealing) and takes item i = L / n_xcc of that XCD: split
// (i + x * S / n_xcc) mod S of group x + n_xcc * (i / S), so every split of a
// group lands on the group's XCD, and the XCDs start their groups at
// different key offsets (the same offsets at once alias HBM channels: 8
// groups x 128 splits ran 110 us in step, 92 rotated).  Padding blocks
// (groups past the last) exit at once.
template <typename T, int P, int GC, bool MASK, int MODE, bool FUSED, bool PIPE = false>
__global__ __launch_bounds__((PIPE ? 512 : split_max_threads<T, P, GC, MASK>())) void decode_split_kernel(DecodeArgs a) {
  using Geo = DecodeGeom<T, P>;
  constexpr int EPC = Geo::kEPC, LPR = Geo::kLPR, CPL = Geo::kCPL,
                E = Geo::kE, RPW = Geo::kRPW, U = Geo::kU;
  static_assert(MODE != 2 || GC == 1, "element loads run one head per block");
  extern __shared__ float smem[];

  const int nw = blockDim.x >> 6;
  const int tid = threadIdx.x;
  const int w = tid >> 6, lane = tid & 63;
  const int rg = lane / LPR, li = lane % LPR;
  const int S = a.num_splits;

  int gid, split;
  if constexpr (FUSED) {
    const int xcd = (int)(blockIdx.x % (unsigned)a.n_xcc);
    const int item = (int)(blockIdx.x / (unsigned)a.n_xcc);
    const int jg = item / S;
    split = item - jg * S + (xcd * S) / a.n_xcc;
    if (split >= S) split -= S;
    gid = xcd + a.n_xcc * jg;
  } else {
    gid = (int)(blockIdx.x / (unsigned)S);
    split = (int)blockIdx.x - gid * S;
  }
  if (gid >= a.n_groups) return;
  const int Y = a.n_groups / a.batch;
  const int z = gid / Y, kvc = gid - z * Y;
  const int kvh = kvc / a.n_chunks;
  const int chunk = kvc - kvh * a.n_chunks;
  int64_t len_b = 0;
  const int b = a.by_length ? length_ranked_batch(a.seq_lens, a.batch, z, lane, &len_b) : z;
  const int h0 = kvh * a.group + chunk * a.chunk_heads;
  const int ng = min(a.chunk_heads, a.group - chunk * a.chunk_heads);
  const int D = MODE == 0 ? P : a.head_dim;

  int leff = a.kv_len;
  if (a.seq_lens != nullptr) {
    const int64_t sl = a.by_length ? len_b : a.seq_lens[b];
    leff = (int)(sl < 0 ? 0 : (sl < leff ? sl : leff));
  }
  // With per-sequence lengths the splits divide each sequence's own keys
  // (the grid is sized for the capacity, so a graph replay at any length
  // keeps every split busy); otherwise they tile kv_len.
  int split_len = a.split_len;
  if (a.seq_lens != nullptr)
    split_len = ((leff + S - 1) / S + 15) & ~15;
  const int start = split * split_len;
  const int end = min(start + split_len, leff);

  // chunk j of this lane holds row elements [(li + j*LPR)*EPC, +EPC); with
  // MODE 1 only chunks below n_vchunks hold any
  bool cvalid[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) cvalid[j] = MODE == 0 || (li + j * LPR) < a.n_vchunks;

  // q chunks for this lane, raw (q.k is done on the stored precision, fp32
  // accumulate, exactly like sum(k.f32 * q.f32) in the reference); elements
  // past head_dim are zero.  All heads' loads are issued before the first
  // wait (one round trip).
  u32x4 qr[GC][CPL];
#pragma unroll
  for (int g = 0; g < GC; ++g) {
    const T* qp = reinterpret_cast<const T*>(a.q) + (int64_t)b * a.q_sb +
                  (int64_t)(h0 + min(g, ng - 1)) * a.q_sh;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int d0 = (li + j * LPR) * EPC;
      if (MODE != 2 && a.q_vec) {
        qr[g][j] = cvalid[j] ? *reinterpret_cast<const u32x4*>(qp + d0) : u32x4{0u, 0u, 0u, 0u};
      } else {
        union { u32x4 u; T t[EPC]; } tmp;
#pragma unroll
        for (int e = 0; e < EPC; ++e)
          tmp.t[e] = (d0 + e < D) ? qp[(int64_t)(d0 + e) * a.q_sd] : Elem<T>::from_f32(0.f);
        qr[g][j] = tmp.u;
      }
    }
  }
  float m[GC], l[GC], acc[GC][E];
#pragma unroll
  for (int g = 0; g < GC; ++g) {
    m[g] = kNegBig;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) acc[g][e] = 0.f;
  }

  const T* kb = reinterpret_cast<const T*>(a.k) + (int64_t)b * a.k_sb +
                (int64_t)kvh * a.k_sh + li * EPC;
  const T* vb = reinterpret_cast<const T*>(a.v) + (int64_t)b * a.v_sb +
                (int64_t)kvh * a.v_sh + li * EPC;
  // MODE 0/1 rows through buffer resources: one resource per pass at the
  // pass's first row (scalar arithmetic); each lane's byte offset of row slot
  // u within a pass is fixed.  Without a mask the resource ends at the
  // window's last row, so rows past it read zeros with no memory access at
  // those same offsets; with a mask, rows past the window or excluded by it
  // get an out-of-range offset instead.  The host keeps a pass's span (step
  // rows x row stride + a row) below kOobOffset.
  const int64_t k_rb = a.k_sl * (int64_t)sizeof(T), v_rb = a.v_sl * (int64_t)sizeof(T);
  const unsigned char* k_slab = reinterpret_cast<const unsigned char*>(a.k) +
                                ((int64_t)b * a.k_sb + (int64_t)kvh * a.k_sh) * (int64_t)sizeof(T);
  const unsigned char* v_slab = reinterpret_cast<const unsigned char*>(a.v) +
                                ((int64_t)b * a.v_sb + (int64_t)kvh * a.v_sh) * (int64_t)sizeof(T);
  const uint8_t* mb = MASK ? a.mask + (int64_t)b * a.mask_sb : nullptr;
  const int my_off = w * RPW + rg;
  // With a mask, the bytes of the current window of rows are staged in LDS
  // (after the wave-merge area) so a pass knows which rows to fetch before it
  // issues their loads: excluded rows are not streamed.
  unsigned char* msk = reinterpret_cast<unsigned char*>(smem + nw * GC * (P + 2));

  // One 16-byte chunk of row data: a 128-bit load (MODE 0/1; chunks past the
  // row load nothing) or EPC element loads (MODE 2; elements past head_dim are
  // zero).
  auto load_chunk = [&](const T* p, const int j) __attribute__((always_inline)) -> u32x4 {
    if constexpr (MODE == 2) {
      union { u32x4 u; T t[EPC]; } tmp;
      const int d0 = (li + j * LPR) * EPC;
#pragma unroll
      for (int e = 0; e < EPC; ++e)
        tmp.t[e] = (d0 + e < D) ? __builtin_nontemporal_load(p + e) : Elem<T>::from_f32(0.f);
      return tmp.u;
    } else {
      if (MODE == 1 && !cvalid[j]) return u32x4{0u, 0u, 0u, 0u};
      return load16_stream(p);
    }
  };

  // One pass over UU row groups per wave (UU * nw * RPW keys from `base`).
  // Full passes of U groups cover the split; a remainder of at most two
  // groups runs in one-group passes (so a split just past a multiple of the
  // U-group step does not pay a whole U-group pass for a few keys), a longer
  // one in one more U-group pass (one round trip instead of up to U).
  // load_rows issues the K and V loads of the UU row groups from `base`;
  // compute_rows folds them into the running softmax.
  auto load_rows = [&](auto uu_c, const int base, const int wbase, const int wend,
                       u32x4 (&kr)[decltype(uu_c)::value][CPL],
                       u32x4 (&vr)[decltype(uu_c)::value][CPL]) __attribute__((always_inline)) {
    constexpr int UU = decltype(uu_c)::value;
    int row[UU];
#pragma unroll
    for (int u = 0; u < UU; ++u) {
      row[u] = base + u * nw * RPW + my_off;
    }
    if constexpr (MODE != 2) {
      // (every term is wave-uniform; readfirstlane keeps the resources scalar)
      const int ub = __builtin_amdgcn_readfirstlane(base);
      // without a mask the resources end at wend's row, so rows at or past it
      // fall outside them (zeros, no memory access) at their fixed offsets:
      // no per-pass offset selection
      uint32_t kn = kOobOffset, vn = kOobOffset;
      if constexpr (!MASK) {
        const int64_t rows_left = (int64_t)__builtin_amdgcn_readfirstlane(wend) - ub;
        const int64_t kb_ = rows_left * k_rb, vb_ = rows_left * v_rb;
        kn = (uint32_t)(kb_ <= 0 ? 0 : (kb_ < (int64_t)kOobOffset ? kb_ : (int64_t)kOobOffset));
        vn = (uint32_t)(vb_ <= 0 ? 0 : (vb_ < (int64_t)kOobOffset ? vb_ : (int64_t)kOobOffset));
      }
      const buf_rsrc krs = make_rsrc(uniform_ptr(k_slab + (int64_t)ub * k_rb), kn);
      const buf_rsrc vrs = make_rsrc(uniform_ptr(v_slab + (int64_t)ub * v_rb), vn);
      bool ok[UU];
#pragma unroll
      for (int u = 0; u < UU; ++u) {
        ok[u] = true;
        // & (not &&): the clamped LDS read is always in bounds, and without the
        // short circuit the selection needs no branch in the pass
        if constexpr (MASK)
          ok[u] = (row[u] < wend) & (msk[min(row[u] - wbase, kMaskWin - 1)] != 0);
      }
      // every K load before any V load: the scores need only K, so the
      // first wait leaves the V stream in flight
#pragma unroll
      for (int u = 0; u < UU; ++u) {
        const int rs = u * nw * RPW + my_off;    // row slot within the pass
        const uint32_t ko = ok[u] ? (uint32_t)(rs * k_rb) + (uint32_t)(li * 16) : kOobOffset;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          kr[u][j] = (MODE == 1 && !cvalid[j]) ? u32x4{0u, 0u, 0u, 0u}
                                               : buf_load16_nt(krs, ko + (uint32_t)(j * LPR * 16));
        }
      }
#pragma unroll
      for (int u = 0; u < UU; ++u) {
        const int rs = u * nw * RPW + my_off;
        const uint32_t vo = ok[u] ? (uint32_t)(rs * v_rb) + (uint32_t)(li * 16) : kOobOffset;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          vr[u][j] = (MODE == 1 && !cvalid[j]) ? u32x4{0u, 0u, 0u, 0u}
                                               : buf_load16_nt(vrs, vo + (uint32_t)(j * LPR * 16));
        }
      }
      return;
    }
    // MODE 2: rows past the window re-read the window's last row (always in
    // bounds, never a key beyond seq_lens: a cache hit, not a stream) and are
    // dropped from the softmax below; with a mask, so are the rows it
    // excludes (2-byte K/V; fp32 keeps the plain clamp).
    auto src_row = [&](const int r) __attribute__((always_inline)) -> int64_t {
      int x = min(r, wend - 1);
      if constexpr (sizeof(T) == 2 && MASK) {
        if ((r < wend) & (msk[min(r - wbase, kMaskWin - 1)] == 0)) x = wend - 1;
      }
      return x;
    };
#pragma unroll
    for (int u = 0; u < UU; ++u) {
      const int64_t rl = src_row(row[u]);
#pragma unroll
      for (int j = 0; j < CPL; ++j)
        kr[u][j] = load_chunk(kb + rl * a.k_sl + j * LPR * EPC, j);
    }
#pragma unroll
    for (int u = 0; u < UU; ++u) {
      const int64_t rl = src_row(row[u]);
#pragma unroll
      for (int j = 0; j < CPL; ++j)
        vr[u][j] = load_chunk(vb + rl * a.v_sl + j * LPR * EPC, j);
    }
  };
  // full_c: every row of the pass is below wend (a pass of the loop body, not
  // the window's last), so only a mask can drop one
  auto compute_rows = [&](auto uu_c, auto full_c, const int base, const int wbase, const int wend,
                          u32x4 (&kr)[decltype(uu_c)::value][CPL],
                          u32x4 (&vr)[decltype(uu_c)::value][CPL]) __attribute__((always_inline)) {
    constexpr int UU = decltype(uu_c)::value;
    constexpr bool FULL = decltype(full_c)::value;
    int row[UU];
#pragma unroll
    for (int u = 0; u < UU; ++u) {
      row[u] = base + u * nw * RPW + my_off;
    }

    float s[UU][GC];
#pragma unroll
    for (int u = 0; u < UU; ++u) {
      bool keep = FULL || row[u] < wend;
      if constexpr (MASK) keep = keep & (msk[min(row[u] - wbase, kMaskWin - 1)] != 0);
      // a stand-in row adds exactly zero (its V is not a key of this row; the
      // buffer loads of MODE 0/1 already read zeros)
      if (MODE == 2 && sizeof(T) == 2 && MASK && !keep) {
#pragma unroll
        for (int j = 0; j < CPL; ++j) vr[u][j] = u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int g = 0; g < GC; ++g) {
        float t = 0.f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) t = dot_chunk<T>(qr[g][j], kr[u][j], t);
        t = group_sum<LPR>(t) * a.scale_log2;
        s[u][g] = keep ? t : -INFINITY;
      }
    }

    float p[UU][GC];
#pragma unroll
    for (int g = 0; g < GC; ++g) {
      float mx = s[0][g];
#pragma unroll
      for (int u = 1; u < UU; ++u) mx = fmaxf(mx, s[u][g]);
      const float mn = fmaxf(m[g], mx);
      const float alpha = fast_exp2(m[g] - mn);
      m[g] = mn;
      float ls = 0.f;
#pragma unroll
      for (int u = 0; u < UU; ++u) {
        p[u][g] = fast_exp2(s[u][g] - mn);
        ls += p[u][g];
      }
      l[g] = l[g] * alpha + ls;
#pragma unroll
      for (int e = 0; e < E; ++e) acc[g][e] *= alpha;
    }

    if constexpr (sizeof(T) == 2 && UU % 2 == 0) {
      // P.V two rows at a time on the packed elements: a dot2 per element and
      // head folds rows u and u+1 (their elements paired by a byte permute,
      // their p rounded to T), half the multiply-adds of fp32 and no unpacking.
      // B8 32/8 D64 at 4097 keys 20.64 -> 20.2 us per call, B16 24/8 D128
      // through mask= 75.2 -> 73.5 us (one MI355X).
#pragma unroll
      for (int u = 0; u < UU; u += 2) {
        uint32_t vp[E];
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          const uint32_t x0[4] = {vr[u][j].x, vr[u][j].y, vr[u][j].z, vr[u][j].w};
          const uint32_t x1[4] = {vr[u + 1][j].x, vr[u + 1][j].y, vr[u + 1][j].z, vr[u + 1][j].w};
#pragma unroll
          for (int wd = 0; wd < 4; ++wd) {
            vp[j * EPC + 2 * wd] = __builtin_amdgcn_perm(x1[wd], x0[wd], 0x05040100u);
            vp[j * EPC + 2 * wd + 1] = __builtin_amdgcn_perm(x1[wd], x0[wd], 0x07060302u);
          }
        }
#pragma unroll
        for (int g = 0; g < GC; ++g) {
          const uint32_t pp = pack_pair<T>(p[u][g], p[u + 1][g]);
#pragma unroll
          for (int e = 0; e < E; ++e) acc[g][e] = dot2_pair<T>(vp[e], pp, acc[g][e]);
        }
      }
    } else {
#pragma unroll
      for (int u = 0; u < UU; ++u) {
        float vf[E];
#pragma unroll
        for (int j = 0; j < CPL; ++j) Chunk<T>::unpack(vr[u][j], vf + j * EPC);
#pragma unroll
        for (int g = 0; g < GC; ++g)
#pragma unroll
          for (int e = 0; e < E; ++e) acc[g][e] = fmaf(p[u][g], vf[e], acc[g][e]);
      }
    }
  };
  auto pass = [&](auto uu_c, auto full_c, const int base, const int wbase, const int wend)
      __attribute__((always_inline)) {
    constexpr int UU = decltype(uu_c)::value;
    u32x4 kr[UU][CPL], vr[UU][CPL];
    load_rows(uu_c, base, wbase, wend, kr, vr);
    compute_rows(uu_c, full_c, base, wbase, wend, kr, vr);
  };
  const int rows_per_group = nw * RPW, step = U * rows_per_group;
  // rows [first, wend) of the window staged from wbase (the split in windows of
  // kMaskWin rows with a mask, one window without)
  auto run_window = [&](const int wbase, const int first, const int wend)
      __attribute__((always_inline)) {
    if constexpr (PIPE) {
      // Software pipeline over two register sets: the loads of the next U-group
      // pass are issued before the current pass is folded in, so a split costs
      // one round trip plus its stream instead of a round trip per pass.  Both
      // sets are named statically (the loop body is unrolled twice) so no
      // register copy waits on a load in flight; every prefetch covers at least
      // one row below wend, and the last pass's rows past wend are dropped.
      if (first >= wend) return;
      constexpr auto uc = std::integral_constant<int, U>{};
      u32x4 ka[U][CPL], va[U][CPL], kb2[U][CPL], vb2[U][CPL];
      // the window's last pass: when its rows fit in the first one or two row
      // slots (the others hold rows past wend, loaded as zeros), fold only
      // those (one slot takes the unpacked P.V: p stays fp32)
      auto last = [&](const int b0, u32x4 (&kr)[U][CPL], u32x4 (&vr)[U][CPL])
          __attribute__((always_inline)) {
        if constexpr (U == 4) {
          if (wend - b0 <= rows_per_group) {
            u32x4 k1[1][CPL], v1[1][CPL];
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
              k1[0][j] = kr[0][j];
              v1[0][j] = vr[0][j];
            }
            compute_rows(std::integral_constant<int, 1>{}, std::false_type{}, b0, wbase, wend, k1, v1);
            return;
          }
          if (wend - b0 <= 2 * rows_per_group) {
            u32x4 k2[2][CPL], v2[2][CPL];
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
              for (int j = 0; j < CPL; ++j) {
                k2[u][j] = kr[u][j];
                v2[u][j] = vr[u][j];
              }
            compute_rows(std::integral_constant<int, 2>{}, std::false_type{}, b0, wbase, wend, k2, v2);
            return;
          }
        }
        compute_rows(uc, std::false_type{}, b0, wbase, wend, kr, vr);
      };
      int base = first;
      load_rows(uc, base, wbase, wend, ka, va);
      while (true) {
        if (base + step >= wend) { last(base, ka, va); break; }
        load_rows(uc, base + step, wbase, wend, kb2, vb2);
        compute_rows(uc, std::true_type{}, base, wbase, wend, ka, va);
        base += step;
        if (base + step >= wend) { last(base, kb2, vb2); break; }
        load_rows(uc, base + step, wbase, wend, ka, va);
        compute_rows(uc, std::true_type{}, base, wbase, wend, kb2, vb2);
        base += step;
      }
      return;
    }
    int base = first;
    for (; base + step <= wend; base += step)
      pass(std::integral_constant<int, U>{}, std::true_type{}, base, wbase, wend);
    if (wend - base > 2 * rows_per_group) {
      pass(std::integral_constant<int, U>{}, std::false_type{}, base, wbase, wend);
    } else {
      for (; base < wend; base += rows_per_group)
        pass(std::integral_constant<int, 1>{}, std::false_type{}, base, wbase, wend);
    }
  };
  if constexpr (MASK) {
    for (int wbase = start; wbase < end; wbase += kMaskWin) {
      const int wend = min(wbase + kMaskWin, end);
      __syncthreads();  // the previous window's mask reads are done
      // 16 consecutive rows per thread, all 16 byte loads issued before the
      // first use (one round trip per 16 * blockDim rows; a 4096-row window
      // in one pass at 256 threads or more); rows past wend re-read the last
      // row and are never selected.  The first and last selected rows of the
      // window bound the rows streamed: a padding mask (keys j < L_b) costs
      // the keys it selects, not the cache capacity.
      const int n = wend - wbase;
      int lo = n, hi = -1;
      for (int c = tid * 16; c < n; c += blockDim.x * 16) {
        unsigned char mv[16];
#pragma unroll
        for (int e = 0; e < 16; ++e)
          mv[e] = mb[(int64_t)min(wbase + c + e, wend - 1) * a.mask_sl];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          if (mv[e] != 0 && c + e < n) {
            lo = min(lo, c + e);
            hi = max(hi, c + e);
          }
        }
        uint32_t* dst = reinterpret_cast<uint32_t*>(msk + c);
#pragma unroll
        for (int wd = 0; wd < 4; ++wd)
          dst[wd] = (uint32_t)(mv[4 * wd] != 0) | ((uint32_t)(mv[4 * wd + 1] != 0) << 8) |
                    ((uint32_t)(mv[4 * wd + 2] != 0) << 16) |
                    ((uint32_t)(mv[4 * wd + 3] != 0) << 24);
      }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        lo = min(lo, __shfl_xor(lo, off));
        hi = max(hi, __shfl_xor(hi, off));
      }
      int* bnd = reinterpret_cast<int*>(msk + kMaskWin);   // [nw] lo, [nw] hi
      if (lane == 0) {
        bnd[w] = lo;
        bnd[nw + w] = hi;
      }
      __syncthreads();
      int wlo = n, whi = -1;
      for (int ww = 0; ww < nw; ++ww) {
        wlo = min(wlo, bnd[ww]);
        whi = max(whi, bnd[nw + ww]);
      }
      if (whi >= 0) run_window(wbase, wbase + wlo, wbase + whi + 1);
    }
  } else {
    run_window(start, start, end);
  }

  // Merge the RPW row groups of this wave (butterfly over lane strides).
  auto merge_off = [&](auto off_c) {
    constexpr int OFF = decltype(off_c)::value;
#pragma unroll
    for (int g = 0; g < GC; ++g) {
      const float mo = lane_xor<OFF>(m[g], lane);
      const float lo = lane_xor<OFF>(l[g], lane);
      const float mn = fmaxf(m[g], mo);
      const float wa = fast_exp2(m[g] - mn), wb = fast_exp2(mo - mn);
      l[g] = l[g] * wa + lo * wb;
#pragma unroll
      for (int e = 0; e < E; ++e)
        acc[g][e] = acc[g][e] * wa + lane_xor<OFF>(acc[g][e], lane) * wb;
      m[g] = mn;
    }
  };
  if constexpr (LPR <= 1) merge_off(std::integral_constant<int, 1>{});
  if constexpr (LPR <= 2) merge_off(std::integral_constant<int, 2>{});
  if constexpr (LPR <= 4) merge_off(std::integral_constant<int, 4>{});
  if constexpr (LPR <= 8) merge_off(std::integral_constant<int, 8>{});
  if constexpr (LPR <= 16) merge_off(std::integral_constant<int, 16>{});
  merge_off(std::integral_constant<int, 32>{});

  // Cross-wave merge through LDS: [nw][GC] m, l and [nw][GC][P] acc.
  float* sm_m = smem;
  float* sm_l = smem + nw * GC;
  float* sm_acc = smem + 2 * nw * GC;
  if (rg == 0) {
#pragma unroll
    for (int g = 0; g < GC; ++g) {
#pragma unroll
      for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int e = 0; e < EPC; ++e)
          sm_acc[(w * GC + g) * P + (li + j * LPR) * EPC + e] =
              acc[g][j * EPC + e];
      if (li == 0) {
        sm_m[w * GC + g] = m[g];
        sm_l[w * GC + g] = l[g];
      }
    }
  }
  __syncthreads();

  for (int idx = tid; idx < ng * D; idx += blockDim.x) {
    const int g = idx / D, d = idx - g * D;
    float M = kNegBig;
    for (int ww = 0; ww < nw; ++ww) M = fmaxf(M, sm_m[ww * GC + g]);
    float L = 0.f, A = 0.f;
    for (int ww = 0; ww < nw; ++ww) {
      const float wt = fast_exp2(sm_m[ww * GC + g] - M);
      L += wt * sm_l[ww * GC + g];
      A += wt * sm_acc[(ww * GC + g) * P + d];
    }
    const int h = h0 + g;
    if (a.direct) {
      float o;
      if (L > 0.f)
        o = A / L;
      else
        o = a.empty_nan ? __builtin_nanf("") : 0.f;
      T* op = reinterpret_cast<T*>(a.out) + (int64_t)b * a.o_sb +
              (int64_t)h * a.o_sh + (int64_t)d * a.o_sd;
      *op = Elem<T>::from_f32(o);
      if (d == 0 && a.lse != nullptr)
        a.lse[(int64_t)b * a.n_heads + h] =
            L > 0.f ? (M + __log2f(L)) * kLn2 : -INFINITY;
    } else {
      const int64_t bh = (int64_t)b * a.n_heads + h;
      a.part_acc[(bh * S + split) * D + d] = A;
      if (d == 0) {
        a.part_m[bh * S + split] = M;
        a.part_l[bh * S + split] = L;
      }
    }
  }

  if constexpr (!FUSED) return;
  // In-launch combine.  Every split of this group ran on this group's XCD,
  // whose L2 holds the partials once each thread's stores are acknowledged
  // (s_waitcnt vmcnt(0)).  One arrival per block, one 64-bit atomic add of
  // (1, v, v*v) with v = XCD id + 1 into the fields [15:0] count, [31:16] sum
  // of v, [63:32] sum of v^2 (exact for S <= 4095).  The block that completes
  // the count learns whether every arrival came from its own XCD -- sum ==
  // S*v and sum of squares == S*v^2 hold iff all S values equal v (zero
  // variance) -- the only case in which its L2 is known to hold all partials;
  // it resets the counter for the next call, drops its CU's L1 copies
  // (buffer_inv sc0) and combines the group's rows, one wave per query head
  // (NaN rows if the arrivals were not all on its XCD).  The others exit: no
  // block waits for another.
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  int* flag = reinterpret_cast<int*>(smem);   // the merge area is no longer read
  if (tid == 0) {
    const unsigned long long v = xcc_id() + 1;
    const unsigned long long inc = 1ull | (v << 16) | ((v * v) << 32);
    const unsigned long long now =
        __hip_atomic_fetch_add(a.arrive + gid, inc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) +
        inc;
    int st = 0;
    if ((int)(now & 0xffff) == S) {
      __hip_atomic_store(a.arrive + gid, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const unsigned long long s1 = (now >> 16) & 0xffff, s2 = now >> 32;
      st = (s1 == (unsigned long long)S * v && s2 == (unsigned long long)S * v * v) ? 1 : 2;
    }
    flag[0] = st;
  }
  __syncthreads();
  const int st = flag[0];
  if (st == 0) return;
  __asm__ volatile("buffer_inv sc0" ::: "memory");
  CombineArgs c{};
  c.part_m = a.part_m;
  c.part_l = a.part_l;
  c.part_acc = a.part_acc;
  c.out = a.out;
  c.lse = a.lse;
  c.o_sb = a.o_sb; c.o_sh = a.o_sh; c.o_sd = a.o_sd;
  c.n_heads = a.n_heads;
  c.head_dim = D;
  c.num_splits = S;
  c.empty_nan = a.empty_nan;
  for (int g = w; g < ng; g += nw)
    combine_row_wave<T>(c, (int64_t)b * a.n_heads + h0 + g, lane, st == 2);
}

// One wave per (batch, head) row, four per workgroup (combine_row_wave).
template <typename T>
__global__ __launch_bounds__(256) void decode_combine_wave_kernel(CombineArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t bh = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (bh >= a.n_rows) return;
  combine_row_wave<T>(a, bh, lane, false);
}

// Many splits: one workgroup per (batch, head): weights exp2(m_s - M) for splits with
// l_s > 0 (src/flash_decode.py:182-192), numerator over splits in VEC-wide
// columns (VEC 4 for head_dim % 4 == 0, else 1), out = num/den or 0/NaN for
// empty rows (src/flash_decode.py:203-205).
// Latency-bound (a few KB per row): every thread issues all of its partial
// loads (m, l and its first 8 numerator rows) before it reduces, so a call of
// up to 256 splits costs one round trip to the partials, not one per split.
template <typename T, int VEC>
__global__ __launch_bounds__(256) void decode_combine_block_kernel(CombineArgs a) {
  constexpr int kUnroll = 8;
  typedef float vec_t __attribute__((ext_vector_type(VEC)));
  extern __shared__ float smem[];
  __shared__ float red[2][4];
  const int S = a.num_splits, D = a.head_dim;
  const int64_t bh = blockIdx.x;
  const int b = (int)(bh / a.n_heads), h = (int)(bh % a.n_heads);
  const float* pm = a.part_m + bh * S;
  const float* pl = a.part_l + bh * S;
  const float* pacc = a.part_acc + bh * S * D;
  float* sw = smem;        // [S] weights
  float* sacc = smem + S;  // [NSP][D] partial numerators
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;

  // Every load of the first pass is issued before any reduction: this
  // thread's (m, l) of split `tid` and its numerator columns of splits
  // sp, sp + nsp, ... (the barriers below would otherwise order the numerator
  // loads behind the max and the denominator: two round trips instead of one).
  // Column slots past D / VEC (padding to a power of two) load column 0 and
  // store nothing.
  const int ncol = D / VEC;
  const int ncp = next_pow2_int(ncol);
  const int nsp = 256 / ncp;
  const int c = tid & (ncp - 1), sp = tid / ncp;
  const int cc = c < ncol ? c : 0;
  const bool own = tid < S;                       // splits past 256: loops below
  const float my_m = own ? pm[tid] : kNegBig;
  const float my_l = own ? pl[tid] : 0.f;
  vec_t pv[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int s = sp + u * nsp;
    pv[u] = s < S ? *reinterpret_cast<const vec_t*>(pacc + (int64_t)s * D + VEC * cc)
                  : vec_t(0.f);
  }

  // max over non-empty splits
  float mx = my_l > 0.f ? my_m : kNegBig;
  for (int s = tid + 256; s < S; s += 256)
    if (pl[s] > 0.f) mx = fmaxf(mx, pm[s]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, shfl_xor_f32(mx, off));
  if (lane == 0) red[0][w] = mx;
  __syncthreads();
  const float M = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));

  float den = 0.f;
  if (own) {
    const float wt = my_l > 0.f ? fast_exp2(my_m - M) : 0.f;
    sw[tid] = wt;
    den = wt * my_l;
  }
  for (int s = tid + 256; s < S; s += 256) {
    const float ls = pl[s];
    const float wt = ls > 0.f ? fast_exp2(pm[s] - M) : 0.f;
    sw[s] = wt;
    den += wt * ls;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) den += shfl_xor_f32(den, off);
  if (lane == 0) red[1][w] = den;
  __syncthreads();  // also publishes sw[]
  den = red[1][0] + red[1][1] + red[1][2] + red[1][3];

  vec_t acc = vec_t(0.f);
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int s = sp + u * nsp;
    const float wt = s < S ? sw[s] : 0.f;
    if (wt != 0.f) acc += wt * pv[u];
  }
  for (int s0 = sp + nsp * kUnroll; s0 < S; s0 += nsp * kUnroll) {
    float wt[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int s = s0 + u * nsp;
      const bool ok = s < S;
      wt[u] = ok ? sw[s] : 0.f;
      pv[u] = ok ? *reinterpret_cast<const vec_t*>(pacc + (int64_t)s * D + VEC * cc)
                 : vec_t(0.f);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (wt[u] != 0.f) acc += wt[u] * pv[u];
  }
  if (c < ncol) *reinterpret_cast<vec_t*>(sacc + sp * D + VEC * c) = acc;
  __syncthreads();
  for (int d = tid; d < D; d += 256) {
    float num = 0.f;
    for (int i = 0; i < nsp; ++i) num += sacc[i * D + d];
    float o;
    if (den > 0.f)
      o = num / fmaxf(den, 1.0f);
    else
      o = a.empty_nan ? __builtin_nanf("") : 0.f;
    T* op = reinterpret_cast<T*>(a.out) + (int64_t)b * a.o_sb +
            (int64_t)h * a.o_sh + (int64_t)d * a.o_sd;
    *op = Elem<T>::from_f32(o);
  }
  if (tid == 0 && a.lse != nullptr)
    a.lse[bh] = den > 0.f ? (M + __log2f(den)) * kLn2 : -INFINITY;
}

// ------------------------------------------------------------------ host
// Launch plan shared by both translation units.
struct DecodePlan {
  int n_chunks, chunk_heads, split_len, nw;
  int n_xcc, n_groups;
  int P, mode;
  bool fused;   // in-launch combine (MODE 0, no mask; a.arrive set)
  bool pipe;    // software-pipelined passes (2-byte MODE 0; at most 8 waves)
  bool pipe2;   // two blocks per CU: pipelined passes for calls without a mask
  int nw_pipe2; // waves per block of those launches
};

template <typename T, int P, int GC, int MODE>
hipError_t launch_split_unpiped(const DecodeArgs& a, const DecodePlan& p, hipStream_t stream);

template <typename T, int P, int GC, int MODE>
hipError_t launch_split_t(const DecodeArgs& a, const DecodePlan& p, hipStream_t stream) {
  const int S = a.num_splits;
  if constexpr (MODE == 0 && sizeof(T) == 2) {
    // 2-byte K/V with whole-chunk rows: the software-pipelined kernels when
    // the plan asks for them
    const bool piped = p.pipe || (p.pipe2 && a.mask == nullptr);
    if (!piped) return launch_split_unpiped<T, P, GC, MODE>(a, p, stream);
    const int nw = min(p.pipe ? p.nw : p.nw_pipe2, 8);   // built for at most 512 threads
    const size_t shmem = (size_t)nw * GC * (P + 2) * sizeof(float);
    const dim3 grid((unsigned)(p.n_groups * S));
    if (a.mask != nullptr) {
      hipLaunchKernelGGL((decode_split_kernel<T, P, GC, true, 0, false, true>), grid,
                         dim3((unsigned)(nw * 64)), shmem + kMaskWin + 8 * nw, stream, a);
    } else if (p.fused) {
      const int per_xcc = (p.n_groups + p.n_xcc - 1) / p.n_xcc;
      hipLaunchKernelGGL((decode_split_kernel<T, P, GC, false, 0, true, true>),
                         dim3((unsigned)(p.n_xcc * per_xcc * S)), dim3((unsigned)(nw * 64)),
                         shmem, stream, a);
    } else {
      hipLaunchKernelGGL((decode_split_kernel<T, P, GC, false, 0, false, true>), grid,
                         dim3((unsigned)(nw * 64)), shmem, stream, a);
    }
    return hipGetLastError();
  } else {
    return launch_split_unpiped<T, P, GC, MODE>(a, p, stream);
  }
}

// One pass of loads in flight per wave, up to 16 waves per block.
template <typename T, int P, int GC, int MODE>
hipError_t launch_split_unpiped(const DecodeArgs& a, const DecodePlan& p, hipStream_t stream) {
  const int S = a.num_splits;
  if (a.mask != nullptr) {
    const int nw = min(p.nw, split_max_threads<T, P, GC, true>() / 64);
    const size_t shmem = (size_t)nw * GC * (P + 2) * sizeof(float) + kMaskWin + 8 * nw;
    hipLaunchKernelGGL((decode_split_kernel<T, P, GC, true, MODE, false>),
                       dim3((unsigned)(p.n_groups * S)), dim3((unsigned)(nw * 64)), shmem, stream,
                       a);
    return hipGetLastError();
  }
  const int nw = min(p.nw, split_max_threads<T, P, GC, false>() / 64);
  const size_t shmem = (size_t)nw * GC * (P + 2) * sizeof(float);
  if constexpr (MODE == 0) {
    if (p.fused) {
      const int per_xcc = (p.n_groups + p.n_xcc - 1) / p.n_xcc;
      hipLaunchKernelGGL((decode_split_kernel<T, P, GC, false, 0, true>),
                         dim3((unsigned)(p.n_xcc * per_xcc * S)), dim3((unsigned)(nw * 64)),
                         shmem, stream, a);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((decode_split_kernel<T, P, GC, false, MODE, false>),
                     dim3((unsigned)(p.n_groups * S)), dim3((unsigned)(nw * 64)), shmem, stream,
                     a);
  return hipGetLastError();
}

template <typename T, int P, int MODE>
hipError_t launch_split_p(const DecodeArgs& a, const DecodePlan& p, hipStream_t stream) {
  if constexpr (MODE == 2) {
    if (p.chunk_heads == 1) return launch_split_t<T, P, 1, 2>(a, p, stream);
    return hipErrorInvalidValue;
  } else {
    constexpr int gmax = DecodeGeom<T, P>::kGCMax;
    switch (p.chunk_heads) {
      case 1: return launch_split_t<T, P, 1, MODE>(a, p, stream);
      case 2: return launch_split_t<T, P, 2, MODE>(a, p, stream);
      case 3:
        if constexpr (gmax >= 3) return launch_split_t<T, P, 3, MODE>(a, p, stream);
        break;
      case 4:
        if constexpr (gmax >= 4) return launch_split_t<T, P, 4, MODE>(a, p, stream);
        break;
      default: break;
    }
    return hipErrorInvalidValue;
  }
}

template <typename T, int MODE>
hipError_t launch_split_mode(const DecodeArgs& a, const DecodePlan& p, hipStream_t stream) {
  switch (p.P) {
    case 8: return launch_split_p<T, 8, MODE>(a, p, stream);
    case 16: return launch_split_p<T, 16, MODE>(a, p, stream);
    case 32: return launch_split_p<T, 32, MODE>(a, p, stream);
    case 64: return launch_split_p<T, 64, MODE>(a, p, stream);
    case 128: return launch_split_p<T, 128, MODE>(a, p, stream);
    case 256: return launch_split_p<T, 256, MODE>(a, p, stream);
    default: return hipErrorInvalidValue;
  }
}

// MODE 1 and 2 launches (decode_pad.hip).
hipError_t launch_split_padded(int32_t dtype, const DecodeArgs& a, const DecodePlan& p,
                               hipStream_t stream);

}  // namespace mi
