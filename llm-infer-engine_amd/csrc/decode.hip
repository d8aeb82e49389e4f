// Split-KV single-token decode attention for gfx950 (bandwidth-bound path).
//
// Math follows the reference's split/combine decode
// (src/flash_decode.py:8-137 per-split partials, :140-212 LSE combine), but the
// work decomposition is MI355X-first:
//   * one workgroup per (batch, kv-head, split) computes the partial state of
//     ALL query heads that share the kv-head (GQA), so every K/V byte is read
//     from HBM exactly once (the reference re-reads it once per query head);
//   * each lane owns one 16-byte chunk of a K/V row per load (coalesced
//     128-bit global loads; a row of D elements spans LPR = D*sizeof(T)/16
//     lanes, capped at 16 = one DPP row);
//   * q.k row sums use DPP row reductions (no LDS round trip), the softmax is
//     kept per row group in registers (log2 domain, v_exp_f32); the row
//     groups of a wave merge through DPP / permlane swaps and the waves once
//     through LDS;
//   * no MFMA: at one query token per head there is nothing to amortise a
//     matrix tile over, and the loop is HBM-bound.
// Keys beyond seq_lens[b] are never loaded.  The grid is static (sized for
// the capacity, so the launch is hipGraph-safe) and with seq_lens the splits
// divide each sequence's own length, so a replay at any length keeps every
// split busy.
#include <math.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "common.hpp"

// Workspace of mi_flash_decode_noalloc: the split partials (acc, m, l) of one
// call, for callers that cannot allocate.  Each device holds its own copy for
// the life of the process; host code reaches it only through the address
// hipGetSymbolAddress returns for the current device (scratch_base below).
static __device__ __align__(256) unsigned char scratch[MI_DECODE_NOALLOC_SCRATCH_BYTES];

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
  int64_t q_sb, q_sh, q_sd;
  int64_t k_sb, k_sh, k_sl;
  int64_t v_sb, v_sh, v_sl;
  int64_t o_sb, o_sh, o_sd;
  int32_t n_heads, group, kv_len;
  int32_t split_len, num_splits, n_chunks, chunk_heads;
  float scale_log2;
  int32_t direct;     // num_splits == 1: normalise and write out/lse here
  int32_t empty_nan;  // empty rows -> NaN instead of 0
  int32_t q_vec;      // q rows are 16-byte aligned with unit d-stride
  int32_t by_length;  // seq_lens given, 2 <= B <= 64: grid rows dealt by length
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

template <typename T, int D>
struct DecodeGeom {
  static constexpr int kEPC = 16 / Elem<T>::kBytes;       // elems per chunk
  static constexpr int kCH = D / kEPC;                     // chunks per row
  static constexpr int kLPR = kCH < 16 ? kCH : 16;         // lanes per row
  static constexpr int kCPL = kCH / kLPR;                  // chunks per lane
  static constexpr int kE = kCPL * kEPC;                   // elems per lane
  static constexpr int kRPW = 64 / kLPR;                   // rows per wave-load
  static constexpr int kU = kE <= 8 ? 4 : 2;               // row unroll
  static constexpr int kGCMax = kE <= 8 ? 4 : 2;           // heads per block
  static_assert(kCH * kEPC == D, "head_dim must fill whole 16-byte chunks");
  static_assert(kCH % kLPR == 0, "chunks must split evenly across lanes");
};

// Mask bytes staged in LDS per window of rows (a longer split is processed in
// windows of this many rows).
constexpr int kMaskWin = 4096;

// fp32 K/V at head_dim >= 128 hold twice the registers per row chunk, and the
// masked 2-byte kernels with 4 heads per block add the row selection to the
// largest score tile: those kernels run at most 8 waves (512 threads, 256
// VGPRs), the others up to 16 (128 VGPRs).
template <typename T, int D, int GC, bool MASK>
constexpr int split_max_threads() {
  return ((sizeof(T) == 4 && D >= 128) || (sizeof(T) == 2 && MASK && GC >= 4)) ? 512 : 1024;
}

// MASK: a.mask is set (rows are staged per window and the mask-excluded ones
// are not streamed); the no-mask instantiation is a single window.
template <typename T, int D, int GC, bool MASK>
__global__ __launch_bounds__((split_max_threads<T, D, GC, MASK>())) void decode_split_kernel(DecodeArgs a) {
  using Geo = DecodeGeom<T, D>;
  constexpr int EPC = Geo::kEPC, LPR = Geo::kLPR, CPL = Geo::kCPL,
                E = Geo::kE, RPW = Geo::kRPW, U = Geo::kU;
  extern __shared__ float smem[];

  const int nw = blockDim.x >> 6;
  const int tid = threadIdx.x;
  const int w = tid >> 6, lane = tid & 63;
  const int rg = lane / LPR, li = lane % LPR;

  const int split = blockIdx.x;
  const int kvh = blockIdx.y / a.n_chunks;
  const int chunk = blockIdx.y - kvh * a.n_chunks;
  int64_t len_b = 0;
  const int b = a.by_length
                    ? length_ranked_batch(a.seq_lens, (int)gridDim.z, (int)blockIdx.z, lane, &len_b)
                    : (int)blockIdx.z;
  const int h0 = kvh * a.group + chunk * a.chunk_heads;
  const int ng = min(a.chunk_heads, a.group - chunk * a.chunk_heads);

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
    split_len = ((leff + a.num_splits - 1) / a.num_splits + 15) & ~15;
  const int start = split * split_len;
  const int end = min(start + split_len, leff);

  // q chunks for this lane, raw (q.k is done on the stored precision, fp32
  // accumulate, exactly like sum(k.f32 * q.f32) in the reference).
  // All heads' loads are issued before the first wait (one round trip).
  u32x4 qr[GC][CPL];
  if (a.q_vec) {
#pragma unroll
    for (int g = 0; g < GC; ++g) {
      const T* qp = reinterpret_cast<const T*>(a.q) + (int64_t)b * a.q_sb +
                    (int64_t)(h0 + min(g, ng - 1)) * a.q_sh;
#pragma unroll
      for (int j = 0; j < CPL; ++j)
        qr[g][j] = *reinterpret_cast<const u32x4*>(qp + (li + j * LPR) * EPC);
    }
  } else {
#pragma unroll
    for (int g = 0; g < GC; ++g) {
      const T* qp = reinterpret_cast<const T*>(a.q) + (int64_t)b * a.q_sb +
                    (int64_t)(h0 + min(g, ng - 1)) * a.q_sh;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int d0 = (li + j * LPR) * EPC;
        union { u32x4 u; T t[EPC]; } tmp;
#pragma unroll
        for (int e = 0; e < EPC; ++e) tmp.t[e] = qp[(int64_t)(d0 + e) * a.q_sd];
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
  const uint8_t* mb = MASK ? a.mask + (int64_t)b * a.mask_sb : nullptr;
  const int my_off = w * RPW + rg;
  // With a mask, the bytes of the current window of rows are staged in LDS
  // (after the wave-merge area) so a pass knows which rows to fetch before it
  // issues their loads: excluded rows are not streamed.
  unsigned char* msk = reinterpret_cast<unsigned char*>(smem + nw * GC * (D + 2));

  // One pass over UU row groups per wave (UU * nw * RPW keys from `base`).
  // Full passes of U groups cover the split; a remainder of at most two
  // groups runs in one-group passes (so a split just past a multiple of the
  // U-group step does not pay a whole U-group pass for a few keys), a longer
  // one in one more U-group pass (one round trip instead of up to U).
  auto pass = [&](auto uu_c, const int base, const int wbase, const int wend)
      __attribute__((always_inline)) {
    constexpr int UU = decltype(uu_c)::value;
    u32x4 kr[UU][CPL], vr[UU][CPL];
    int row[UU];
#pragma unroll
    for (int u = 0; u < UU; ++u) {
      row[u] = base + u * nw * RPW + my_off;
    }
    // Rows past the window re-read the window's last row (always in bounds,
    // never a key beyond seq_lens: a cache hit, not a stream) and are dropped
    // from the softmax below; with a mask, so are the rows it excludes (2-byte
    // K/V; fp32 keeps the plain clamp, the 1024-thread kernels have no
    // registers to spare for the row selection).
    auto src_row = [&](const int r) __attribute__((always_inline)) -> int64_t {
      int x = min(r, wend - 1);
      if constexpr (sizeof(T) == 2 && MASK) {
        if (r < wend && msk[r - wbase] == 0) x = wend - 1;
      }
      return x;
    };
#pragma unroll
    for (int u = 0; u < UU; ++u) {
      const int64_t rl = src_row(row[u]);
#pragma unroll
      for (int j = 0; j < CPL; ++j)
        kr[u][j] = load16_stream(kb + rl * a.k_sl + j * LPR * EPC);
    }
#pragma unroll
    for (int u = 0; u < UU; ++u) {
      const int64_t rl = src_row(row[u]);
#pragma unroll
      for (int j = 0; j < CPL; ++j)
        vr[u][j] = load16_stream(vb + rl * a.v_sl + j * LPR * EPC);
    }

    float s[UU][GC];
#pragma unroll
    for (int u = 0; u < UU; ++u) {
      bool keep = row[u] < wend;
      if (MASK && keep) keep = msk[row[u] - wbase] != 0;
      // a stand-in row adds exactly zero (its V is not a key of this row)
      if (sizeof(T) == 2 && MASK && !keep) {
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
  };
  const int grp = nw * RPW, step = U * grp;
  // the split in windows of kMaskWin rows with a mask (one window without)
  auto run_window = [&](const int wbase, const int wend) __attribute__((always_inline)) {
    int base = wbase;
    for (; base + step <= wend; base += step)
      pass(std::integral_constant<int, U>{}, base, wbase, wend);
    if (wend - base > 2 * grp) {
      pass(std::integral_constant<int, U>{}, base, wbase, wend);
    } else {
      for (; base < wend; base += grp) pass(std::integral_constant<int, 1>{}, base, wbase, wend);
    }
  };
  if constexpr (MASK) {
    for (int wbase = start; wbase < end; wbase += kMaskWin) {
      const int wend = min(wbase + kMaskWin, end);
      __syncthreads();  // the previous window's mask reads are done
      for (int i = tid; i < wend - wbase; i += blockDim.x)
        msk[i] = mb[(int64_t)(wbase + i) * a.mask_sl] != 0;
      __syncthreads();
      run_window(wbase, wend);
    }
  } else {
    run_window(start, end);
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

  // Cross-wave merge through LDS: [nw][GC] m, l and [nw][GC][D] acc.
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
          sm_acc[(w * GC + g) * D + (li + j * LPR) * EPC + e] =
              acc[g][j * EPC + e];
      if (li == 0) {
        sm_m[w * GC + g] = m[g];
        sm_l[w * GC + g] = l[g];
      }
    }
  }
  __syncthreads();

  const int S = a.num_splits;
  for (int idx = tid; idx < ng * D; idx += blockDim.x) {
    const int g = idx / D, d = idx - g * D;
    float M = kNegBig;
    for (int ww = 0; ww < nw; ++ww) M = fmaxf(M, sm_m[ww * GC + g]);
    float L = 0.f, A = 0.f;
    for (int ww = 0; ww < nw; ++ww) {
      const float wt = fast_exp2(sm_m[ww * GC + g] - M);
      L += wt * sm_l[ww * GC + g];
      A += wt * sm_acc[(ww * GC + g) * D + d];
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
}

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

// Wave-wide reductions over all 64 lanes (DPP within rows of 16, permlane
// swaps across them; no LDS).
__device__ inline float wave_max(float x, int lane) {
  x = group_max<16>(x);
  x = fmaxf(x, lane_xor<16>(x, lane));
  return fmaxf(x, lane_xor<32>(x, lane));
}
__device__ inline float wave_sum(float x, int lane) {
  x = group_sum<16>(x);
  x += lane_xor<16>(x, lane);
  return x + lane_xor<32>(x, lane);
}

// One wave per (batch, head), four per workgroup: weights exp2(m_s - M) for
// splits with l_s > 0 (src/flash_decode.py:182-192), numerator over splits in
// float4 columns, out = num / max(den, 1) or 0 / NaN for empty rows
// (src/flash_decode.py:203-205).  Latency-bound (a few KB per row): every
// load of the first pass is issued before any reduction (one round trip to
// the partials), and the reductions stay in registers -- no barrier.
//   lanes: 64 = NSG split groups x (D / 4) column chunks
template <typename T>
__global__ __launch_bounds__(256) void decode_combine_wave_kernel(CombineArgs a) {
  constexpr int kUnroll = 8;
  const int lane = threadIdx.x & 63;
  const int64_t bh = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (bh >= a.n_rows) return;
  const int S = a.num_splits, D = a.head_dim;
  const int b = (int)(bh / a.n_heads), h = (int)(bh % a.n_heads);
  const float* pm = a.part_m + bh * S;
  const float* pl = a.part_l + bh * S;
  const float* pacc = a.part_acc + bh * S * D;
  const int ncol = D >> 2;                   // float4 columns (<= 64)
  const int nsg = 64 / ncol;                 // split groups
  const int c = lane % ncol, sg = lane / ncol;

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
    pv[u] = *reinterpret_cast<const f32x4*>(pacc + (int64_t)si * D + 4 * c);
    pvm[u] = pm[si];
    pvl[u] = ok ? pl[si] : 0.f;
  }

  // max over non-empty splits, then the denominator
  float mx = my_l > 0.f ? my_m : kNegBig;
  for (int sp = lane + 64; sp < S; sp += 64)
    if (pl[sp] > 0.f) mx = fmaxf(mx, pm[sp]);
  const float M = wave_max(mx, lane);
  float den = my_l > 0.f ? fast_exp2(my_m - M) * my_l : 0.f;
  for (int sp = lane + 64; sp < S; sp += 64) {
    const float ls = pl[sp];
    if (ls > 0.f) den += fast_exp2(pm[sp] - M) * ls;
  }
  den = wave_sum(den, lane);

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
      pv[u] = *reinterpret_cast<const f32x4*>(pacc + (int64_t)si * D + 4 * c);
      pvm[u] = pm[si];
      pvl[u] = ok ? pl[si] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (pvl[u] > 0.f) acc += fast_exp2(pvm[u] - M) * pv[u];
  }
  // sum the split groups: lanes c, c + ncol, c + 2 ncol, ... hold the same columns
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float x = acc[i];
    if (ncol <= 4) x += lane_xor<4>(x, lane);
    if (ncol <= 8) x += lane_xor<8>(x, lane);
    if (ncol <= 16) x += lane_xor<16>(x, lane);
    if (ncol <= 32) x += lane_xor<32>(x, lane);
    acc[i] = x;
  }
  if (sg == 0) {
    T ov[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float o;
      if (den > 0.f)
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
    a.lse[bh] = den > 0.f ? (M + __log2f(den)) * kLn2 : -INFINITY;
}

// Many splits: one workgroup per (batch, head): weights exp2(m_s - M) for splits with
// l_s > 0 (src/flash_decode.py:182-192), numerator over splits in float4
// columns, out = num/den or 0/NaN for empty rows (src/flash_decode.py:203-205).
// Latency-bound (a few KB per row): every thread issues all of its partial
// loads (m, l and its first 8 numerator rows) before it reduces, so a call of
// up to 256 splits costs one round trip to the partials, not one per split.
template <typename T>
__global__ __launch_bounds__(256) void decode_combine_block_kernel(CombineArgs a) {
  constexpr int kUnroll = 8;
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
  const int ncol = D >> 2;
  const int nsp = 256 / ncol;
  const int c = tid % ncol, sp = tid / ncol;
  const bool own = tid < S;                       // splits past 256: loops below
  const float my_m = own ? pm[tid] : kNegBig;
  const float my_l = own ? pl[tid] : 0.f;
  f32x4 pv[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int s = sp + u * nsp;
    pv[u] = s < S ? *reinterpret_cast<const f32x4*>(pacc + (int64_t)s * D + 4 * c)
                  : f32x4{0.f, 0.f, 0.f, 0.f};
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

  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
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
      pv[u] = ok ? *reinterpret_cast<const f32x4*>(pacc + (int64_t)s * D + 4 * c)
                 : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (wt[u] != 0.f) acc += wt[u] * pv[u];
  }
  *reinterpret_cast<f32x4*>(sacc + sp * D + 4 * c) = acc;
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
namespace {

int elem_bytes(int32_t dtype) { return dtype == MI_DTYPE_F32 ? 4 : 2; }

// Host mirror of DecodeGeom: lanes per row, elements per lane, row unroll
// and heads per block for a dtype / head_dim.
struct HostGeom {
  int lpr, e, rpw, u, gcmax;
};
HostGeom host_geom(int32_t dtype, int64_t D) {
  const int eb = elem_bytes(dtype);
  const int ch = (int)(D * eb / 16), epc = 16 / eb;
  HostGeom g;
  g.lpr = ch < 16 ? ch : 16;
  g.e = (ch / g.lpr) * epc;
  g.rpw = 64 / g.lpr;
  g.u = g.e <= 8 ? 4 : 2;
  g.gcmax = g.e <= 8 ? 4 : 2;
  return g;
}

int gc_max(int32_t dtype, int64_t D) { return host_geom(dtype, D).gcmax; }

bool supported_head_dim(int32_t dtype, int64_t D) {
  return D == 16 || D == 32 || D == 64 || D == 128 || D == 256;
}

struct Plan {
  int n_chunks, chunk_heads, split_len, nw;
};

Plan make_plan(int32_t dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t L,
               int64_t D, int64_t S) {
  Plan p;
  const int64_t G = Hq / Hkv;
  const int gmax = gc_max(dtype, D);
  p.n_chunks = (int)((G + gmax - 1) / gmax);
  p.chunk_heads = (int)((G + p.n_chunks - 1) / p.n_chunks);
  p.split_len = (int)((L + S - 1) / S);
  const int64_t blocks = B * Hkv * p.n_chunks * S;
  const int cus = device_cu_count();
  int nw = 4;
  if (blocks < cus)
    nw = 16;
  else if (blocks < 2 * cus)
    nw = 8;
  // No more waves than the split has row-loads for.
  const HostGeom geo = host_geom(dtype, D);
  if (dtype == MI_DTYPE_F32 && D >= 128 && nw > 8) nw = 8;   // split_max_threads
  while (nw > 1 && (int64_t)nw * geo.rpw * geo.u > p.split_len) nw >>= 1;
  p.nw = nw;
  return p;
}

template <typename T, int D, int GC>
hipError_t launch_split_t(const DecodeArgs& a, const Plan& p, int64_t B,
                          int64_t Hkv, hipStream_t stream) {
  dim3 grid((unsigned)a.num_splits, (unsigned)(Hkv * p.n_chunks),
            (unsigned)B);
  if (a.mask != nullptr) {
    const int nw = min(p.nw, split_max_threads<T, D, GC, true>() / 64);
    const size_t shmem = (size_t)nw * GC * (D + 2) * sizeof(float) + kMaskWin;
    hipLaunchKernelGGL((decode_split_kernel<T, D, GC, true>), grid, dim3((unsigned)(nw * 64)),
                       shmem, stream, a);
  } else {
    const int nw = min(p.nw, split_max_threads<T, D, GC, false>() / 64);
    const size_t shmem = (size_t)nw * GC * (D + 2) * sizeof(float);
    hipLaunchKernelGGL((decode_split_kernel<T, D, GC, false>), grid, dim3((unsigned)(nw * 64)),
                       shmem, stream, a);
  }
  return hipGetLastError();
}

template <typename T, int D>
hipError_t launch_split_d(const DecodeArgs& a, const Plan& p, int64_t B,
                          int64_t Hkv, hipStream_t stream) {
  constexpr int gmax = DecodeGeom<T, D>::kGCMax;
  switch (p.chunk_heads) {
    case 1: return launch_split_t<T, D, 1>(a, p, B, Hkv, stream);
    case 2: return launch_split_t<T, D, 2>(a, p, B, Hkv, stream);
    case 3:
      if constexpr (gmax >= 3) return launch_split_t<T, D, 3>(a, p, B, Hkv, stream);
      break;
    case 4:
      if constexpr (gmax >= 4) return launch_split_t<T, D, 4>(a, p, B, Hkv, stream);
      break;
    default: break;
  }
  return hipErrorInvalidValue;
}

template <typename T>
hipError_t launch_split(const DecodeArgs& a, const Plan& p, int64_t B,
                        int64_t Hkv, int64_t D, hipStream_t stream) {
  switch (D) {
    case 16: return launch_split_d<T, 16>(a, p, B, Hkv, stream);
    case 32: return launch_split_d<T, 32>(a, p, B, Hkv, stream);
    case 64: return launch_split_d<T, 64>(a, p, B, Hkv, stream);
    case 128: return launch_split_d<T, 128>(a, p, B, Hkv, stream);
    case 256: return launch_split_d<T, 256>(a, p, B, Hkv, stream);
    default: return hipErrorInvalidValue;
  }
}

int32_t check_common(const void* q, const void* k, const void* v,
                     int64_t B, int64_t Hq, int64_t Hkv, int64_t L,
                     int64_t D, int64_t S, int64_t k_sl, int64_t v_sl,
                     int32_t dtype) {
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
  if (!supported_head_dim(dtype, D)) {
    set_last_error("decode: head_dim %lld has no kernel (supported: 16, 32, 64, 128, 256)",
                   (long long)D);
    return MI_ERR_UNSUPPORTED;
  }
  if (L > INT32_MAX / 2 || B > 65535 || Hkv * 4 > 65535 || S > INT32_MAX / 2) {
    set_last_error("decode: shape exceeds launch limits");
    return MI_ERR_UNSUPPORTED;
  }
  const int eb = elem_bytes(dtype);
  if (((uintptr_t)k % 16) != 0 || ((uintptr_t)v % 16) != 0 ||
      ((k_sl * eb) % 16) != 0 || ((v_sl * eb) % 16) != 0) {
    set_last_error("decode: K/V rows must be 16-byte aligned");
    return MI_ERR_INVALID;
  }
  return MI_OK;
}

DecodeArgs fill_args(const void* q, const void* k, const void* v,
                     const uint8_t* mask, int64_t mask_sb, int64_t mask_sl,
                     const int64_t* seq_lens, int64_t B, int64_t Hq, int64_t Hkv,
                     int64_t L, int64_t S, int64_t q_sb, int64_t q_sh,
                     int64_t q_sd, int64_t k_sb, int64_t k_sh, int64_t k_sl,
                     int64_t v_sb, int64_t v_sh, int64_t v_sl, float sm_scale,
                     const Plan& p, int dtype_bytes) {
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
  a.n_heads = (int32_t)Hq;
  a.group = (int32_t)(Hq / Hkv);
  a.kv_len = (int32_t)L;
  a.split_len = p.split_len;
  a.num_splits = (int32_t)S;
  a.n_chunks = p.n_chunks;
  a.chunk_heads = p.chunk_heads;
  a.scale_log2 = sm_scale * kLog2e;
  const int64_t eb = dtype_bytes;
  a.q_vec = (q_sd == 1 && ((uintptr_t)q % 16) == 0 && ((q_sb * eb) % 16) == 0 &&
             ((q_sh * eb) % 16) == 0) ? 1 : 0;
  a.by_length = (seq_lens != nullptr && mask == nullptr && B >= 2 && B <= 64) ? 1 : 0;
  return a;
}

hipError_t launch_split_any(int32_t dtype, const DecodeArgs& a, const Plan& p,
                            int64_t B, int64_t Hkv, int64_t D,
                            hipStream_t stream) {
  switch (dtype) {
    case MI_DTYPE_BF16: return launch_split<bf16_t>(a, p, B, Hkv, D, stream);
    case MI_DTYPE_F16: return launch_split<f16_t>(a, p, B, Hkv, D, stream);
    default: return launch_split<float>(a, p, B, Hkv, D, stream);
  }
}

// Many rows with up to 16 splits each: one wave per (batch, head) row (no
// barriers); otherwise one workgroup per row (the splits' loads spread over
// 256 threads, which a few rows need to fill the GPU).
hipError_t launch_combine_any(int32_t dtype, const CombineArgs& c, int64_t B,
                              int64_t Hq, hipStream_t stream) {
  dim3 block(256);
  if (c.num_splits <= 16 && B * Hq >= 64) {
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
  const int D = c.head_dim;
  const int nsp = 256 / (D / 4);
  const size_t shmem = ((size_t)c.num_splits + (size_t)nsp * D) * sizeof(float);
  dim3 grid((unsigned)(B * Hq));
  switch (dtype) {
    case MI_DTYPE_BF16:
      hipLaunchKernelGGL(decode_combine_block_kernel<bf16_t>, grid, block, shmem, stream, c);
      break;
    case MI_DTYPE_F16:
      hipLaunchKernelGGL(decode_combine_block_kernel<f16_t>, grid, block, shmem, stream, c);
      break;
    default:
      hipLaunchKernelGGL(decode_combine_block_kernel<float>, grid, block, shmem, stream, c);
      break;
  }
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

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int64_t mi_decode_default_splits(int64_t batch, int64_t n_heads,
                                            int64_t n_kv_heads, int64_t kv_len,
                                            int64_t head_dim) {
  if (batch <= 0 || n_heads <= 0 || n_kv_heads <= 0 || kv_len <= 0) return 1;
  const int64_t G = n_heads / (n_kv_heads > 0 ? n_kv_heads : 1);
  const int gmax = gc_max(MI_DTYPE_BF16, head_dim > 0 ? head_dim : 128);
  const int64_t chunks = (G + gmax - 1) / gmax;
  const int64_t units = batch * n_kv_heads * (chunks > 0 ? chunks : 1);
  const int64_t cus = device_cu_count();
  int64_t s = (2 * cus + units - 1) / units;       // two blocks per CU
  // Splits keep >= 512 KB of K + V (at kv_len, the cache capacity in graph
  // mode) once the blocks already cover every CU: a block's merge and partial
  // write cost a few microseconds however little it streams, so past that
  // point shorter splits lose more than their parallelism gains (measured:
  // B8 Hkv8 D64 at 4097 of 8192 keys, 4 splits 22.9 us vs 8 splits 25.0 us).
  const int64_t row_bytes = 2LL * 2 * (head_dim > 0 ? head_dim : 128);   // bf16 K + V
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
  const int64_t G = n_heads / n_kv_heads;
  const int gmax = gc_max(MI_DTYPE_BF16, head_dim > 0 ? head_dim : 128);
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

extern "C" int32_t mi_decode_split(
    const void* q, const void* k, const void* v, const uint8_t* mask,
    int64_t mask_sb, int64_t mask_sl, const int64_t* seq_lens, float* part_m,
    float* part_l, float* part_acc, int64_t batch, int64_t n_heads,
    int64_t n_kv_heads, int64_t kv_len, int64_t head_dim, int64_t num_splits,
    int64_t q_sb, int64_t q_sh, int64_t q_sd, int64_t k_sb, int64_t k_sh,
    int64_t k_sl, int64_t v_sb, int64_t v_sh, int64_t v_sl, float sm_scale,
    int32_t dtype, void* stream) {
  int32_t st = check_common(q, k, v, batch, n_heads, n_kv_heads, kv_len,
                            head_dim, num_splits, k_sl, v_sl, dtype);
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
  Plan p = make_plan(dtype, batch, n_heads, n_kv_heads, kv_len, head_dim, num_splits);
  DecodeArgs a = fill_args(q, k, v, mask, mask_sb, mask_sl, seq_lens, batch, n_heads,
                           n_kv_heads, kv_len, num_splits, q_sb, q_sh, q_sd,
                           k_sb, k_sh, k_sl, v_sb, v_sh, v_sl, sm_scale, p,
                           elem_bytes(dtype));
  a.part_m = part_m;
  a.part_l = part_l;
  a.part_acc = part_acc;
  a.direct = 0;
  hipError_t e = launch_split_any(dtype, a, p, batch, n_kv_heads, head_dim,
                                  (hipStream_t)stream);
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
  if (head_dim != 16 && head_dim != 32 && head_dim != 64 && head_dim != 128 && head_dim != 256) {
    set_last_error("decode_combine: head_dim %lld unsupported", (long long)head_dim);
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
    float* part_l, float* part_acc, void* out, float* lse, int64_t batch,
    int64_t n_heads, int64_t n_kv_heads, int64_t kv_len, int64_t head_dim,
    int64_t num_splits, int64_t q_sb, int64_t q_sh, int64_t q_sd, int64_t k_sb,
    int64_t k_sh, int64_t k_sl, int64_t v_sb, int64_t v_sh, int64_t v_sl,
    int64_t o_sb, int64_t o_sh, int64_t o_sd, float sm_scale,
    int32_t empty_rows_nan, int32_t dtype, void* stream) {
  if (out == nullptr) {
    set_last_error("flash_decode: null output pointer");
    return MI_ERR_INVALID;
  }
  if (num_splits != 1) {
    int32_t st = mi_decode_split(q, k, v, mask, mask_sb, mask_sl, seq_lens,
                                 part_m, part_l, part_acc, batch, n_heads,
                                 n_kv_heads, kv_len, head_dim, num_splits, q_sb,
                                 q_sh, q_sd, k_sb, k_sh, k_sl, v_sb, v_sh, v_sl,
                                 sm_scale, dtype, stream);
    if (st != MI_OK) return st;
    return mi_decode_combine(part_m, part_l, part_acc, out, lse, batch, n_heads,
                             head_dim, num_splits, o_sb, o_sh, o_sd,
                             empty_rows_nan, dtype, stream);
  }
  int32_t st = check_common(q, k, v, batch, n_heads, n_kv_heads, kv_len,
                            head_dim, 1, k_sl, v_sl, dtype);
  if (st != MI_OK) return st;
  Plan p = make_plan(dtype, batch, n_heads, n_kv_heads, kv_len, head_dim, 1);
  DecodeArgs a = fill_args(q, k, v, mask, mask_sb, mask_sl, seq_lens, batch, n_heads,
                           n_kv_heads, kv_len, 1, q_sb, q_sh, q_sd, k_sb, k_sh,
                           k_sl, v_sb, v_sh, v_sl, sm_scale, p, elem_bytes(dtype));
  a.out = out;
  a.lse = lse;
  a.o_sb = o_sb; a.o_sh = o_sh; a.o_sd = o_sd;
  a.direct = 1;
  a.empty_nan = empty_rows_nan;
  hipError_t e = launch_split_any(dtype, a, p, batch, n_kv_heads, head_dim,
                                  (hipStream_t)stream);
  if (e != hipSuccess) {
    set_last_error("flash_decode: launch failed: %s", hipGetErrorString(e));
    return (int32_t)e;
  }
  return MI_OK;
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
  if (num_splits == 1)  // single pass: no partials at all
    return mi_flash_decode(q, k, v, mask, mask_sb, mask_sl, seq_lens, nullptr, nullptr,
                           nullptr, out, lse, batch, n_heads, n_kv_heads, kv_len, head_dim,
                           1, q_sb, q_sh, q_sd, k_sb, k_sh, k_sl, v_sb, v_sh, v_sl, o_sb,
                           o_sh, o_sd, sm_scale, empty_rows_nan, dtype, stream);
  // fewer splits than fill the GPU are subdivided, as flash_decode does
  num_splits = mi_decode_effective_splits(batch, n_heads, n_kv_heads, kv_len, head_dim,
                                          num_splits);
  // layout in scratch: acc [B*Hq*S*D] fp32, then m and l [B*Hq*S] fp32 each,
  // every array starting on a 256-byte boundary
  const int64_t rows = batch * n_heads * num_splits;
  auto up = [](int64_t b) { return (b + 255) & ~(int64_t)255; };
  const int64_t acc_bytes = up(rows * head_dim * 4), ml_bytes = up(rows * 4);
  if (head_dim > 1024 || rows > (int64_t)MI_DECODE_NOALLOC_SCRATCH_BYTES ||
      acc_bytes + 2 * ml_bytes > (int64_t)MI_DECODE_NOALLOC_SCRATCH_BYTES) {
    set_last_error("flash_decode_noalloc: partials of batch*n_heads*num_splits = %lld rows x "
                   "(head_dim %lld + 2) fp32 exceed the %lld-byte scratch; use fewer splits "
                   "or mi_flash_decode with a workspace",
                   (long long)rows, (long long)head_dim,
                   (long long)MI_DECODE_NOALLOC_SCRATCH_BYTES);
    return MI_ERR_UNSUPPORTED;
  }
  unsigned char* base = nullptr;
  int32_t st = scratch_base(&base);
  if (st != MI_OK) return st;
  float* part_acc = reinterpret_cast<float*>(base);
  float* part_m = reinterpret_cast<float*>(base + acc_bytes);
  float* part_l = reinterpret_cast<float*>(base + acc_bytes + ml_bytes);
  return mi_flash_decode(q, k, v, mask, mask_sb, mask_sl, seq_lens, part_m, part_l, part_acc,
                         out, lse, batch, n_heads, n_kv_heads, kv_len, head_dim, num_splits,
                         q_sb, q_sh, q_sd, k_sb, k_sh, k_sl, v_sb, v_sh, v_sl, o_sb, o_sh,
                         o_sd, sm_scale, empty_rows_nan, dtype, stream);
}
