// Causal GQA flash-attention prefill on bf16/fp16 MFMA (gfx950).
//
// Math: out[b,h,i] = softmax_j<=i(q_i.k_j / sqrt(D)) . V, query head h reading
// kv head h // G, keys bounded by the query length S
// (src/flash_attn.py:42-83, :85-111), plus lse[b,h,i] = logsumexp_j of the
// scaled scores (natural log), an output this build adds.
//
// Design (MI355X-first, not a translation of the Triton tile loop):
//  * A workgroup owns one (batch, kv-head, block of query positions) and runs
//    one wave per (query head of the GQA group, 32-row slice).  Every K/V tile
//    is staged in LDS once and consumed by all query heads that share it.
//  * Scores are computed transposed, S^T = K Q^T, with
//    v_mfma_f32_32x32x16_{bf16,f16}: the accumulator layout then gives each
//    lane all scores of ONE query row (16 per 32-key block), so the row max
//    and row sum are in-lane plus a single permlane32 swap.
//  * The K rows feeding the MFMA are permuted (bits 2 and 3 of the row index
//    swapped) so that the bf16-converted P^T accumulator is directly the B
//    operand of O^T = V^T P^T: no register shuffles between the two products.
//  * V is written to LDS transposed (V^T, key-contiguous) so each lane reads
//    its A operand with one 16-byte ds_read; K and V^T rows use XOR swizzles
//    of the 16-byte chunk index to spread LDS banks.
//  * Online softmax in fp32 registers in the log2 domain (v_exp_f32), scale
//    folded into one FMA per score; the row sum is taken over fp32 P and P is
//    rounded to the input dtype only for the PV product (as the reference does,
//    src/flash_attn.py:63,72).
//  * Double-buffered LDS tiles with the next tile's global loads in flight
//    during the current tile's MFMAs; one barrier per tile.
//  * Blocks are ordered heaviest-first (longest causal prefix) and mapped so
//    that all blocks of one (batch, kv-head) land on the same XCD, whose L2
//    then serves the K/V re-reads.
#include <math.h>

#include "common.hpp"

namespace mi {

struct PrefillArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int32_t B, Hq, Hkv, S, G;
  int32_t heads_per_block;  // GH: query heads of the group handled per block
  int32_t head_chunks;      // G / GH
  int32_t pj;               // 32-row slices per head per block
  int32_t n_pb;             // position blocks (of 32*pj rows)
  float scale_log2;         // sm_scale * log2(e)
};

template <typename T> struct Mfma;
template <> struct Mfma<bf16_t> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  __device__ static inline f32x16 mma(const v8& a, const v8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static inline uint32_t pack2(float x, float y) {
    typedef __bf16 v2 __attribute__((ext_vector_type(2)));
    v2 r = {(__bf16)x, (__bf16)y};
    return __builtin_bit_cast(uint32_t, r);
  }
};
template <> struct Mfma<f16_t> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  __device__ static inline f32x16 mma(const v8& a, const v8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  __device__ static inline uint32_t pack2(float x, float y) {
    typedef _Float16 v2 __attribute__((ext_vector_type(2)));
    v2 r = {(_Float16)x, (_Float16)y};
    return __builtin_bit_cast(uint32_t, r);
  }
};

// bits 2 and 3 of a row index inside a 32-row MFMA block, swapped
__device__ inline int perm_row(int r) {
  return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1);
}

template <typename T, int D>
struct PrefillGeom {
  static constexpr int kBN = 64;             // keys per tile
  static constexpr int kKCH = D / 8;         // 16-byte chunks per K row
  static constexpr int kDC = D / 16;         // MFMA k-steps over the head dim
  static constexpr int kDB = D / 32;         // 32-row blocks of O^T
  static constexpr int kKTile = kBN * D;     // elements per K tile
  static constexpr int kVTile = D * kBN;     // elements per V^T tile
  static constexpr int kKUnits = kBN * kKCH;         // 16B chunks per K tile
  static constexpr int kVUnits = (kBN / 2) * kKCH;   // (key pair, chunk) units
  static constexpr int kMinThreads = 256;            // blocks are 4 waves
  static constexpr int kKPer = (kKUnits + kMinThreads - 1) / kMinThreads;
  static constexpr int kVPer = (kVUnits + kMinThreads - 1) / kMinThreads;
  static constexpr size_t kSmem = 2 * (size_t)(kKTile + kVTile) * sizeof(T);
};

// physical 16-byte chunk of logical chunk c in K row r / V^T row d
template <int D>
__device__ inline int k_swz(int r, int c) {
  if constexpr (D == 64) return c ^ ((r >> 1) & 7);
  else return c ^ (r & 15);
}
__device__ inline int vt_swz(int d, int kc) { return kc ^ ((d >> 1) & 7); }

template <typename T, int D>
__global__ __launch_bounds__(256, 2) void prefill_kernel(PrefillArgs a) {
  using Geo = PrefillGeom<T, D>;
  using MM = Mfma<T>;
  typedef typename MM::v8 v8;
  constexpr int BN = Geo::kBN, KCH = Geo::kKCH, DC = Geo::kDC, DB = Geo::kDB;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* k_lds = reinterpret_cast<T*>(smem_raw);            // [2][BN][D]
  T* vt_lds = k_lds + 2 * Geo::kKTile;                  // [2][D][BN]

  const int tid = threadIdx.x, nthr = blockDim.x;
  const int lane = tid & 63, w = tid >> 6;
  const int hh = lane >> 5, lr = lane & 31;

  // ---- block -> (batch, kv head, head chunk, position block), heavy first,
  //      all blocks of one (b, kvh, chunk) on one XCD
  const int n_pairs = a.B * a.Hkv * a.head_chunks;
  const int bid = blockIdx.x;
  int pair, pb_rank;
  if ((n_pairs & 7) == 0) {
    const int xcd = bid & 7, slot = bid >> 3, ppx = n_pairs >> 3;
    pair = xcd * ppx + slot % ppx;
    pb_rank = slot / ppx;
  } else {
    pair = bid % n_pairs;
    pb_rank = bid / n_pairs;
  }
  const int pb = a.n_pb - 1 - pb_rank;
  const int hc = pair % a.head_chunks;
  const int kvh = (pair / a.head_chunks) % a.Hkv;
  const int b = pair / (a.head_chunks * a.Hkv);
  const int GH = a.heads_per_block;
  const int rows_pb = 32 * a.pj;
  const int p0 = pb * rows_pb;

  const int g = w % GH, j = w / GH;
  const int head = kvh * a.G + hc * GH + g;
  const int qpos0 = p0 + 32 * j;          // first query row of this wave
  const int qrow = qpos0 + lr;            // this lane's query row
  const bool wave_active = qpos0 < a.S;

  // ---- Q as the B operand of S^T = K Q^T (lane: row lr, 8 dims per k-step)
  v8 qreg[DC];
  {
    const T* qp = reinterpret_cast<const T*>(a.q) + (int64_t)b * a.q_sb +
                  (int64_t)head * a.q_sh + (int64_t)min(qrow, a.S - 1) * a.q_ss;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      u32x4 raw = load16(qp + 16 * c + 8 * hh);
      if (qrow >= a.S) raw = u32x4{0, 0, 0, 0};
      qreg[c] = __builtin_bit_cast(v8, raw);
    }
  }

  const T* kbase = reinterpret_cast<const T*>(a.k) + (int64_t)b * a.k_sb + (int64_t)kvh * a.k_sh;
  const T* vbase = reinterpret_cast<const T*>(a.v) + (int64_t)b * a.v_sb + (int64_t)kvh * a.v_sh;
  const int last_row = min(p0 + rows_pb, a.S) - 1;
  const int n_tiles = last_row / BN + 1;

  u32x4 kpre[Geo::kKPer];
  u32x4 vpre[Geo::kVPer][2];

  auto fetch = [&](int kt) {
    const int r0 = kt * BN;
#pragma unroll
    for (int i = 0; i < Geo::kKPer; ++i) {
      const int u = tid + i * nthr;
      if (u < Geo::kKUnits) {
        const int r = u / KCH, c = u % KCH;
        const int row = min(r0 + r, a.S - 1);
        kpre[i] = load16(kbase + (int64_t)row * a.k_ss + c * 8);
      }
    }
#pragma unroll
    for (int i = 0; i < Geo::kVPer; ++i) {
      const int u = tid + i * nthr;
      if (u < Geo::kVUnits) {
        const int kp = u / KCH, c = u % KCH;
        const int row0 = min(r0 + 2 * kp, a.S - 1), row1 = min(r0 + 2 * kp + 1, a.S - 1);
        vpre[i][0] = load16(vbase + (int64_t)row0 * a.v_ss + c * 8);
        vpre[i][1] = load16(vbase + (int64_t)row1 * a.v_ss + c * 8);
      }
    }
  };
  auto stash = [&](int buf) {
    T* kl = k_lds + buf * Geo::kKTile;
    T* vl = vt_lds + buf * Geo::kVTile;
#pragma unroll
    for (int i = 0; i < Geo::kKPer; ++i) {
      const int u = tid + i * nthr;
      if (u < Geo::kKUnits) {
        const int r = u / KCH, c = u % KCH;
        *reinterpret_cast<u32x4*>(kl + r * D + k_swz<D>(r, c) * 8) = kpre[i];
      }
    }
#pragma unroll
    for (int i = 0; i < Geo::kVPer; ++i) {
      const int u = tid + i * nthr;
      if (u < Geo::kVUnits) {
        const int kp = u / KCH, c = u % KCH;
        const uint32_t w0[4] = {vpre[i][0].x, vpre[i][0].y, vpre[i][0].z, vpre[i][0].w};
        const uint32_t w1[4] = {vpre[i][1].x, vpre[i][1].y, vpre[i][1].z, vpre[i][1].w};
        const int kc = kp >> 2, kw = kp & 3;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
          const int d = 8 * c + jj;
          const uint32_t sel = (jj & 1) ? 0x07060302u : 0x05040100u;
          const uint32_t word = __builtin_amdgcn_perm(w1[jj >> 1], w0[jj >> 1], sel);
          uint32_t* dst = reinterpret_cast<uint32_t*>(vl + d * BN + vt_swz(d, kc) * 8) + kw;
          *dst = word;
        }
      }
    }
  };

  f32x16 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[db][i] = 0.f;
  float m = kNegBig, l = 0.f;
  const float sl2 = a.scale_log2;
  const int prow = perm_row(lr);

  fetch(0);
  stash(0);
  __syncthreads();

  for (int kt = 0; kt < n_tiles; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < n_tiles) fetch(kt + 1);

    const int kbase_pos = kt * BN;
    if (wave_active && kbase_pos <= qpos0 + 31) {
      const T* kl = k_lds + buf * Geo::kKTile;
      const T* vl = vt_lds + buf * Geo::kVTile;
      f32x16 s[2];
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
#pragma unroll
        for (int i = 0; i < 16; ++i) s[sb][i] = 0.f;
        const int r = 32 * sb + prow;
#pragma unroll
        for (int c = 0; c < DC; ++c) {
          const v8 kv = __builtin_bit_cast(
              v8, *reinterpret_cast<const u32x4*>(kl + r * D + k_swz<D>(r, 2 * c + hh) * 8));
          s[sb] = MM::mma(kv, qreg[c], s[sb]);
        }
      }
      // causal mask (keys > query row, which also covers keys >= S)
      if (kbase_pos + BN - 1 > qpos0) {
#pragma unroll
        for (int sb = 0; sb < 2; ++sb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = kbase_pos + 32 * sb + 16 * (i >> 3) + 8 * hh + (i & 7);
            if (key > qrow) s[sb][i] = -INFINITY;
          }
      }
      float mx = s[0][0];
#pragma unroll
      for (int i = 1; i < 16; ++i) mx = fmaxf(mx, s[0][i]);
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[1][i]);
      {
        auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
        mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
      }
      const float m_new = fmaxf(m, mx * sl2);
      const float alpha = fast_exp2(m - m_new);
      m = m_new;
      v8 pb[2][2];
      float ls = 0.f;
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
          uint32_t wds[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const float p0v = fast_exp2(fmaf(s[sb][8 * cc + 2 * t], sl2, -m_new));
            const float p1v = fast_exp2(fmaf(s[sb][8 * cc + 2 * t + 1], sl2, -m_new));
            wds[t] = MM::pack2(p0v, p1v);
            ls += p0v + p1v;
          }
          pb[sb][cc] = __builtin_bit_cast(v8, u32x4{wds[0], wds[1], wds[2], wds[3]});
        }
      l = l * alpha + ls;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
          const int kc = 4 * sb + 2 * cc + hh;  // 8-key chunk of this lane's keys
#pragma unroll
          for (int db = 0; db < DB; ++db) {
            const int d = 32 * db + lr;
            const v8 vv = __builtin_bit_cast(
                v8, *reinterpret_cast<const u32x4*>(vl + d * BN + vt_swz(d, kc) * 8));
            o[db] = MM::mma(vv, pb[sb][cc], o[db]);
          }
        }
    }

    if (kt + 1 < n_tiles) stash(buf ^ 1);
    __syncthreads();
  }

  if (!wave_active) return;
  // both lane halves hold partial sums of the same row
  {
    auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l), __float_as_uint(l), false, false);
    l = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  if (qrow >= a.S) return;
  const float inv = 1.0f / l;
  T* op = reinterpret_cast<T*>(a.o) + (int64_t)b * a.o_sb + (int64_t)head * a.o_sh +
          (int64_t)qrow * a.o_ss;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d = 32 * db + 8 * q4 + 4 * hh;
      const uint32_t w0 = MM::pack2(o[db][4 * q4] * inv, o[db][4 * q4 + 1] * inv);
      const uint32_t w1 = MM::pack2(o[db][4 * q4 + 2] * inv, o[db][4 * q4 + 3] * inv);
      typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
      *reinterpret_cast<u32x2*>(op + d) = u32x2{w0, w1};
    }
  if (a.lse != nullptr && hh == 0)
    a.lse[((int64_t)b * a.Hq + head) * a.S + qrow] = (m + __log2f(l)) * kLn2;
}


// fp32 inputs: plain VALU flash attention (no fp32 MFMA tiles), TPR = D/32
// lanes per query row, 32 dims each; K/V tiles of 64 keys staged in LDS and
// read as broadcasts.  Used for fp32 models (e.g. the CPU-shaped parity case).
template <int D>
__global__ __launch_bounds__(256) void prefill_f32_kernel(PrefillArgs a) {
  constexpr int TPR = D / 32, BN = 4096 / D;  // K+V tiles stay at ~33 KB of LDS
  constexpr int ROWS = 256 / TPR;  // query rows per block
  __shared__ float ks[BN][D + 1];
  __shared__ float vs[BN][D + 1];
  const int tid = threadIdx.x;
  const int part = tid % TPR, row_in = tid / TPR;
  const int n_rb = (a.S + ROWS - 1) / ROWS;
  const int rb = n_rb - 1 - (int)(blockIdx.x % n_rb);
  const int bh = (int)(blockIdx.x / n_rb);
  const int head = bh % a.Hq, b = bh / a.Hq;
  const int kvh = head / a.G;
  const int qrow = rb * ROWS + row_in;
  const int qr = min(qrow, a.S - 1);
  const float* qp = reinterpret_cast<const float*>(a.q) + (int64_t)b * a.q_sb +
                    (int64_t)head * a.q_sh + (int64_t)qr * a.q_ss + part * 32;
  float qv[32], acc[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) { qv[i] = qp[i]; acc[i] = 0.f; }
  float m = kNegBig, l = 0.f;
  const float* kb = reinterpret_cast<const float*>(a.k) + (int64_t)b * a.k_sb + (int64_t)kvh * a.k_sh;
  const float* vb = reinterpret_cast<const float*>(a.v) + (int64_t)b * a.v_sb + (int64_t)kvh * a.v_sh;
  const int last = min(rb * ROWS + ROWS, a.S) - 1;
  for (int k0 = 0; k0 <= last; k0 += BN) {
    __syncthreads();
    for (int e = tid; e < BN * D; e += 256) {
      const int r = e / D, d = e % D;
      const int row = min(k0 + r, a.S - 1);
      ks[r][d] = kb[(int64_t)row * a.k_ss + d];
      vs[r][d] = vb[(int64_t)row * a.v_ss + d];
    }
    __syncthreads();
    const int nk = min(BN, qrow - k0 + 1);  // keys k0..qrow are visible
    for (int jj = 0; jj < nk; ++jj) {
      float sdot = 0.f;
#pragma unroll
      for (int i = 0; i < 32; ++i) sdot = fmaf(qv[i], ks[jj][part * 32 + i], sdot);
      sdot = group_sum<TPR>(sdot) * a.scale_log2;
      const float mn = fmaxf(m, sdot);
      const float alpha = fast_exp2(m - mn), p = fast_exp2(sdot - mn);
      l = l * alpha + p;
#pragma unroll
      for (int i = 0; i < 32; ++i) acc[i] = fmaf(p, vs[jj][part * 32 + i], acc[i] * alpha);
      m = mn;
    }
  }
  if (qrow >= a.S) return;
  float* op = reinterpret_cast<float*>(a.o) + (int64_t)b * a.o_sb + (int64_t)head * a.o_sh +
              (int64_t)qrow * a.o_ss + part * 32;
  const float inv = 1.0f / l;
#pragma unroll
  for (int i = 0; i < 32; ++i) op[i] = acc[i] * inv;
  if (a.lse != nullptr && part == 0)
    a.lse[((int64_t)b * a.Hq + head) * a.S + qrow] = (m + __log2f(l)) * kLn2;
}

namespace {

template <typename T, int D>
hipError_t launch(const PrefillArgs& a, int nwaves, hipStream_t stream) {
  using Geo = PrefillGeom<T, D>;
  const int n_pairs = a.B * a.Hkv * a.head_chunks;
  dim3 grid((unsigned)(n_pairs * a.n_pb));
  dim3 block((unsigned)(nwaves * 64));
  hipLaunchKernelGGL((prefill_kernel<T, D>), grid, block, Geo::kSmem, stream, a);
  return hipGetLastError();
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int32_t mi_attn_prefill(const void* q, const void* k, const void* v,
                                   void* o, float* lse, int64_t batch,
                                   int64_t n_heads, int64_t n_kv_heads,
                                   int64_t seq_len, int64_t kv_len,
                                   int64_t head_dim, int64_t q_sb, int64_t q_sh,
                                   int64_t q_ss, int64_t k_sb, int64_t k_sh,
                                   int64_t k_ss, int64_t v_sb, int64_t v_sh,
                                   int64_t v_ss, int64_t o_sb, int64_t o_sh,
                                   int64_t o_ss, float sm_scale, int32_t dtype,
                                   void* stream) {
  if (q == nullptr || k == nullptr || v == nullptr || o == nullptr) {
    set_last_error("attn_prefill: null pointer");
    return MI_ERR_INVALID;
  }
  if (batch <= 0 || n_heads <= 0 || n_kv_heads <= 0 || seq_len <= 0) {
    set_last_error("attn_prefill: sizes must be positive");
    return MI_ERR_INVALID;
  }
  if (n_heads % n_kv_heads != 0) {
    set_last_error("attn_prefill: query heads (%lld) must be divisible by KV heads (%lld)",
                   (long long)n_heads, (long long)n_kv_heads);
    return MI_ERR_INVALID;
  }
  if (kv_len < seq_len) {
    set_last_error("attn_prefill: kv_len (%lld) must be >= seq_len (%lld)",
                   (long long)kv_len, (long long)seq_len);
    return MI_ERR_INVALID;
  }
  if (dtype != MI_DTYPE_BF16 && dtype != MI_DTYPE_F16 && dtype != MI_DTYPE_F32) {
    set_last_error("attn_prefill: unknown dtype code %d", (int)dtype);
    return MI_ERR_INVALID;
  }
  if (head_dim != 64 && head_dim != 128) {
    set_last_error("attn_prefill: head_dim %lld has no kernel (supported: 64, 128)",
                   (long long)head_dim);
    return MI_ERR_UNSUPPORTED;
  }
  const int64_t eb = dtype == MI_DTYPE_F32 ? 4 : 2;
  const uintptr_t pq = (uintptr_t)q, pk = (uintptr_t)k, pv = (uintptr_t)v, po = (uintptr_t)o;
  if ((pq | pk | pv) % 16 != 0 || po % 8 != 0 ||
      ((q_sb | q_sh | q_ss | k_sb | k_sh | k_ss | v_sb | v_sh | v_ss) * eb) % 16 != 0 ||
      ((o_sb | o_sh | o_ss) * eb) % 8 != 0) {
    set_last_error("attn_prefill: rows must be 16-byte aligned with unit head-dim stride");
    return MI_ERR_INVALID;
  }
  if (seq_len > (1 << 30) || batch * n_kv_heads * n_heads > (1 << 30)) {
    set_last_error("attn_prefill: shape exceeds launch limits");
    return MI_ERR_UNSUPPORTED;
  }
  const int G = (int)(n_heads / n_kv_heads);
  // 4 waves per block: 4 query heads x 32 rows, 2 heads x 64 rows or
  // 1 head x 128 rows, whichever divides the GQA group size.
  const int gh = (G % 4 == 0) ? 4 : (G % 2 == 0) ? 2 : 1;
  const int pj = 4 / gh;
  PrefillArgs a{};
  a.q = q; a.k = k; a.v = v; a.o = o; a.lse = lse;
  a.q_sb = q_sb; a.q_sh = q_sh; a.q_ss = q_ss;
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_ss = k_ss;
  a.v_sb = v_sb; a.v_sh = v_sh; a.v_ss = v_ss;
  a.o_sb = o_sb; a.o_sh = o_sh; a.o_ss = o_ss;
  a.B = (int32_t)batch; a.Hq = (int32_t)n_heads; a.Hkv = (int32_t)n_kv_heads;
  a.S = (int32_t)seq_len; a.G = G;
  a.heads_per_block = gh;
  a.head_chunks = G / gh;
  a.pj = pj;
  a.n_pb = (int32_t)((seq_len + 32 * pj - 1) / (32 * pj));
  a.scale_log2 = sm_scale * kLog2e;
  const int nwaves = gh * pj;
  const int64_t blocks = (int64_t)a.B * a.Hkv * a.head_chunks * a.n_pb;
  if (blocks > INT32_MAX) {
    set_last_error("attn_prefill: grid too large");
    return MI_ERR_UNSUPPORTED;
  }
  hipError_t e;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == MI_DTYPE_F32) {
    const int rows = 256 / (int)(head_dim / 32);
    const int64_t nblk = (int64_t)a.B * a.Hq * ((a.S + rows - 1) / rows);
    if (head_dim == 64)
      hipLaunchKernelGGL(prefill_f32_kernel<64>, dim3((unsigned)nblk), dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL(prefill_f32_kernel<128>, dim3((unsigned)nblk), dim3(256), 0, st, a);
    e = hipGetLastError();
  } else if (dtype == MI_DTYPE_BF16)
    e = head_dim == 64 ? launch<bf16_t, 64>(a, nwaves, st) : launch<bf16_t, 128>(a, nwaves, st);
  else
    e = head_dim == 64 ? launch<f16_t, 64>(a, nwaves, st) : launch<f16_t, 128>(a, nwaves, st);
  if (e != hipSuccess) {
    set_last_error("attn_prefill: launch failed: %s", hipGetErrorString(e));
    return (int32_t)e;
  }
  return MI_OK;
}
