// Causal GQA flash-attention prefill on bf16/fp16 MFMA (gfx950).
//
// Math: out[b,h,i] = softmax_j<=i(q_i.k_j / sqrt(D)) . V, query head h reading
// kv head h // G, keys bounded by the query length S
// (src/flash_attn.py:42-83, :85-111), plus lse[b,h,i] = logsumexp_j of the
// scaled scores (natural log), an output this build adds.
//
// Design (MI355X-first, not a translation of the Triton tile loop):
//  * A workgroup owns one (batch, kv-head, block of query positions) and runs
//    one wave per (query head of the GQA group, row slice).  Every K/V tile is
//    copied into LDS once (global->LDS DMA, no register round trip) and read
//    by all query heads that share it; each wave uses every K/V operand it
//    reads from LDS for two 32-row MFMA blocks.
//  * Scores are computed transposed, S^T = K Q^T, with
//    v_mfma_f32_32x32x16_{bf16,f16}: the accumulator layout then gives each
//    lane all scores of ONE query row (16 per 32-key block), so the row max
//    and row sum are in-lane plus a single permlane32 swap.
//  * The K rows feeding the MFMA are permuted (bits 2 and 3 of the row index
//    swapped) so that the bf16-converted P^T accumulator is directly the B
//    operand of O^T = V^T P^T: no register shuffles between the two products.
//  * V stays key-major in LDS; the V^T operand is read with the transposing
//    ds_read_b64_tr_b16.  K and V rows use XOR swizzles of the 16-byte chunk
//    index to spread LDS banks.
//  * Online softmax in fp32 registers in the log2 domain (v_exp_f32), scale
//    folded into one FMA per score; the row sum is taken over fp32 P and P is
//    rounded to the input dtype only for the PV product (as the reference does,
//    src/flash_attn.py:63,72).
//  * head_dim 64: a software-pipelined kernel (each wave overlaps its own
//    MFMAs with its softmax, 4-slot LDS ring, one barrier per tile);
//    head_dim 128: the same schedule with separate K and V double buffers and
//    bank-conflict-free V reads; head_dim 32 / 256: double-buffered tiles,
//    one barrier per tile.
//  * The prologue issues the first tile copies before the Q loads (one memory
//    round trip for both); the epilogue stages the output rows in the freed
//    LDS and writes whole 2*D-byte rows with 16-byte lanes.
//  * Blocks are ordered heaviest-first (longest causal prefix) and mapped so
//    that all blocks of one (batch, kv-head) land on the same XCD, whose L2
//    then serves the K/V re-reads.
#include <math.h>

#include <type_traits>

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
  // Optional RoPE of q in the Q prologue (rcos == nullptr: q is used as
  // given).  Rotate-half with the table row rpos[s] (or s when rpos is null)
  // of cos/sin [rows, D/2] in q's dtype, unit column stride, row stride r_ss.
  const void* rcos;
  const void* rsin;
  const int64_t* rpos;
  int64_t r_ss, r_rows;     // positions are clamped into the table's rows
  int32_t o_line;           // out and its rows are 16-byte aligned (whole-row epilogue)
};

// RoPE of the Q fragments a lane holds for one 32-row block: chunk c (dims
// 16c + 8hh .. +7) pairs with chunk c + DC/2 (the same dims + D/2), so every
// rotation pair is in the lane's own registers.  qrow is the lane's query row
// (clamped into [0, S)); the rounding is that of the RoPE kernels.
template <typename T, int DC, typename V8>
__device__ inline void rope_q_fragments(const PrefillArgs& a, int qrow, int hh, V8 (&qf)[DC]) {
  int64_t crow = qrow;
  if (a.rpos != nullptr) crow = min(max(a.rpos[qrow], (int64_t)0), a.r_rows - 1);
  const T* cp = reinterpret_cast<const T*>(a.rcos) + crow * a.r_ss;
  const T* sp = reinterpret_cast<const T*>(a.rsin) + crow * a.r_ss;
#pragma unroll
  for (int c = 0; c < DC / 2; ++c) {
    const int i0 = 16 * c + 8 * hh;
    const V8 cv = __builtin_bit_cast(V8, load16(cp + i0));
    const V8 sv = __builtin_bit_cast(V8, load16(sp + i0));
    V8 lo = qf[c], hi = qf[c + DC / 2];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      T y1, y2;
      rope_rotate<T, T>(Elem<T>::to_f32(lo[e]), Elem<T>::to_f32(hi[e]), cv[e], sv[e], y1, y2);
      lo[e] = y1;
      hi[e] = y2;
    }
    qf[c] = lo;
    qf[c + DC / 2] = hi;
  }
}

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


// LDS tile layouts (one buffer): K [BN][D] and V [BN][D], both row-major in
// 16-byte chunks with the chunk index XOR-swizzled per row.  Tiles are filled
// by global->LDS DMA (global_load_lds_dwordx4): a wave instruction writes 1 KB
// contiguously, lane t at +16t, so the swizzle is realised by choosing which
// logical chunk each lane fetches.
template <int D>
__device__ inline int k_swz(int r) {  // XOR mask for K row r (< the row's chunk count)
  if constexpr (D == 32) return (r >> 1) & 3;
  else if constexpr (D == 64) return (r >> 1) & 7;
  else return r & 15;
}
__device__ inline int v_swz(int r) { return (r >> 1) & 3; }  // XOR mask for V row r

// Online-softmax rescale threshold (log2 units): the running row max used for
// exp2 is only moved when a new score exceeds it by more than this, so
// probabilities stay <= 2^8 (exact maths is unchanged: O and l share the same
// reference max) and O is rescaled on rare tiles instead of on every tile.
constexpr float kRescaleThreshold = 8.0f;
// Row-sum bound of the max-free softmax half (16 scores per lane): 16 * 2^8.
constexpr float kFastSumLimit = 4096.0f;

typedef short s16x4 __attribute__((ext_vector_type(4)));


// Transposed 64-bit LDS read: within each 16-lane group, lane i receives
// element (i % 4) of the 8-byte chunks addressed by lanes 4e + i/4, e = 0..3.
__device__ inline uint2 lds_read_tr(const unsigned char* p) {
  s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(p));
  return __builtin_bit_cast(uint2, r);
}

// Each wave owns RB blocks of 32 query rows (RB = 2 at D = 64):
// every K / V operand read from LDS feeds two MFMAs, and the two row blocks are
// independent instruction streams the scheduler interleaves (the softmax VALU
// of one block runs while the other's MFMAs execute).
template <int D>
constexpr int prefill_row_blocks() { return D == 64 ? 2 : 1; }  // D=128: registers
// Blocks per CU the registers are sized for: at D = 256 one block (a wave then
// holds its 32 x 256 fp32 O tile and the tile's K operands in 512 registers)
// and its double-buffered K/V tiles take 128 KB of LDS.
template <int D>
constexpr int prefill_min_blocks() { return D >= 256 ? 1 : 2; }

template <typename T, int D>
__global__ __launch_bounds__(256, prefill_min_blocks<D>()) void prefill_kernel(PrefillArgs a) {
  using MM = Mfma<T>;
  typedef typename MM::v8 v8;
  constexpr int BN = 64, KCH = D / 8, DC = D / 16, DB = D / 32, RB = prefill_row_blocks<D>();
  constexpr bool kEarlyV = D == 64;
  constexpr int ROW_B = D * 2;                  // bytes per K/V row
  constexpr int TILE_B = BN * ROW_B;            // bytes per K or V tile
  constexpr int NI = TILE_B / 1024 / 4;         // DMA instructions per wave per tile
  static_assert(NI * 4 * 1024 == TILE_B, "tile must split into 1 KB wave copies");
  extern __shared__ __align__(16) unsigned char smem_raw[];
  unsigned char* const lds = smem_raw;          // [2][K tile | V tile]

  const int tid = threadIdx.x;
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
  const int rows_pb = 32 * RB * a.pj;
  const int p0 = pb * rows_pb;

  const int g = w % GH, j = w / GH;
  const int head = kvh * a.G + hc * GH + g;
  const int qpos0 = p0 + 32 * RB * j;     // first query row of this wave
  const bool wave_active = qpos0 < a.S;

  // ---- Q as the B operand of S^T = K Q^T (lane: row lr of each row block),
  //      loaded in the prologue after the first tile copy is issued
  v8 qreg[RB][DC];

  // ---- DMA geometry: wave w copies 1 KB pieces (w*NI + i) of each tile
  const unsigned char* kbase = reinterpret_cast<const unsigned char*>(a.k) +
                               ((int64_t)b * a.k_sb + (int64_t)kvh * a.k_sh) * 2;
  const unsigned char* vbase = reinterpret_cast<const unsigned char*>(a.v) +
                               ((int64_t)b * a.v_sb + (int64_t)kvh * a.v_sh) * 2;
  int dma_row[NI];
  uint32_t k_goff[NI], v_goff[NI];
  int k_lc[NI], v_lc[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int idx = (w * NI + i) * 64 + lane;   // physical chunk index in the tile
    const int r = idx / KCH, pc = idx % KCH;
    dma_row[i] = r;
    k_lc[i] = pc ^ k_swz<D>(r);                 // logical chunk this lane fetches
    v_lc[i] = pc ^ v_swz(r);
    k_goff[i] = (uint32_t)(r * a.k_ss + k_lc[i] * 8) * 2u;
    v_goff[i] = (uint32_t)(r * a.v_ss + v_lc[i] * 8) * 2u;
  }
  const uint32_t lds0 = lds_addr(lds) + w * NI * 1024;
  auto issue = [&](int kt, int buf) {
    const int r0 = kt * BN;
    const uint32_t kl = lds0 + buf * (2 * TILE_B), vl = kl + TILE_B;
    const unsigned char* kt_base = kbase + (int64_t)r0 * a.k_ss * 2;
    const unsigned char* vt_base = vbase + (int64_t)r0 * a.v_ss * 2;
    if (r0 + BN <= a.S) {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        lds_dma16(kt_base, k_goff[i], kl + i * 1024);
        lds_dma16(vt_base, v_goff[i], vl + i * 1024);
      }
    } else {  // last, partial tile: rows clamped to S-1 (masked out later)
      const int lim = a.S - 1 - r0;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int r = min(dma_row[i], lim);
        lds_dma16(kt_base, (uint32_t)(r * a.k_ss + k_lc[i] * 8) * 2u, kl + i * 1024);
        lds_dma16(vt_base, (uint32_t)(r * a.v_ss + v_lc[i] * 8) * 2u, vl + i * 1024);
      }
    }
  };

  // ---- per-lane operand read offsets (bytes, within one buffer)
  const int prow = perm_row(lr);
  int k_rd[DC];
#pragma unroll
  for (int c = 0; c < DC; ++c) k_rd[c] = prow * ROW_B + (((2 * c + hh) ^ k_swz<D>(prow)) * 16);
  const int gq = lane >> 4, sl = lane & 15;
  int v_rd[8];
#pragma unroll
  for (int q8 = 0; q8 < 8; ++q8) {  // q8 = 4*sb + 2*cc + half
    const int sb = q8 >> 2, cc = (q8 >> 1) & 1, half = q8 & 1;
    const int r = 32 * sb + 16 * cc + 8 * (gq >> 1) + 4 * half + (sl >> 2);
    const int d0 = 16 * (gq & 1) + 4 * (sl & 3);  // db = 0; db adds 32 dims = 4 chunks
    v_rd[q8] = r * ROW_B + (((d0 >> 3) ^ v_swz(r)) * 16) + (d0 & 7) * 2;
  }

  const int last_row = min(p0 + rows_pb, a.S) - 1;
  const int n_tiles = last_row / BN + 1;

  f32x16 o[RB][DB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[rb][db][i] = 0.f;
  float m[RB], l[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) { m[rb] = kNegBig; l[rb] = 0.f; }
  const float sl2 = a.scale_log2;

  // prologue: tile 0 in flight, then Q (and its RoPE table rows), so both
  // share one memory round trip (loads complete in issue order, and the
  // compiler's wait for Q covers the copy).  Rows past S read row S - 1:
  // finite scores in rows whose output is never stored.
  issue(0, 0);
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int qrow = min(qpos0 + 32 * rb + lr, a.S - 1);
    const T* qp = reinterpret_cast<const T*>(a.q) + (int64_t)b * a.q_sb +
                  (int64_t)head * a.q_sh + (int64_t)qrow * a.q_ss;
#pragma unroll
    for (int c = 0; c < DC; ++c) qreg[rb][c] = __builtin_bit_cast(v8, load16(qp + 16 * c + 8 * hh));
    if (a.rcos != nullptr) rope_q_fragments<T, DC>(a, qrow, hh, qreg[rb]);
  }
  dma_wait_all();
  __syncthreads();

  auto tile = [&](int kt, auto buf_c) {
    constexpr int buf = decltype(buf_c)::value;
    if (kt + 1 < n_tiles) issue(kt + 1, buf ^ 1);
    const int kpos = kt * BN;
    if (wave_active && kpos <= qpos0 + 32 * RB - 1) {
      const unsigned char* kl = lds + buf * (2 * TILE_B);
      const unsigned char* vl = kl + TILE_B;
      // S^T for both row blocks: each K operand read feeds two MFMAs
      f32x16 s[RB][2];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int sb = 0; sb < 2; ++sb)
#pragma unroll
          for (int i = 0; i < 16; ++i) s[rb][sb][i] = 0.f;
      // all K operands of the tile are read before the first MFMA so the LDS
      // latency is paid once per tile, not once per k-step (at D = 256 one
      // 32-key half at a time: the registers are not there for both)
      constexpr int KH = D >= 256 ? 1 : 2;   // halves whose K operands are live at once
#pragma unroll
      for (int s0 = 0; s0 < 2; s0 += KH) {
        v8 ka[KH][DC];
#pragma unroll
        for (int sh = 0; sh < KH; ++sh)
#pragma unroll
          for (int c = 0; c < DC; ++c)
            ka[sh][c] = __builtin_bit_cast(
                v8, *reinterpret_cast<const u32x4*>(kl + k_rd[c] + (s0 + sh) * 32 * ROW_B));
#pragma unroll
        for (int sh = 0; sh < KH; ++sh)
#pragma unroll
          for (int c = 0; c < DC; ++c)
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
              s[rb][s0 + sh] = MM::mma(ka[sh][c], qreg[rb][c], s[rb][s0 + sh]);
      }
      // V^T operands of the PV product.  At D = 64 they are read here, so
      // their latency hides under the softmax; at D = 128 the registers are
      // not there and they are read next to their MFMAs.
      v8 vv[4][DB];
      auto read_v = [&](int q4, int db) {
        const uint2 lo = lds_read_tr(vl + v_rd[2 * q4] + db * 64);
        const uint2 hi = lds_read_tr(vl + v_rd[2 * q4 + 1] + db * 64);
        vv[q4][db] = __builtin_bit_cast(v8, u32x4{lo.x, lo.y, hi.x, hi.y});
      };
      if constexpr (kEarlyV) {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
#pragma unroll
          for (int db = 0; db < DB; ++db) read_v(q4, db);
        // schedule: the K reads first, then the QK MFMAs with the V reads
        // interleaved between them
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * DC, 0);
#pragma unroll
        for (int i = 0; i < 2 * DC * RB; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
      } else {
        // schedule: one 32-key half of K at a time
#pragma unroll
        for (int sb = 0; sb < 2; ++sb) {
          __builtin_amdgcn_sched_group_barrier(0x100, DC, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, DC * RB, 0);
        }
      }
      v8 pb[RB][4];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const int r0 = qpos0 + 32 * rb;
        if (kpos + BN - 1 > r0) {  // diagonal tile for this row block
          const int rel = r0 + lr - kpos - 8 * hh;  // visible iff key offset <= rel
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int kk = 16 * (i >> 3) + (i & 7);
            if (kk > rel) s[rb][0][i] = -INFINITY;
            if (kk + 32 > rel) s[rb][1][i] = -INFINITY;
          }
        }
        float mx = fmaxf(s[rb][0][0], s[rb][0][1]);
#pragma unroll
        for (int i = 2; i < 16; i += 2) mx = fmaxf(mx, fmaxf(s[rb][0][i], s[rb][0][i + 1]));
#pragma unroll
        for (int i = 0; i < 16; i += 2) mx = fmaxf(mx, fmaxf(s[rb][1][i], s[rb][1][i + 1]));
        {
          auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
          mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * sl2;
        }
        if (__builtin_amdgcn_ballot_w64(mx > m[rb] + kRescaleThreshold) != 0) {
          const float m_new = fmaxf(m[rb], mx);
          const float alpha = fast_exp2(m[rb] - m_new);
          m[rb] = m_new;
          l[rb] *= alpha;
#pragma unroll
          for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[rb][db][i] *= alpha;
        }
        const float mr = m[rb];
        float ls0 = 0.f, ls1 = 0.f;
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
          uint32_t w0[4], w1[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const float a0 = fast_exp2(fmaf(s[rb][0][8 * cc + 2 * t], sl2, -mr));
            const float a1 = fast_exp2(fmaf(s[rb][0][8 * cc + 2 * t + 1], sl2, -mr));
            const float b0 = fast_exp2(fmaf(s[rb][1][8 * cc + 2 * t], sl2, -mr));
            const float b1 = fast_exp2(fmaf(s[rb][1][8 * cc + 2 * t + 1], sl2, -mr));
            ls0 += a0 + a1;
            ls1 += b0 + b1;
            w0[t] = MM::pack2(a0, a1);
            w1[t] = MM::pack2(b0, b1);
          }
          pb[rb][cc] = __builtin_bit_cast(v8, u32x4{w0[0], w0[1], w0[2], w0[3]});
          pb[rb][2 + cc] = __builtin_bit_cast(v8, u32x4{w1[0], w1[1], w1[2], w1[3]});
        }
        l[rb] += ls0 + ls1;
      }
      // O^T += V^T P^T: each V operand read feeds both row blocks
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4)
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          if constexpr (!kEarlyV) read_v(q4, db);
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) o[rb][db] = MM::mma(vv[q4][db], pb[rb][q4], o[rb][db]);
        }
    }
    dma_wait_all();
    __syncthreads();
  };
  for (int kt = 0; kt < n_tiles; kt += 2) {
    tile(kt, std::integral_constant<int, 0>{});
    if (kt + 1 < n_tiles) tile(kt + 1, std::integral_constant<int, 1>{});
  }

  if (!wave_active) return;
  if (a.o_line) {
    // Whole-row stores: every wave has passed the last tile's barrier, so the
    // tile buffers are free; each wave stages its 32 rows at a time there and
    // writes a row's 2*D bytes with D/8 lanes x 16 bytes of one instruction.
    constexpr int RS = 2 * D + 8;            // staged row stride (bytes, padded)
    constexpr int LPRO = D / 8, RPI = 64 / LPRO;
    static_assert(4 * 32 * RS <= 2 * 2 * 64 * D * (int)sizeof(T), "staging fits the tile buffers");
    unsigned char* const stg = lds + w * 32 * RS;
    T* const ob = reinterpret_cast<T*>(a.o) + (int64_t)b * a.o_sb + (int64_t)head * a.o_sh;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      float lt = l[rb];
      {  // both lane halves hold partial sums of the same row
        auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(lt), __float_as_uint(lt), false, false);
        lt = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
      }
      const float inv = 1.0f / lt;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const int d = 32 * db + 8 * q4 + 4 * hh;
          const uint32_t w0 = MM::pack2(o[rb][db][4 * q4] * inv, o[rb][db][4 * q4 + 1] * inv);
          const uint32_t w1 = MM::pack2(o[rb][db][4 * q4 + 2] * inv, o[rb][db][4 * q4 + 3] * inv);
          typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
          *reinterpret_cast<u32x2*>(stg + lr * RS + d * 2) = u32x2{w0, w1};
        }
      __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // this wave's rows are staged
#pragma unroll
      for (int i = 0; i < 32 / RPI; ++i) {
        const int rr = RPI * i + lane / LPRO, cc = lane % LPRO;
        const u32x4 v = *reinterpret_cast<const u32x4*>(stg + rr * RS + cc * 16);
        const int qr = qpos0 + 32 * rb + rr;
        if (qr < a.S) *reinterpret_cast<u32x4*>(ob + (int64_t)qr * a.o_ss + 8 * cc) = v;
      }
      const int qrow = qpos0 + 32 * rb + lr;
      if (a.lse != nullptr && hh == 0 && qrow < a.S)
        a.lse[((int64_t)b * a.Hq + head) * a.S + qrow] = (m[rb] + __log2f(lt)) * kLn2;
    }
    return;
  }
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    float lt = l[rb];
    {  // both lane halves hold partial sums of the same row
      auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(lt), __float_as_uint(lt), false, false);
      lt = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    const int qrow = qpos0 + 32 * rb + lr;
    if (qrow >= a.S) continue;
    const float inv = 1.0f / lt;
    T* op = reinterpret_cast<T*>(a.o) + (int64_t)b * a.o_sb + (int64_t)head * a.o_sh +
            (int64_t)qrow * a.o_ss;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d = 32 * db + 8 * q4 + 4 * hh;
        const uint32_t w0 = MM::pack2(o[rb][db][4 * q4] * inv, o[rb][db][4 * q4 + 1] * inv);
        const uint32_t w1 = MM::pack2(o[rb][db][4 * q4 + 2] * inv, o[rb][db][4 * q4 + 3] * inv);
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        *reinterpret_cast<u32x2*>(op + d) = u32x2{w0, w1};
      }
    if (a.lse != nullptr && hh == 0)
      a.lse[((int64_t)b * a.Hq + head) * a.S + qrow] = (m[rb] + __log2f(lt)) * kLn2;
  }
}


// ---------------------------------------------------------------------------
// Software-pipelined variant (D = 64, 16-bit).  At D = 64 the softmax VALU work
// of a tile (one exp, fma, add per score plus the row max and packing) issues
// for about as long as its MFMAs take to execute, and a wave issues its VALU
// instructions one at a time.  Each wave therefore overlaps its own matrix and
// vector work: keys are processed in 32-key halves, and while the softmax of
// half u runs on the VALU, the same wave has the MFMAs of half u+1 (S^T =
// K Q^T) and half u-1 (O^T += V^T P^T) in flight.  Two 4-wave blocks share a
// CU (two waves per SIMD, not coupled by barriers), so the SIMD can co-issue
// VALU work of one wave while the other's MFMAs execute.
//
//   slot A(t): softmax(t.h0) | PV(t-1.h1), QK(t.h1)
//   ---- wait for tile t+1, barrier, copy tile t+3 into the ring ----
//   slot B(t): softmax(t.h1) | PV(t.h0),   QK(t+1.h0)
//
// Tile t is read in slots B(t-1), A(t), B(t), A(t+1); the 4-slot LDS ring lets
// the copy of tile t+3 start right after A(t), two slots before its first use.
// A wave owns 64 query rows (two 32-row MFMA blocks that share every K and V
// operand read from LDS); every key tile is visible in full except the wave's
// last (diagonal) tile, whose first half masks row block 0 with the causal
// triangle and whose second half is invisible to row block 0 and masks row
// block 1.  The online-softmax rescale is decided once per half for the wave
// (the max is only moved past the threshold, so it is rare) and applied in a
// branch after the half's MFMAs are issued.
constexpr int kSpBufs = 4;

template <typename T>
__global__ __launch_bounds__(256, 2) void prefill_sp_kernel(PrefillArgs a) {
  using MM = Mfma<T>;
  typedef typename MM::v8 v8;
  constexpr int D = 64, BN = 64, KCH = D / 8, DC = D / 16;
  constexpr int ROW_B = D * 2, TILE_B = BN * ROW_B, SLOT_B = 2 * TILE_B;
  constexpr int NI = TILE_B / 1024 / 4;        // 1 KB copies per wave per K (V) tile
  static_assert(NI * 4 * 1024 == TILE_B, "tile must split into 1 KB wave copies");
  extern __shared__ __align__(16) unsigned char smem_raw[];
  unsigned char* const lds = smem_raw;

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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
  const int GH = a.heads_per_block, PJ = a.pj;
  const int p0 = pb * 64 * PJ;
  const int g = w % GH, j = w / GH;
  const int head = kvh * a.G + hc * GH + g;
  const int r0 = p0 + 64 * j;                        // first query row of this wave
  const int n_tw = r0 < a.S ? r0 / BN + 1 : 0;       // tiles this wave reads (last = diagonal)
  const int n_tiles = (min(p0 + 64 * PJ, a.S) - 1) / BN + 1;  // tiles the block copies

  // ---- Q as the B operand of S^T = K Q^T (lane: row lr of each row block),
  //      loaded in the prologue after the first tile copies are issued
  v8 qreg[2][DC];

  // ---- tile copies: wave w copies 1 KB pieces (w*NI + i) of each tile
  const unsigned char* kbase = reinterpret_cast<const unsigned char*>(a.k) +
                               ((int64_t)b * a.k_sb + (int64_t)kvh * a.k_sh) * 2;
  const unsigned char* vbase = reinterpret_cast<const unsigned char*>(a.v) +
                               ((int64_t)b * a.v_sb + (int64_t)kvh * a.v_sh) * 2;
  const uint32_t lds0 = lds_addr(lds) + w * NI * 1024;
  // Copy tile t into ring slot t % kSpBufs.  The lane -> chunk geometry is
  // recomputed here (a few integer ops per tile) rather than kept in registers.
  auto issue = [&](int t) {
    const int r0t = t * BN;
    const uint32_t kl = lds0 + (t % kSpBufs) * SLOT_B, vl = kl + TILE_B;
    const unsigned char* kt_base = kbase + (int64_t)r0t * a.k_ss * 2;
    const unsigned char* vt_base = vbase + (int64_t)r0t * a.v_ss * 2;
    const int lim = a.S - 1 - r0t;   // rows past S are clamped (masked out later)
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int idx = (w * NI + i) * 64 + lane;   // physical chunk index in the tile
      const int r = idx / KCH, pc = idx % KCH;
      const int rr = min(r, lim);
      lds_dma16(kt_base, (uint32_t)(rr * a.k_ss + (pc ^ k_swz<D>(r)) * 8) * 2u, kl + i * 1024);
      lds_dma16(vt_base, (uint32_t)(rr * a.v_ss + (pc ^ v_swz(r)) * 8) * 2u, vl + i * 1024);
    }
  };

  // ---- per-lane operand read offsets (bytes, within one ring slot)
  const int prow = perm_row(lr);
  int k_rd[DC];
#pragma unroll
  for (int c = 0; c < DC; ++c) k_rd[c] = prow * ROW_B + (((2 * c + hh) ^ k_swz<D>(prow)) * 16);
  // V^T operand rows r = 32*half + 16*cc + 8*(gq>>1) + 4*part + (sl>>2): the
  // swizzle (r>>1)&3 depends only on `part` and the lane, so two base offsets
  // plus immediates address every read.
  const int gq = lane >> 4, sl = lane & 15;
  int v_rd[2];
#pragma unroll
  for (int part = 0; part < 2; ++part) {
    const int r = 8 * (gq >> 1) + 4 * part + (sl >> 2);
    const int d0 = 16 * (gq & 1) + 4 * (sl & 3);  // db = 0; db adds 32 dims = 4 chunks
    v_rd[part] = TILE_B + r * ROW_B + (((d0 >> 3) ^ v_swz(r)) * 16) + (d0 & 7) * 2;
  }
  // causal triangle of a diagonal half: score i of this lane is key offset
  // kk(i) within the half, visible iff kk(i) <= tri
  const int tri = lr - 8 * hh;

  f32x16 o[2][2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[rb][db][i] = 0.f;
  float m[2] = {kNegBig, kNegBig}, l[2] = {0.f, 0.f};
  const float sl2 = a.scale_log2;
  f32x16 sA[2], sB[2];   // scores of the current / next half
  v8 pA[2][2], pB[2][2]; // bf16 P^T of half 0 / half 1 of a tile

  // S^T for one half (K rows 32h..32h+31 of the tile in ring slot `sp`);
  // RB0: row block 0 takes part
  auto qk = [&](const unsigned char* sp, int h, f32x16 (&s)[2], auto rb0_c) {
    constexpr bool RB0 = decltype(rb0_c)::value;
    v8 ka[DC];
#pragma unroll
    for (int c = 0; c < DC; ++c)
      ka[c] = __builtin_bit_cast(v8, *reinterpret_cast<const u32x4*>(sp + k_rd[c] + h * 32 * ROW_B));
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int i = 0; i < 16; ++i) s[rb][i] = 0.f;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      if constexpr (RB0) s[0] = MM::mma(ka[c], qreg[0][c], s[0]);
      s[1] = MM::mma(ka[c], qreg[1][c], s[1]);
    }
  };
  // O^T += V^T P^T for one half (V rows 32h..32h+31 of the tile in slot `sp`)
  auto pv = [&](const unsigned char* sp, int h, const v8 (&p)[2][2], auto rb0_c) {
    constexpr bool RB0 = decltype(rb0_c)::value;
#pragma unroll
    for (int cc = 0; cc < 2; ++cc)
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        const int off = (32 * h + 16 * cc) * ROW_B + db * 64;
        const uint2 lo = lds_read_tr(sp + v_rd[0] + off);
        const uint2 hi = lds_read_tr(sp + v_rd[1] + off);
        const v8 vv = __builtin_bit_cast(v8, u32x4{lo.x, lo.y, hi.x, hi.y});
        if constexpr (RB0) o[0][db] = MM::mma(vv, p[0][cc], o[0][db]);
        o[1][db] = MM::mma(vv, p[1][cc], o[1][db]);
      }
  };
  // Online softmax of one half.  Row block rb takes part iff USE0 (rb 0) /
  // always (rb 1); MASKrb applies the causal triangle.  The running max and
  // sum are updated without branches (alpha = 1 when the max stays), so the
  // whole half is one scheduling region with its MFMAs; the returned flag says
  // whether O must be rescaled once those MFMAs are done.
  float alpha[2] = {1.f, 1.f};
  auto smax = [&](f32x16 (&s)[2], v8 (&p)[2][2], auto use0_c, auto mask0_c, auto mask1_c) {
    constexpr bool USE0 = decltype(use0_c)::value;
    constexpr bool MASK[2] = {decltype(mask0_c)::value, decltype(mask1_c)::value};
    float mx[2] = {kNegBig, kNegBig};
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      if (rb == 0 && !USE0) continue;
      if (MASK[rb]) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (16 * (i >> 3) + (i & 7) > tri) s[rb][i] = -INFINITY;
      }
      // running max as a chain of 3-input maxima (v_max3_f32: 8 ops per 16)
      float x = fmaxf(fmaxf(s[rb][0], s[rb][1]), s[rb][2]);
#pragma unroll
      for (int i = 3; i < 15; i += 2) x = fmaxf(fmaxf(x, s[rb][i]), s[rb][i + 1]);
      x = fmaxf(x, s[rb][15]);
      auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
      mx[rb] = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * sl2;
    }
    const bool up = (USE0 && mx[0] > m[0] + kRescaleThreshold) || mx[1] > m[1] + kRescaleThreshold;
    const bool resc = __builtin_amdgcn_ballot_w64(up) != 0;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      if (rb == 0 && !USE0) continue;
      const float m_new = resc ? fmaxf(m[rb], mx[rb]) : m[rb];
      alpha[rb] = fast_exp2(m[rb] - m_new);
      m[rb] = m_new;
      const float mr = m_new;
      float ls0 = 0.f, ls1 = 0.f;
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        uint32_t wd[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float e0 = fast_exp2(fmaf(s[rb][8 * cc + 2 * t], sl2, -mr));
          const float e1 = fast_exp2(fmaf(s[rb][8 * cc + 2 * t + 1], sl2, -mr));
          if (t & 1) ls1 += e0 + e1; else ls0 += e0 + e1;
          wd[t] = MM::pack2(e0, e1);
        }
        p[rb][cc] = __builtin_bit_cast(v8, u32x4{wd[0], wd[1], wd[2], wd[3]});
      }
      l[rb] = fmaf(l[rb], alpha[rb], ls0 + ls1);
      // keep this half's softmax inside its slot: without a use here the
      // compiler sinks it past the tile barrier into the next slot
#pragma unroll
      for (int cc = 0; cc < 2; ++cc)
        __asm__ volatile("" ::"v"(__builtin_bit_cast(u32x4, p[rb][cc])));
      __asm__ volatile("" ::"v"(l[rb]), "v"(m[rb]));
    }
    return resc;
  };
  // Softmax of one half against the running max, without the half's own max:
  // every p is at most the lane's row sum of the half, so while that sum stays
  // at or below 16 * 2^kRescaleThreshold no p exceeds 2^(kRescaleThreshold + 4)
  // and the running max may stay (the same lazy rule as above, with 4 more
  // bits of headroom).  Returns true (uniform over the wave) when some lane's
  // sum is larger; the caller then runs smax on the same scores, which finds
  // the max, moves it and recomputes P (the scores are left intact here apart
  // from the causal mask).  A wave's first tile always takes that path (its
  // running max is still kNegBig).
  auto smax_fast = [&](f32x16 (&s)[2], v8 (&p)[2][2], auto use0_c, auto mask0_c, auto mask1_c) {
    constexpr bool USE0 = decltype(use0_c)::value;
    constexpr bool MASK[2] = {decltype(mask0_c)::value, decltype(mask1_c)::value};
    float lsum[2] = {0.f, 0.f};
    bool big = false;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      if (rb == 0 && !USE0) continue;
      if (MASK[rb]) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (16 * (i >> 3) + (i & 7) > tri) s[rb][i] = -INFINITY;
      }
      const float mr = m[rb];
      float ls0 = 0.f, ls1 = 0.f;
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        uint32_t wd[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float e0 = fast_exp2(fmaf(s[rb][8 * cc + 2 * t], sl2, -mr));
          const float e1 = fast_exp2(fmaf(s[rb][8 * cc + 2 * t + 1], sl2, -mr));
          if (t & 1) ls1 += e0 + e1; else ls0 += e0 + e1;
          wd[t] = MM::pack2(e0, e1);
        }
        p[rb][cc] = __builtin_bit_cast(v8, u32x4{wd[0], wd[1], wd[2], wd[3]});
      }
      lsum[rb] = ls0 + ls1;
      big = big || !(lsum[rb] <= kFastSumLimit);
    }
    const bool fb = __builtin_amdgcn_ballot_w64(big) != 0;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      if (rb == 0 && !USE0) continue;
      l[rb] = fb ? l[rb] : l[rb] + lsum[rb];
#pragma unroll
      for (int cc = 0; cc < 2; ++cc)
        __asm__ volatile("" ::"v"(__builtin_bit_cast(u32x4, p[rb][cc])));
      __asm__ volatile("" ::"v"(l[rb]));
    }
    return fb;
  };
  auto rescale_o = [&](auto use0_c) {
    constexpr bool USE0 = decltype(use0_c)::value;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      if (rb == 0 && !USE0) continue;
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[rb][db][i] *= alpha[rb];
    }
  };
  // wait until at most `keep` tiles' copies of this wave are in flight
  auto wait_tiles = [&](int keep) {
    if (keep >= 2) __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * NI) : "memory");
    else if (keep == 1) __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * NI) : "memory");
    else dma_wait_all();
  };
  using TT = std::true_type;
  using FF = std::false_type;
  // Issue order of a steady-state slot: the slot's LDS operand reads first,
  // then one MFMA followed by a run of softmax VALU work, repeated.  A wave's
  // own VALU issue stalls for about half of each 32x32x16 MFMA, so spreading
  // the 16 MFMAs evenly through the ~150 softmax instructions keeps the matrix
  // pipe fed instead of bunching MFMAs behind the row-max chain.
  auto interleave = [&]() {
    __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);   // DS reads
    __builtin_amdgcn_sched_group_barrier(0x402, 12, 0);   // VALU (incl. exp)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x402, 7, 0);  // VALU
    }
  };
  // slot A(t): softmax(t.h0) | PV(t-1.h1), QK(t.h1).  HAS_PV: t > 0;
  // DIAG: t is the wave's diagonal tile (its second half is hidden from rb 0).
  auto slot_a = [&](const unsigned char* cur, const unsigned char* prv, auto has_pv_c, auto diag_c) {
    constexpr bool HAS_PV = decltype(has_pv_c)::value, DIAG = decltype(diag_c)::value;
    if constexpr (HAS_PV) pv(prv, 1, pB, TT{});
    qk(cur, 1, sB, std::integral_constant<bool, !DIAG>{});
    if constexpr (!HAS_PV) {  // the wave's first tile: no running max yet, O still zero
      smax(sA, pA, TT{}, std::integral_constant<bool, DIAG>{}, FF{});
    } else {
      const bool fb = smax_fast(sA, pA, TT{}, std::integral_constant<bool, DIAG>{}, FF{});
      if constexpr (!DIAG) interleave();
      if (fb) {
        if (smax(sA, pA, TT{}, std::integral_constant<bool, DIAG>{}, FF{})) rescale_o(TT{});
      }
    }
  };
  // slot B(t): softmax(t.h1) | PV(t.h0), QK(t+1.h0); on the diagonal tile,
  // rb 1 only, followed by the drain PV(t.h1).
  auto slot_b = [&](const unsigned char* cur, const unsigned char* nxt, auto diag_c) {
    constexpr bool DIAG = decltype(diag_c)::value;
    pv(cur, 0, pA, TT{});
    if constexpr (!DIAG) {
      qk(nxt, 0, sA, TT{});
      const bool fb = smax_fast(sB, pB, TT{}, FF{}, FF{});
      interleave();
      if (fb) {
        if (smax(sB, pB, TT{}, FF{}, FF{})) rescale_o(TT{});
      }
    } else {
      if (smax_fast(sB, pB, FF{}, FF{}, TT{})) {
        if (smax(sB, pB, FF{}, FF{}, TT{})) rescale_o(FF{});
      }
      pv(cur, 1, pB, FF{});
    }
  };

  // wait for tile t+1, publish it, and start copying tile t+3 into the slot
  // that tile t-1 (last read in slot A(t)) has released
  auto sync_tile = [&](int t) {
    wait_tiles(min(n_tiles - 2 - t, 1));
    block_sync_lds();
    if (t + 3 < n_tiles) issue(t + 3);
  };
  auto buf = [&](int t) { return lds + (t % kSpBufs) * SLOT_B; };

  // ---- prologue: tiles 0..2 in flight, then Q (and its RoPE table rows),
  //      so the tile copies and the Q loads share one memory round trip (the
  //      copies are issued first: loads complete in issue order, and the
  //      compiler's wait for Q then covers them).  Rows past S read row S - 1:
  //      finite scores in rows whose output is never stored (each row's
  //      softmax and PV column are its own).  Wait for tile 0, QK(0.h0).
  issue(0);
  if (n_tiles > 1) issue(1);
  if (n_tiles > 2) issue(2);
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int qrow = min(r0 + 32 * rb + lr, a.S - 1);
    const T* qp = reinterpret_cast<const T*>(a.q) + (int64_t)b * a.q_sb +
                  (int64_t)head * a.q_sh + (int64_t)qrow * a.q_ss;
#pragma unroll
    for (int c = 0; c < DC; ++c) qreg[rb][c] = __builtin_bit_cast(v8, load16(qp + 16 * c + 8 * hh));
    if (a.rcos != nullptr) rope_q_fragments<T, DC>(a, qrow, hh, qreg[rb]);
  }
  wait_tiles(min(n_tiles - 1, 2));
  block_sync_lds();
  int t = 0;
  if (n_tw > 0) {
    qk(lds, 0, sA, TT{});
    if (n_tw == 1) {
      slot_a(buf(0), buf(0), FF{}, TT{});
      sync_tile(0);
      slot_b(buf(0), buf(0), TT{});
    } else {
      slot_a(buf(0), buf(0), FF{}, FF{});
      sync_tile(0);
      slot_b(buf(0), buf(1), FF{});
      for (t = 1; t < n_tw - 1; ++t) {   // steady state
        slot_a(buf(t), buf(t - 1), TT{}, FF{});
        sync_tile(t);
        slot_b(buf(t), buf(t + 1), FF{});
      }
      slot_a(buf(t), buf(t - 1), TT{}, TT{});  // diagonal tile
      sync_tile(t);
      slot_b(buf(t), buf(t), TT{});
    }
    t = n_tw;
  }
  for (; t < n_tiles; ++t) sync_tile(t);   // the block's remaining tiles

  if (n_tw == 0) return;
  if (a.o_line) {
    // Whole-row stores: each row block's 32 rows x 128 bytes are staged in a
    // ring slot that no wave reads any more (every wave has passed the last
    // tile barrier; only the last tile's slot is still read) and written back
    // with 8 lanes x 16 bytes per row, one instruction per 8 rows.
    constexpr int RS = 136;                  // staged row stride (bytes, padded)
    unsigned char* const stg =
        lds + ((n_tiles + (w >> 1)) % kSpBufs) * SLOT_B + (w & 1) * (32 * RS);
    T* const ob = reinterpret_cast<T*>(a.o) + (int64_t)b * a.o_sb + (int64_t)head * a.o_sh;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      float lt = l[rb];
      {  // both lane halves hold partial sums of the same row
        auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(lt), __float_as_uint(lt), false, false);
        lt = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
      }
      const float inv = 1.0f / lt;
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const int d = 32 * db + 8 * q4 + 4 * hh;
          const uint32_t w0 = MM::pack2(o[rb][db][4 * q4] * inv, o[rb][db][4 * q4 + 1] * inv);
          const uint32_t w1 = MM::pack2(o[rb][db][4 * q4 + 2] * inv, o[rb][db][4 * q4 + 3] * inv);
          typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
          *reinterpret_cast<u32x2*>(stg + lr * RS + d * 2) = u32x2{w0, w1};
        }
      __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // this wave's rows are staged
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rr = 8 * i + (lane >> 3), cc = lane & 7;
        const u32x4 v = *reinterpret_cast<const u32x4*>(stg + rr * RS + cc * 16);
        const int qr = r0 + 32 * rb + rr;
        if (qr < a.S) *reinterpret_cast<u32x4*>(ob + (int64_t)qr * a.o_ss + 8 * cc) = v;
      }
      const int qrow = r0 + 32 * rb + lr;
      if (a.lse != nullptr && hh == 0 && qrow < a.S)
        a.lse[((int64_t)b * a.Hq + head) * a.S + qrow] = (m[rb] + __log2f(lt)) * kLn2;
    }
    return;
  }
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    float lt = l[rb];
    {  // both lane halves hold partial sums of the same row
      auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(lt), __float_as_uint(lt), false, false);
      lt = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    const int qrow = r0 + 32 * rb + lr;
    if (qrow >= a.S) continue;
    const float inv = 1.0f / lt;
    T* op = reinterpret_cast<T*>(a.o) + (int64_t)b * a.o_sb + (int64_t)head * a.o_sh +
            (int64_t)qrow * a.o_ss;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d = 32 * db + 8 * q4 + 4 * hh;
        const uint32_t w0 = MM::pack2(o[rb][db][4 * q4] * inv, o[rb][db][4 * q4 + 1] * inv);
        const uint32_t w1 = MM::pack2(o[rb][db][4 * q4 + 2] * inv, o[rb][db][4 * q4 + 3] * inv);
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        *reinterpret_cast<u32x2*>(op + d) = u32x2{w0, w1};
      }
    if (a.lse != nullptr && hh == 0)
      a.lse[((int64_t)b * a.Hq + head) * a.S + qrow] = (m[rb] + __log2f(lt)) * kLn2;
  }
}

// ---------------------------------------------------------------------------
// Software-pipelined kernel with separate K and V double buffers, head dims 64
// and 128 (16-bit).  The slot schedule is prefill_sp_kernel's:
//
//   slot A(t): softmax(t.h0) | PV(t-1.h1), QK(t.h1)
//   ---- wait for K(t+1) and V(t), barrier, copy K(t+2) and V(t+1) ----
//   slot B(t): softmax(t.h1) | PV(t.h0),   QK(t+1.h0)
//
// K(t) is read in B(t-1) and A(t), V(t) in B(t) and A(t+1), so two slots of
// each suffice: the copy into a slot starts at the barrier right after the
// slot's previous tile was last read and has one slot pair to complete.  Four
// tiles of LDS (64 KB at D = 128, where a 4-slot ring of K+V tiles would need
// 128 KB), so two 4-wave blocks still share a CU.
// A wave owns RB 32-row blocks: RB = 2 at D = 64 (every K/V operand feeds two
// MFMAs), RB = 1 at D = 128 (the 32 x 128 fp32 O tile, Q and the operands of
// a slot take the registers two waves per SIMD leave).  Head dim 128 runs this
// kernel (119 us against 124 us for prefill_kernel<128> at B4 S2048 24/8
// heads); head dim 64 keeps prefill_sp_kernel (77 us against 79 us here).  Row block rb starts
// at row r0 + 32 rb; its phase is the half of a 64-key tile that row lies in.
// On the wave's diagonal tile a phase-0 row block sees half 0 through the
// causal triangle and none of half 1; a phase-1 row block sees half 0 whole
// and half 1 through the triangle.  Row-block sets are bit masks (PART: row
// blocks that take part, MSK: row blocks masked by the triangle).
// V tile swizzle of the pipelined kernel (XOR of the 16-byte chunk index of
// row r).  A half-wave's transposed V^T read touches rows r0..r0+3 (r0 a
// multiple of 4) at byte offsets 0..63: at D = 128 (256-byte rows, one bank
// row each) chunks ^ 4 (r & 3) put the four rows in the four quarters of the
// banks, at D = 64 (two rows per bank row) chunks ^ 4 ((r >> 1) & 1) put rows
// r0 + 2, r0 + 3 in the other halves of those of r0, r0 + 1 -- conflict-free
// instead of 4-way / 2-way.  Only chunk bits 2-3 change, and rows 16 apart
// share the swizzle.
template <int D>
__device__ inline int v_swz2(int r) { return D == 128 ? 4 * (r & 3) : 4 * ((r >> 1) & 1); }

template <typename T, int D>
__global__ __launch_bounds__(256, 2) void prefill_sp2_kernel(PrefillArgs a) {
  using MM = Mfma<T>;
  typedef typename MM::v8 v8;
  constexpr int RB = D == 64 ? 2 : 1;
  constexpr int BN = 64, KCH = D / 8, DC = D / 16, DB = D / 32;
  constexpr int ROW_B = D * 2, TILE_B = BN * ROW_B;
  constexpr int NI = TILE_B / 1024 / 4;        // 1 KB copies per wave per K (V) tile
  static_assert(NI * 4 * 1024 == TILE_B, "tile must split into 1 KB wave copies");
  constexpr int ALL = (1 << RB) - 1;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  unsigned char* const lds = smem_raw;         // K slot 0 | K slot 1 | V slot 0 | V slot 1

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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
  const int GH = a.heads_per_block, PJ = a.pj;
  constexpr int RW = 32 * RB;                         // query rows per wave
  const int p0 = pb * RW * PJ;
  const int g = w % GH, j = w / GH;
  const int head = kvh * a.G + hc * GH + g;
  const int r0 = p0 + RW * j;                         // first query row of this wave
  const int ph0 = (r0 >> 5) & 1;                      // phase of row block 0 (0 at RB = 2)
  const int n_tw = r0 < a.S ? r0 / BN + 1 : 0;        // tiles this wave reads (last = diagonal)
  const int n_tiles = (min(p0 + RW * PJ, a.S) - 1) / BN + 1;  // tiles the block copies

  v8 qreg[RB][DC];

  // ---- tile copies: wave w copies 1 KB pieces (w*NI + i) of each tile
  const unsigned char* kbase = reinterpret_cast<const unsigned char*>(a.k) +
                               ((int64_t)b * a.k_sb + (int64_t)kvh * a.k_sh) * 2;
  const unsigned char* vbase = reinterpret_cast<const unsigned char*>(a.v) +
                               ((int64_t)b * a.v_sb + (int64_t)kvh * a.v_sh) * 2;
  const uint32_t lds_k = lds_addr(lds) + w * NI * 1024, lds_v = lds_k + 2 * TILE_B;
  // copy the K (IS_V false) or V tile t into its slot t % 2; the lane -> chunk
  // geometry is recomputed per tile rather than kept in registers
  auto issue = [&](int t, auto is_v_c) __attribute__((always_inline)) {
    constexpr bool IS_V = decltype(is_v_c)::value;
    const int r0t = t * BN;
    const int64_t ss = IS_V ? a.v_ss : a.k_ss;
    const unsigned char* tb = (IS_V ? vbase : kbase) + (int64_t)r0t * ss * 2;
    const uint32_t dst = (IS_V ? lds_v : lds_k) + (t & 1) * TILE_B;
    const int lim = a.S - 1 - r0t;   // rows past S are clamped (masked out later)
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int idx = (w * NI + i) * 64 + lane;   // physical chunk index in the tile
      const int r = idx / KCH, pc = idx % KCH;
      const int rr = min(r, lim);
      const int lc = pc ^ (IS_V ? v_swz2<D>(r) : k_swz<D>(r));
      lds_dma16(tb, (uint32_t)(rr * ss + lc * 8) * 2u, dst + i * 1024);
    }
  };
  auto kslot = [&](int t) __attribute__((always_inline)) { return lds + (t & 1) * TILE_B; };
  auto vslot = [&](int t) __attribute__((always_inline)) { return lds + (2 + (t & 1)) * TILE_B; };

  // ---- per-lane operand read offsets (bytes, within one slot)
  const int prow = perm_row(lr);
  int k_rd[DC];
#pragma unroll
  for (int c = 0; c < DC; ++c) k_rd[c] = prow * ROW_B + (((2 * c + hh) ^ k_swz<D>(prow)) * 16);
  // V^T operand rows r = 32*half + 16*cc + 8*(gq>>1) + 4*part + (sl>>2), dims
  // 32 db + d0 .. +3: the swizzle changes the chunk's bits 2-3 (which db
  // selects) by a value of `part` and the lane, so one base offset per
  // (part, db) plus immediates address every read.
  const int gq = lane >> 4, sl = lane & 15;
  int v_rd[2][DB];
#pragma unroll
  for (int part = 0; part < 2; ++part) {
    const int r = 8 * (gq >> 1) + 4 * part + (sl >> 2);
    const int d0 = 16 * (gq & 1) + 4 * (sl & 3);
#pragma unroll
    for (int db = 0; db < DB; ++db)
      v_rd[part][db] = r * ROW_B + (((d0 >> 3) + 4 * db) ^ v_swz2<D>(r)) * 16 + (d0 & 7) * 2;
  }
  // causal triangle of a diagonal half: score i of this lane is key offset
  // kk(i) within the half, visible iff kk(i) <= tri
  const int tri = lr - 8 * hh;

  f32x16 o[RB][DB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[rb][db][i] = 0.f;
  float m[RB], l[RB], alpha[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) { m[rb] = kNegBig; l[rb] = 0.f; alpha[rb] = 1.f; }
  const float sl2 = a.scale_log2;
  f32x16 sA[RB], sB[RB];   // scores of the current / next half
  v8 pA[RB][2], pB[RB][2]; // P^T of half 0 / half 1 of a tile

  // S^T for one half (K rows 32h..32h+31 of the tile in K slot ks)
  auto qk = [&](const unsigned char* ks, int h, f32x16 (&s)[RB], auto part_c) __attribute__((always_inline)) {
    constexpr int PART = decltype(part_c)::value;
    if constexpr (PART != 0) {
      v8 ka[DC];
#pragma unroll
      for (int c = 0; c < DC; ++c)
        ka[c] = __builtin_bit_cast(v8, *reinterpret_cast<const u32x4*>(ks + k_rd[c] + h * 32 * ROW_B));
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
        if ((PART >> rb) & 1)
#pragma unroll
          for (int i = 0; i < 16; ++i) s[rb][i] = 0.f;
#pragma unroll
      for (int c = 0; c < DC; ++c)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          if ((PART >> rb) & 1) s[rb] = MM::mma(ka[c], qreg[rb][c], s[rb]);
    }
  };
  // O^T += V^T P^T for one half (V rows 32h..32h+31 of the tile in V slot vs)
  auto pv = [&](const unsigned char* vs, int h, const v8 (&p)[RB][2], auto part_c) __attribute__((always_inline)) {
    constexpr int PART = decltype(part_c)::value;
    if constexpr (PART != 0) {
#pragma unroll
      for (int cc = 0; cc < 2; ++cc)
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const int off = (32 * h + 16 * cc) * ROW_B;
          const uint2 lo = lds_read_tr(vs + v_rd[0][db] + off);
          const uint2 hi = lds_read_tr(vs + v_rd[1][db] + off);
          const v8 vv = __builtin_bit_cast(v8, u32x4{lo.x, lo.y, hi.x, hi.y});
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
            if ((PART >> rb) & 1) o[rb][db] = MM::mma(vv, p[rb][cc], o[rb][db]);
        }
    }
  };
  // PV of one half (V slot vs, half hv) and QK of another (K slot ks, half hk)
  // for every row block, as DC steps of one K operand read, one V^T operand
  // read and their MFMAs, so that each step's LDS reads are in flight while
  // the previous step's MFMAs run (the two products are independent; reads and
  // MFMAs issued as separate loops end up as read, wait, MFMA at these
  // register counts).
  auto pvqk = [&](const unsigned char* vs, int hv, const v8 (&p)[RB][2],
                  const unsigned char* ks, int hk, f32x16 (&s)[RB]) __attribute__((always_inline)) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int i = 0; i < 16; ++i) s[rb][i] = 0.f;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      const int cc = c / DB, db = c % DB;    // PV step c: 16 keys cc, 32 dims db
      const v8 ka = __builtin_bit_cast(v8, *reinterpret_cast<const u32x4*>(ks + k_rd[c] + hk * 32 * ROW_B));
      const int off = (32 * hv + 16 * cc) * ROW_B;
      const uint2 lo = lds_read_tr(vs + v_rd[0][db] + off);
      const uint2 hi = lds_read_tr(vs + v_rd[1][db] + off);
      const v8 vv = __builtin_bit_cast(v8, u32x4{lo.x, lo.y, hi.x, hi.y});
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) s[rb] = MM::mma(ka, qreg[rb][c], s[rb]);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) o[rb][db] = MM::mma(vv, p[rb][cc], o[rb][db]);
    }
  };
  // Online softmax of one half for the row blocks of PART (MSK: with the
  // causal triangle).  The running max and sum are updated without branches
  // (alpha = 1 when the max stays); the returned flag says whether O must be
  // rescaled once the half's MFMAs are done.
  auto smax = [&](f32x16 (&s)[RB], v8 (&p)[RB][2], auto part_c, auto msk_c) __attribute__((always_inline)) {
    constexpr int PART = decltype(part_c)::value, MSK = decltype(msk_c)::value;
    float mx[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      mx[rb] = kNegBig;
      if (!((PART >> rb) & 1)) continue;
      if ((MSK >> rb) & 1) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (16 * (i >> 3) + (i & 7) > tri) s[rb][i] = -INFINITY;
      }
      float x = fmaxf(fmaxf(s[rb][0], s[rb][1]), s[rb][2]);
#pragma unroll
      for (int i = 3; i < 15; i += 2) x = fmaxf(fmaxf(x, s[rb][i]), s[rb][i + 1]);
      x = fmaxf(x, s[rb][15]);
      auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
      mx[rb] = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * sl2;
    }
    bool up = false;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
      if ((PART >> rb) & 1) up = up || mx[rb] > m[rb] + kRescaleThreshold;
    const bool resc = __builtin_amdgcn_ballot_w64(up) != 0;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      if (!((PART >> rb) & 1)) continue;
      const float m_new = resc ? fmaxf(m[rb], mx[rb]) : m[rb];
      alpha[rb] = fast_exp2(m[rb] - m_new);
      m[rb] = m_new;
      const float mr = m_new;
      float ls0 = 0.f, ls1 = 0.f;
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        uint32_t wd[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float e0 = fast_exp2(fmaf(s[rb][8 * cc + 2 * t], sl2, -mr));
          const float e1 = fast_exp2(fmaf(s[rb][8 * cc + 2 * t + 1], sl2, -mr));
          if (t & 1) ls1 += e0 + e1; else ls0 += e0 + e1;
          wd[t] = MM::pack2(e0, e1);
        }
        p[rb][cc] = __builtin_bit_cast(v8, u32x4{wd[0], wd[1], wd[2], wd[3]});
      }
      l[rb] = fmaf(l[rb], alpha[rb], ls0 + ls1);
      // keep this half's softmax inside its slot: without a use here the
      // compiler sinks it past the tile barrier into the next slot
#pragma unroll
      for (int cc = 0; cc < 2; ++cc)
        __asm__ volatile("" ::"v"(__builtin_bit_cast(u32x4, p[rb][cc])));
      __asm__ volatile("" ::"v"(l[rb]), "v"(m[rb]));
    }
    return resc;
  };
  // Softmax of one half against the running max, without the half's own max
  // (prefill_sp_kernel's smax_fast): while a lane's row sum of the half stays
  // at or below 16 * 2^kRescaleThreshold no p exceeds 2^(kRescaleThreshold+4)
  // and the running max may stay.  Returns true (uniform over the wave) when
  // some lane's sum is larger; the caller then runs smax on the same scores.
  auto smax_fast = [&](f32x16 (&s)[RB], v8 (&p)[RB][2], auto part_c, auto msk_c) __attribute__((always_inline)) {
    constexpr int PART = decltype(part_c)::value, MSK = decltype(msk_c)::value;
    float lsum[RB];
    bool big = false;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      lsum[rb] = 0.f;
      if (!((PART >> rb) & 1)) continue;
      if ((MSK >> rb) & 1) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (16 * (i >> 3) + (i & 7) > tri) s[rb][i] = -INFINITY;
      }
      const float mr = m[rb];
      float ls0 = 0.f, ls1 = 0.f;
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        uint32_t wd[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float e0 = fast_exp2(fmaf(s[rb][8 * cc + 2 * t], sl2, -mr));
          const float e1 = fast_exp2(fmaf(s[rb][8 * cc + 2 * t + 1], sl2, -mr));
          if (t & 1) ls1 += e0 + e1; else ls0 += e0 + e1;
          wd[t] = MM::pack2(e0, e1);
        }
        p[rb][cc] = __builtin_bit_cast(v8, u32x4{wd[0], wd[1], wd[2], wd[3]});
      }
      lsum[rb] = ls0 + ls1;
      big = big || !(lsum[rb] <= kFastSumLimit);
    }
    const bool fb = __builtin_amdgcn_ballot_w64(big) != 0;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      if (!((PART >> rb) & 1)) continue;
      l[rb] = fb ? l[rb] : l[rb] + lsum[rb];
#pragma unroll
      for (int cc = 0; cc < 2; ++cc)
        __asm__ volatile("" ::"v"(__builtin_bit_cast(u32x4, p[rb][cc])));
      __asm__ volatile("" ::"v"(l[rb]));
    }
    return fb;
  };
  auto rescale_o = [&](auto part_c) __attribute__((always_inline)) {
    constexpr int PART = decltype(part_c)::value;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      if (!((PART >> rb) & 1)) continue;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[rb][db][i] *= alpha[rb];
    }
  };
  // Issue order of a steady-state slot: the slot's LDS operand reads first,
  // then one MFMA followed by a run of softmax VALU work, repeated (a wave's
  // own VALU issue stalls for about half of each 32x32x16 MFMA).
  // Steady-state slot order: pvqk's step c + 1 reads (one K, two V^T) are
  // issued before step c's MFMAs, and a run of softmax VALU work follows each
  // MFMA (a wave's own VALU issue stalls for about half of each 32x32x16
  // MFMA, so the softmax spreads over the matrix work).
  constexpr int kVa0 = D == 64 ? 12 : 6, kVa = D == 64 ? 7 : 4;
  auto interleave = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);     // step 0 reads
    __builtin_amdgcn_sched_group_barrier(0x402, kVa0, 0);  // VALU (incl. exp)
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      if (c + 1 < DC) __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);   // step c+1 reads
#pragma unroll
      for (int m = 0; m < 2 * RB; ++m) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
        __builtin_amdgcn_sched_group_barrier(0x402, kVa, 0);  // VALU
      }
    }
  };
  using TT = std::true_type;
  using FF = std::false_type;
  using IAll = std::integral_constant<int, ALL>;
  using I0 = std::integral_constant<int, 0>;
  // slot A(t): softmax(t.h0) | PV(t-1.h1), QK(t.h1).  HAS_PV: t > 0 (tile t-1
  // is below the diagonal: every row block takes part in PV(t-1.h1)).  P_H1:
  // row blocks that see half 1 of tile t; M_H0: row blocks whose half 0 is
  // the causal triangle (both ALL / 0 below the diagonal).
  auto slot_a = [&](int t, auto has_pv_c, auto p_h1_c, auto m_h0_c) __attribute__((always_inline)) {
    constexpr bool HAS_PV = decltype(has_pv_c)::value;
    constexpr int P_H1 = decltype(p_h1_c)::value, M_H0 = decltype(m_h0_c)::value;
    if constexpr (HAS_PV && P_H1 == ALL) {
      pvqk(vslot(t - 1), 1, pB, kslot(t), 1, sB);
    } else {
      if constexpr (HAS_PV) pv(vslot(t - 1), 1, pB, IAll{});
      qk(kslot(t), 1, sB, p_h1_c);
    }
    if constexpr (!HAS_PV) {  // the wave's first tile: no running max yet, O still zero
      smax(sA, pA, IAll{}, m_h0_c);
    } else {
      const bool fb = smax_fast(sA, pA, IAll{}, m_h0_c);
      if constexpr (P_H1 == ALL && M_H0 == 0) interleave();
      if (fb) {
        if (smax(sA, pA, IAll{}, m_h0_c)) rescale_o(IAll{});
      }
    }
  };
  // slot B(t): softmax(t.h1) | PV(t.h0), QK(t+1.h0); on the diagonal tile the
  // softmax of half 1 for the row blocks P_H1 that see it, then their drain
  // PV(t.h1).
  auto slot_b = [&](int t, auto diag_c, auto p_h1_c) __attribute__((always_inline)) {
    constexpr bool DIAG = decltype(diag_c)::value;
    constexpr int P_H1 = decltype(p_h1_c)::value;
    if constexpr (!DIAG) {
      pvqk(vslot(t), 0, pA, kslot(t + 1), 0, sA);
      const bool fb = smax_fast(sB, pB, IAll{}, I0{});
      interleave();
      if (fb) {
        if (smax(sB, pB, IAll{}, I0{})) rescale_o(IAll{});
      }
    } else if constexpr (P_H1 == 0) {
      pv(vslot(t), 0, pA, IAll{});
    } else {
      pv(vslot(t), 0, pA, IAll{});
      if (smax_fast(sB, pB, p_h1_c, p_h1_c)) {
        if (smax(sB, pB, p_h1_c, p_h1_c)) rescale_o(p_h1_c);
      }
      pv(vslot(t), 1, pB, p_h1_c);
    }
  };
  // the diagonal tile's slots: at RB = 2 row block 0 is phase 0 and row block 1
  // phase 1; at RB = 1 the wave's one row block has phase PH (the phase of its
  // first row, a compile-time branch of the whole tile loop below: a branch on
  // it inside the loop leaves the register allocator 100+ spills)
  auto diag_a = [&](int t, auto has_pv_c, auto ph_c) __attribute__((always_inline)) {
    constexpr int PH = decltype(ph_c)::value;
    if constexpr (RB == 2)
      slot_a(t, has_pv_c, std::integral_constant<int, 2>{}, std::integral_constant<int, 1>{});
    else if constexpr (PH == 0)
      slot_a(t, has_pv_c, I0{}, std::integral_constant<int, 1>{});
    else
      slot_a(t, has_pv_c, std::integral_constant<int, 1>{}, I0{});
  };
  auto diag_b = [&](int t, auto ph_c) __attribute__((always_inline)) {
    constexpr int PH = decltype(ph_c)::value;
    if constexpr (RB == 2)
      slot_b(t, TT{}, std::integral_constant<int, 2>{});
    else if constexpr (PH == 0)
      slot_b(t, TT{}, I0{});
    else
      slot_b(t, TT{}, std::integral_constant<int, 1>{});
  };
  // wait for K(t+1) and V(t), publish them, then copy K(t+2) into the slot
  // K(t) (last read in slot A(t)) released and V(t+1) into V(t-1)'s
  auto sync_tile = [&](int t) __attribute__((always_inline)) {
    dma_wait_all();
    block_sync_lds();
    if (t + 2 < n_tiles) issue(t + 2, FF{});
    if (t + 1 < n_tiles) issue(t + 1, TT{});
  };

  // ---- prologue: K(0), V(0), K(1) in flight, then Q (and its RoPE table
  //      rows), so the copies and the Q loads share one memory round trip.
  //      Rows past S read row S - 1: finite scores in rows whose output is
  //      never stored.
  issue(0, FF{});
  issue(0, TT{});
  if (n_tiles > 1) issue(1, FF{});
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int qrow = min(r0 + 32 * rb + lr, a.S - 1);
    const T* qp = reinterpret_cast<const T*>(a.q) + (int64_t)b * a.q_sb +
                  (int64_t)head * a.q_sh + (int64_t)qrow * a.q_ss;
#pragma unroll
    for (int c = 0; c < DC; ++c) qreg[rb][c] = __builtin_bit_cast(v8, load16(qp + 16 * c + 8 * hh));
    if (a.rcos != nullptr) rope_q_fragments<T, DC>(a, qrow, hh, qreg[rb]);
  }
  dma_wait_all();
  block_sync_lds();
  auto run = [&](auto ph_c) __attribute__((always_inline)) {
    int t = 0;
    if (n_tw > 0) {
      qk(kslot(0), 0, sA, IAll{});
      if (n_tw == 1) {
        diag_a(0, FF{}, ph_c);
        sync_tile(0);
        diag_b(0, ph_c);
      } else {
        slot_a(0, FF{}, IAll{}, I0{});
        sync_tile(0);
        slot_b(0, FF{}, IAll{});
        for (t = 1; t < n_tw - 1; ++t) {   // steady state
          slot_a(t, TT{}, IAll{}, I0{});
          sync_tile(t);
          slot_b(t, FF{}, IAll{});
        }
        diag_a(t, TT{}, ph_c);             // diagonal tile
        sync_tile(t);
        diag_b(t, ph_c);
      }
      t = n_tw;
    }
    for (; t < n_tiles; ++t) sync_tile(t);   // the block's remaining tiles
  };
  if (RB == 2 || ph0 == 0)
    run(I0{});
  else
    run(std::integral_constant<int, 1>{});

  if (n_tw == 0) return;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    float lt = l[rb];
    {  // both lane halves hold partial sums of the same row
      auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(lt), __float_as_uint(lt), false, false);
      lt = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    const int qrow = r0 + 32 * rb + lr;
    if (qrow >= a.S) continue;
    const float inv = 1.0f / lt;
    T* op = reinterpret_cast<T*>(a.o) + (int64_t)b * a.o_sb + (int64_t)head * a.o_sh +
            (int64_t)qrow * a.o_ss;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d = 32 * db + 8 * q4 + 4 * hh;
        const uint32_t w0 = MM::pack2(o[rb][db][4 * q4] * inv, o[rb][db][4 * q4 + 1] * inv);
        const uint32_t w1 = MM::pack2(o[rb][db][4 * q4 + 2] * inv, o[rb][db][4 * q4 + 3] * inv);
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        *reinterpret_cast<u32x2*>(op + d) = u32x2{w0, w1};
      }
    if (a.lse != nullptr && hh == 0)
      a.lse[((int64_t)b * a.Hq + head) * a.S + qrow] = (m[rb] + __log2f(lt)) * kLn2;
  }
}

// Plain VALU flash attention in fp32 arithmetic: every head dim of fp32
// inputs (no fp32 MFMA tiles), and head dims 16 and 256 of bf16/fp16 inputs
// (the MFMA kernels cover 32, 64 and 128).  TPR = D/8 lanes per query row, 8
// dims each (32 rows per 256-thread block at D = 64, 16 at D = 128, so a short
// sequence still gives the GPU hundreds of blocks and a long row's chain of
// keys is split over many lanes); K/V tiles converted to fp32 and staged in
// LDS with 16-byte copies, read back as 16-byte broadcasts.  Keys are taken 8
// at a time: 8 independent dot-product chains, one running-max update and one
// rescale per group of 8.  Optional q RoPE in the prologue (the RoPE kernels'
// rounding to T).  Outputs are rounded once to T.
template <typename T, int D>
__global__ __launch_bounds__(256) void prefill_valu_kernel(PrefillArgs a) {
  constexpr int DL = 8, TPR = D / DL, BN = 4096 / D;  // K+V tiles: 32 KB of LDS
  constexpr int ROWS = 256 / TPR;  // query rows per block
  constexpr int KB = 8;            // keys per softmax update
  constexpr int CN = Chunk<T>::kN; // elements per 16-byte chunk
  __shared__ __align__(16) float ks[BN][D];
  __shared__ __align__(16) float vs[BN][D];
  typedef float f4 __attribute__((ext_vector_type(4)));
  const int tid = threadIdx.x;
  const int part = tid % TPR, row_in = tid / TPR;
  const int n_rb = (a.S + ROWS - 1) / ROWS;
  const int rb = n_rb - 1 - (int)(blockIdx.x % n_rb);
  const int bh = (int)(blockIdx.x / n_rb);
  const int head = bh % a.Hq, b = bh / a.Hq;
  const int kvh = head / a.G;
  const int qrow = rb * ROWS + row_in;
  const int qr = min(qrow, a.S - 1);
  const T* qp = reinterpret_cast<const T*>(a.q) + (int64_t)b * a.q_sb +
                (int64_t)head * a.q_sh + (int64_t)qr * a.q_ss;
  float qv[DL], acc[DL];
#pragma unroll
  for (int i = 0; i < DL; ++i) { qv[i] = Elem<T>::to_f32(qp[part * DL + i]); acc[i] = 0.f; }
  if (a.rcos != nullptr) {
    // rotation partner of dim d is d + D/2 (or d - D/2): lane part +- TPR/2
    int64_t crow = qr;
    if (a.rpos != nullptr) crow = min(max(a.rpos[qr], (int64_t)0), a.r_rows - 1);
    const bool lo = part < TPR / 2;
    const int i0 = (lo ? part : part - TPR / 2) * DL;
    const T* cp = reinterpret_cast<const T*>(a.rcos) + crow * a.r_ss + i0;
    const T* sp = reinterpret_cast<const T*>(a.rsin) + crow * a.r_ss + i0;
#pragma unroll
    for (int i = 0; i < DL; ++i) {
      const float other = Elem<T>::to_f32(qp[(lo ? part + TPR / 2 : part - TPR / 2) * DL + i]);
      T y1, y2;
      rope_rotate<T, T>(lo ? qv[i] : other, lo ? other : qv[i], cp[i], sp[i], y1, y2);
      qv[i] = Elem<T>::to_f32(lo ? y1 : y2);
    }
  }
  float m = kNegBig, l = 0.f;
  const T* kb = reinterpret_cast<const T*>(a.k) + (int64_t)b * a.k_sb + (int64_t)kvh * a.k_sh;
  const T* vb = reinterpret_cast<const T*>(a.v) + (int64_t)b * a.v_sb + (int64_t)kvh * a.v_sh;
  const int last = min(rb * ROWS + ROWS, a.S) - 1;
  for (int k0 = 0; k0 <= last; k0 += BN) {
    __syncthreads();
    for (int e = tid; e < BN * D / CN; e += 256) {
      const int r = e / (D / CN), d = CN * (e % (D / CN));
      const int row = min(k0 + r, a.S - 1);
      float kf[CN], vf[CN];
      Chunk<T>::unpack(load16(kb + (int64_t)row * a.k_ss + d), kf);
      Chunk<T>::unpack(load16(vb + (int64_t)row * a.v_ss + d), vf);
#pragma unroll
      for (int c = 0; c < CN; c += 4) {
        *reinterpret_cast<f4*>(&ks[r][d + c]) = f4{kf[c], kf[c + 1], kf[c + 2], kf[c + 3]};
        *reinterpret_cast<f4*>(&vs[r][d + c]) = f4{vf[c], vf[c + 1], vf[c + 2], vf[c + 3]};
      }
    }
    __syncthreads();
    const int nk = min(BN, qrow - k0 + 1);  // keys k0..qrow are visible
    for (int j0 = 0; j0 < nk; j0 += KB) {
      float sc[KB];
#pragma unroll
      for (int u = 0; u < KB; ++u) {
        const float* kr = &ks[min(j0 + u, BN - 1)][part * DL];
        const f4 k0v = *reinterpret_cast<const f4*>(kr), k1v = *reinterpret_cast<const f4*>(kr + 4);
        float sdot = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) sdot = fmaf(qv[i], k0v[i], sdot);
#pragma unroll
        for (int i = 0; i < 4; ++i) sdot = fmaf(qv[4 + i], k1v[i], sdot);
        sc[u] = sdot;
      }
      float mx = kNegBig;
#pragma unroll
      for (int u = 0; u < KB; ++u) {
        sc[u] = group_sum<TPR>(sc[u]) * a.scale_log2;
        if (j0 + u >= nk) sc[u] = -INFINITY;
        mx = fmaxf(mx, sc[u]);
      }
      const float mn = fmaxf(m, mx);
      const float alpha = fast_exp2(m - mn);
      float ps = 0.f, p[KB];
#pragma unroll
      for (int u = 0; u < KB; ++u) {
        p[u] = fast_exp2(sc[u] - mn);
        ps += p[u];
      }
      l = l * alpha + ps;
#pragma unroll
      for (int i = 0; i < DL; ++i) acc[i] *= alpha;
#pragma unroll
      for (int u = 0; u < KB; ++u) {
        const float* vr = &vs[min(j0 + u, BN - 1)][part * DL];
        const f4 v0 = *reinterpret_cast<const f4*>(vr), v1 = *reinterpret_cast<const f4*>(vr + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = fmaf(p[u], v0[i], acc[i]);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[4 + i] = fmaf(p[u], v1[i], acc[4 + i]);
      }
      m = mn;
    }
  }
  if (qrow >= a.S) return;
  T* op = reinterpret_cast<T*>(a.o) + (int64_t)b * a.o_sb + (int64_t)head * a.o_sh +
          (int64_t)qrow * a.o_ss + part * DL;
  const float inv = 1.0f / l;
#pragma unroll
  for (int i = 0; i < DL; ++i) op[i] = Elem<T>::from_f32(acc[i] * inv);
  if (a.lse != nullptr && part == 0)
    a.lse[((int64_t)b * a.Hq + head) * a.S + qrow] = (m + __log2f(l)) * kLn2;
}

namespace {

template <typename T, int D>
hipError_t launch(const PrefillArgs& a, int nwaves, hipStream_t stream) {
  const int n_pairs = a.B * a.Hkv * a.head_chunks;
  dim3 grid((unsigned)(n_pairs * a.n_pb));
  dim3 block((unsigned)(nwaves * 64));
  constexpr size_t smem = 2 * 2 * 64 * D * sizeof(T);  // 2 buffers x (K + V) tiles
  if constexpr (smem > 65536) {  // above the default dynamic-LDS limit: raise it once
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&prefill_kernel<T, D>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (attr != hipSuccess) return attr;
  }
  hipLaunchKernelGGL((prefill_kernel<T, D>), grid, block, smem, stream, a);
  return hipGetLastError();
}

// VALU kernel: D/8 lanes per query row, 2048/D rows per 256-thread block.
template <typename T>
hipError_t launch_valu(const PrefillArgs& a, int64_t head_dim, hipStream_t st) {
  const int rows = (int)(2048 / head_dim);
  const int64_t nblk = (int64_t)a.B * a.Hq * ((a.S + rows - 1) / rows);
  if (nblk > INT32_MAX) return hipErrorInvalidConfiguration;
  const dim3 grid((unsigned)nblk), block(256);
  switch (head_dim) {
    case 16: hipLaunchKernelGGL((prefill_valu_kernel<T, 16>), grid, block, 0, st, a); break;
    case 32: hipLaunchKernelGGL((prefill_valu_kernel<T, 32>), grid, block, 0, st, a); break;
    case 64: hipLaunchKernelGGL((prefill_valu_kernel<T, 64>), grid, block, 0, st, a); break;
    case 128: hipLaunchKernelGGL((prefill_valu_kernel<T, 128>), grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL((prefill_valu_kernel<T, 256>), grid, block, 0, st, a); break;
  }
  return hipGetLastError();
}

template <typename T, int D>
hipError_t launch_sp2(const PrefillArgs& a, hipStream_t stream) {
  const int n_pairs = a.B * a.Hkv * a.head_chunks;
  dim3 grid((unsigned)(n_pairs * a.n_pb));
  constexpr size_t smem = 4 * 64 * D * sizeof(T);  // K and V tiles, two slots each
  hipLaunchKernelGGL((prefill_sp2_kernel<T, D>), grid, dim3(256), smem, stream, a);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_sp(const PrefillArgs& a, hipStream_t stream) {
  const int n_pairs = a.B * a.Hkv * a.head_chunks;
  dim3 grid((unsigned)(n_pairs * a.n_pb));
  const size_t smem = (size_t)kSpBufs * 2 * 64 * 64 * sizeof(T);  // ring of (K + V) tiles
  hipLaunchKernelGGL((prefill_sp_kernel<T>), grid, dim3(256), smem, stream, a);
  return hipGetLastError();
}

}  // namespace
}  // namespace mi

using namespace mi;

namespace {

// Q RoPE for the prologue (cos == nullptr: none).
struct RopeQ {
  const void* cos = nullptr;
  const void* sin = nullptr;
  const int64_t* pos = nullptr;
  int64_t row_stride = 0, rows = 0;
};

int32_t attn_prefill(const void* q, const void* k, const void* v, void* o, float* lse,
                     int64_t batch, int64_t n_heads, int64_t n_kv_heads, int64_t seq_len,
                     int64_t kv_len, int64_t head_dim, int64_t q_sb, int64_t q_sh,
                     int64_t q_ss, int64_t k_sb, int64_t k_sh, int64_t k_ss, int64_t v_sb,
                     int64_t v_sh, int64_t v_ss, int64_t o_sb, int64_t o_sh, int64_t o_ss,
                     float sm_scale, int32_t dtype, const RopeQ& rq, void* stream) {
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
  if (!(head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128 ||
        head_dim == 256)) {
    set_last_error("attn_prefill: head_dim %lld has no kernel (supported: 16, 32, 64, 128, "
                   "256)", (long long)head_dim);
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
  // tile loads use 32-bit byte offsets from a per-tile base
  if ((k_ss > 0 ? k_ss : -k_ss) * 64 * eb + head_dim * eb >= ((int64_t)1 << 31) ||
      (v_ss > 0 ? v_ss : -v_ss) * 64 * eb + head_dim * eb >= ((int64_t)1 << 31) ||
      k_ss <= 0 || v_ss <= 0) {
    set_last_error("attn_prefill: K/V row stride out of range for 32-bit tile offsets");
    return MI_ERR_UNSUPPORTED;
  }
  if (seq_len > (1 << 30) || batch * n_kv_heads * n_heads > (1 << 30)) {
    set_last_error("attn_prefill: shape exceeds launch limits");
    return MI_ERR_UNSUPPORTED;
  }
  const int G = (int)(n_heads / n_kv_heads);
  // 4 waves per block, each 32*RB query rows of one head: 4 query heads, 2
  // heads x 2 slices or 1 head x 4 slices, whichever divides the group size.
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
  // D = 64 (16-bit): software-pipelined kernel, 4 waves of 64 rows; D = 32 and
  // 128: 4 waves of 32 rows.
  const bool sp = head_dim == 64 && dtype != MI_DTYPE_F32;
  const int rows_per_block = sp ? 64 * pj : 32 * prefill_row_blocks<128>() * pj;
  a.n_pb = (int32_t)((seq_len + rows_per_block - 1) / rows_per_block);
  a.scale_log2 = sm_scale * kLog2e;
  a.rcos = rq.cos; a.rsin = rq.sin; a.rpos = rq.pos;
  a.r_ss = rq.row_stride; a.r_rows = rq.rows;
  a.o_line = (po % 16 == 0 && ((o_sb | o_sh | o_ss) * eb) % 16 == 0) ? 1 : 0;
  const int nwaves = gh * pj;
  const int64_t blocks = (int64_t)a.B * a.Hkv * a.head_chunks * a.n_pb;
  if (blocks > INT32_MAX) {
    set_last_error("attn_prefill: grid too large");
    return MI_ERR_UNSUPPORTED;
  }
  hipError_t e;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == MI_DTYPE_F32 || head_dim == 16) {
    e = dtype == MI_DTYPE_F32   ? launch_valu<float>(a, head_dim, st)
        : dtype == MI_DTYPE_BF16 ? launch_valu<bf16_t>(a, head_dim, st)
                                 : launch_valu<f16_t>(a, head_dim, st);
  } else if (dtype == MI_DTYPE_BF16) {
    e = sp ? launch_sp<bf16_t>(a, st)
        : head_dim == 32 ? launch<bf16_t, 32>(a, nwaves, st)
        : head_dim == 128 ? launch_sp2<bf16_t, 128>(a, st) : launch<bf16_t, 256>(a, nwaves, st);
  } else {
    e = sp ? launch_sp<f16_t>(a, st)
        : head_dim == 32 ? launch<f16_t, 32>(a, nwaves, st)
        : head_dim == 128 ? launch_sp2<f16_t, 128>(a, st) : launch<f16_t, 256>(a, nwaves, st);
  }
  if (e != hipSuccess) {
    set_last_error("attn_prefill: launch failed: %s", hipGetErrorString(e));
    return (int32_t)e;
  }
  return MI_OK;
}

}  // namespace

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
  return attn_prefill(q, k, v, o, lse, batch, n_heads, n_kv_heads, seq_len, kv_len, head_dim,
                      q_sb, q_sh, q_ss, k_sb, k_sh, k_ss, v_sb, v_sh, v_ss, o_sb, o_sh, o_ss,
                      sm_scale, dtype, RopeQ{}, stream);
}

extern "C" int32_t mi_attn_prefill_rope(
    const void* q, const void* k, const void* v, void* o, float* lse, int64_t batch,
    int64_t n_heads, int64_t n_kv_heads, int64_t seq_len, int64_t kv_len, int64_t head_dim,
    int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t k_sb, int64_t k_sh, int64_t k_ss,
    int64_t v_sb, int64_t v_sh, int64_t v_ss, int64_t o_sb, int64_t o_sh, int64_t o_ss,
    float sm_scale, const void* cos, const void* sin, int64_t table_rows,
    int64_t table_row_stride, const int64_t* positions, int32_t dtype, void* stream) {
  if (dtype != MI_DTYPE_BF16 && dtype != MI_DTYPE_F16 && dtype != MI_DTYPE_F32) {
    set_last_error("attn_prefill_rope: unknown dtype code %d", (int)dtype);
    return MI_ERR_INVALID;
  }
  if (cos == nullptr || sin == nullptr) {
    set_last_error("attn_prefill_rope: null cos/sin table");
    return MI_ERR_INVALID;
  }
  // rows of D/2 entries; 16-bit tables 16-byte aligned (a lane reads 8 at once)
  const bool wide = dtype == MI_DTYPE_F32;
  if (table_rows <= 0 || table_row_stride < head_dim / 2 ||
      (!wide && ((table_row_stride * 2) % 16 != 0 || ((uintptr_t)cos | (uintptr_t)sin) % 16 != 0))) {
    set_last_error("attn_prefill_rope: cos/sin tables must hold rows of head_dim/2 entries with "
                   "16-byte aligned rows (rows %lld, row stride %lld)",
                   (long long)table_rows, (long long)table_row_stride);
    return MI_ERR_INVALID;
  }
  if (positions == nullptr && table_rows < seq_len) {
    set_last_error("attn_prefill_rope: %lld table rows for %lld query rows",
                   (long long)table_rows, (long long)seq_len);
    return MI_ERR_INVALID;
  }
  RopeQ rq;
  rq.cos = cos; rq.sin = sin; rq.pos = positions;
  rq.row_stride = table_row_stride; rq.rows = table_rows;
  return attn_prefill(q, k, v, o, lse, batch, n_heads, n_kv_heads, seq_len, kv_len, head_dim,
                      q_sb, q_sh, q_ss, k_sb, k_sh, k_ss, v_sb, v_sh, v_ss, o_sb, o_sh, o_ss,
                      sm_scale, dtype, rq, stream);
}
