// Causal GQA flash-attention prefill on bf16/fp16 MFMA (gfx950).
//
// Math: out[b,h,i] = softmax_j<=i(q_i.k_j / sqrt(D)) . V, query head h reading
// kv head h // G, keys bounded by the query length S
// (src/flash_attn.py:42-83, :85-111), plus lse[b,h,i] = logsumexp_j of the
// scaled scores (natural log), an output this build adds.
//
// Design (MI355X-first, not a translation of the Triton tile loop):
//  * A workgroup owns one (batch, kv-head, block of query positions) and runs
//    one wave per (query head of the GQA group, 64-row slice).  Every K/V tile
//    is staged in LDS once and consumed by all query heads that share it; each
//    wave uses every K/V operand it reads from LDS for two 32-row MFMA blocks.
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


// LDS tile layouts (one buffer): K [BN][D] and V [BN][D], both row-major in
// 16-byte chunks with the chunk index XOR-swizzled per row.  Tiles are filled
// by global->LDS DMA (global_load_lds_dwordx4): a wave instruction writes 1 KB
// contiguously, lane t at +16t, so the swizzle is realised by choosing which
// logical chunk each lane fetches.
template <int D>
__device__ inline int k_swz(int r) {  // XOR mask for K row r
  if constexpr (D == 64) return (r >> 1) & 7;
  else return r & 15;
}
__device__ inline int v_swz(int r) { return (r >> 1) & 3; }  // XOR mask for V row r

// Online-softmax rescale threshold (log2 units): the running row max used for
// exp2 is only moved when a new score exceeds it by more than this, so
// probabilities stay <= 2^8 (exact maths is unchanged: O and l share the same
// reference max) and O is rescaled on rare tiles instead of on every tile.
constexpr float kRescaleThreshold = 8.0f;

typedef short s16x4 __attribute__((ext_vector_type(4)));

// One wave-wide 16-byte-per-lane global->LDS copy: lane t's 16 bytes at
// base + voff land at LDS byte address lds + 16 t.  Issued as inline asm on
// purpose: the compiler does not track it, so it does not insert a wait for
// the copy before unrelated LDS reads of the other buffer; completion is
// awaited explicitly (dma_wait_all) before the barrier that publishes the tile.
// The compiler's hazard recognizer does not look inside inline asm, so the asm
// supplies the wait states itself: s_nop 4 (5 wait states) covers both a VALU
// write of the base SGPRs (v_readlane / v_readfirstlane, 5 required before a
// VMEM read) and the M0 write (1 required before an LDS DMA).
__device__ inline void lds_dma16(const unsigned char* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "{m0}"(lds)
               : "memory");
}
__device__ inline uint32_t lds_addr(const unsigned char* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) unsigned char*)(p);
}
__device__ inline void dma_wait_all() { __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

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

template <typename T, int D>
__global__ __launch_bounds__(256, 2) void prefill_kernel(PrefillArgs a) {
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

  // ---- Q as the B operand of S^T = K Q^T (lane: row lr of each row block)
  v8 qreg[RB][DC];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int qrow = qpos0 + 32 * rb + lr;
    const T* qp = reinterpret_cast<const T*>(a.q) + (int64_t)b * a.q_sb +
                  (int64_t)head * a.q_sh + (int64_t)min(qrow, a.S - 1) * a.q_ss;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      u32x4 raw = load16(qp + 16 * c + 8 * hh);
      if (qrow >= a.S) raw = u32x4{0, 0, 0, 0};
      qreg[rb][c] = __builtin_bit_cast(v8, raw);
    }
  }

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

  issue(0, 0);
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
      // latency is paid once per tile, not once per k-step
      v8 ka[2][DC];
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int c = 0; c < DC; ++c)
          ka[sb][c] = __builtin_bit_cast(
              v8, *reinterpret_cast<const u32x4*>(kl + k_rd[c] + sb * 32 * ROW_B));
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int c = 0; c < DC; ++c)
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) s[rb][sb] = MM::mma(ka[sb][c], qreg[rb][c], s[rb][sb]);
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
// Ping-pong variant (D = 64).  A wave issues instructions in order, so its own
// MFMAs and softmax VALU work run one after the other; the matrix core and the
// VALU of a SIMD do run side by side when the two streams come from different
// waves.  This kernel therefore runs 8 waves per block in two groups of four
// (wave w on SIMD w % 4, so every SIMD holds one wave of each group) and
// alternates them with block barriers: while group A issues the MFMAs of
// PV(t-1) + QK(t), group B runs the softmax of its tile t-1, then the roles
// swap.  Tiles live in a 3-slot LDS ring: tile t is read during four
// consecutive phases (QK by A then B, PV by A then B), and the copy of tile
// t+1 is issued two phases before it is needed.
constexpr int kPpSlots = 3;

__device__ inline void block_sync_lds() {
  // LDS reads of this wave are complete and every wave has arrived; the
  // tile copies (vmcnt) are waited for separately where a tile is published.
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <typename T, int D>
__global__ __launch_bounds__(512, 1) void prefill_pp_kernel(PrefillArgs a) {
  using MM = Mfma<T>;
  typedef typename MM::v8 v8;
  constexpr int BN = 64, KCH = D / 8, DC = D / 16, DB = D / 32, RB = 2;
  constexpr int ROW_B = D * 2;                  // bytes per K/V row
  constexpr int TILE_B = BN * ROW_B;            // bytes per K or V tile
  constexpr int SLOT_B = 2 * TILE_B;            // K tile | V tile
  constexpr int NI = TILE_B / 1024 / 8;         // 1 KB copies per wave per K (V) tile
  static_assert(NI >= 1 && NI * 8 * 1024 == TILE_B, "tile must split into 1 KB wave copies");
  extern __shared__ __align__(16) unsigned char smem_raw[];
  unsigned char* const lds = smem_raw;

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int grp = w >> 2, wi = w & 3;
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
  const int rows_pb = 2 * 32 * RB * PJ;         // two groups of PJ 64-row slices
  const int p0 = pb * rows_pb;

  const int g = wi % GH, j = wi / GH;
  const int head = kvh * a.G + hc * GH + g;
  const int qpos0 = p0 + 32 * RB * (grp * PJ + j);  // first query row of this wave
  const bool wave_active = qpos0 < a.S;

  // ---- Q as the B operand of S^T = K Q^T (lane: row lr of each row block)
  v8 qreg[RB][DC];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int qrow = qpos0 + 32 * rb + lr;
    const T* qp = reinterpret_cast<const T*>(a.q) + (int64_t)b * a.q_sb +
                  (int64_t)head * a.q_sh + (int64_t)min(qrow, a.S - 1) * a.q_ss;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      u32x4 raw = load16(qp + 16 * c + 8 * hh);
      if (qrow >= a.S) raw = u32x4{0, 0, 0, 0};
      qreg[rb][c] = __builtin_bit_cast(v8, raw);
    }
  }

  // ---- tile copies: wave w copies 1 KB pieces (w*NI + i) of each tile
  const unsigned char* kbase = reinterpret_cast<const unsigned char*>(a.k) +
                               ((int64_t)b * a.k_sb + (int64_t)kvh * a.k_sh) * 2;
  const unsigned char* vbase = reinterpret_cast<const unsigned char*>(a.v) +
                               ((int64_t)b * a.v_sb + (int64_t)kvh * a.v_sh) * 2;
  int dma_row[NI], k_lc[NI], v_lc[NI];
  uint32_t k_goff[NI], v_goff[NI];
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
  auto issue = [&](int t, int slot) {
    const int r0 = t * BN;
    const uint32_t kl = lds0 + slot * SLOT_B, vl = kl + TILE_B;
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

  // ---- per-lane operand read offsets (bytes, within one slot)
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
    v_rd[q8] = TILE_B + r * ROW_B + (((d0 >> 3) ^ v_swz(r)) * 16) + (d0 & 7) * 2;
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
  f32x16 s[RB][2];
  v8 pbuf[RB][4];

  // S^T = K Q^T for one tile (both row blocks; every K operand feeds RB MFMAs)
  auto qk = [&](const unsigned char* sp) {
    v8 ka[2][DC];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
      for (int c = 0; c < DC; ++c)
        ka[sb][c] = __builtin_bit_cast(
            v8, *reinterpret_cast<const u32x4*>(sp + k_rd[c] + sb * 32 * ROW_B));
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int i = 0; i < 16; ++i) s[rb][sb][i] = 0.f;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
      for (int c = 0; c < DC; ++c)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) s[rb][sb] = MM::mma(ka[sb][c], qreg[rb][c], s[rb][sb]);
  };
  // O^T += V^T P^T for one tile (every V operand feeds RB MFMAs)
  auto pv = [&](const unsigned char* sp) {
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4)
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const uint2 lo = lds_read_tr(sp + v_rd[2 * q4] + db * 64);
        const uint2 hi = lds_read_tr(sp + v_rd[2 * q4 + 1] + db * 64);
        const v8 vv = __builtin_bit_cast(v8, u32x4{lo.x, lo.y, hi.x, hi.y});
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) o[rb][db] = MM::mma(vv, pbuf[rb][q4], o[rb][db]);
      }
  };
  // online softmax of one tile's scores: s -> pbuf, running m / l, O rescale
  auto softmax = [&](int kpos) {
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
        pbuf[rb][cc] = __builtin_bit_cast(v8, u32x4{w0[0], w0[1], w0[2], w0[3]});
        pbuf[rb][2 + cc] = __builtin_bit_cast(v8, u32x4{w1[0], w1[1], w1[2], w1[3]});
      }
      l[rb] += ls0 + ls1;
    }
  };

  // Phase schedule (one barrier after each phase):
  //   phase 2t   : copy tile t+1 | A: PV(t-1), QK(t) | B: softmax(t-1)
  //   phase 2t+1 :                 A: softmax(t)     | B: PV(t-1), QK(t)
  //   phase 2n   : A: PV(n-1) | B: softmax(n-1);  phase 2n+1: B: PV(n-1)
  // A tile is live for a wave iff it holds a key visible to one of its rows.
  issue(0, 0);
  dma_wait_all();
  block_sync_lds();
  const int last_q = qpos0 + 32 * RB - 1;
  bool live_prev = false;
  int slot = 0, slot_prev = 0;
  for (int t = 0; t < n_tiles; ++t) {
    const bool live = wave_active && t * BN <= last_q;
    const int slot_next = slot == kPpSlots - 1 ? 0 : slot + 1;
    if (t + 1 < n_tiles) issue(t + 1, slot_next);
    const unsigned char* cur = lds + slot * SLOT_B;
    const unsigned char* prev = lds + slot_prev * SLOT_B;
    if (grp == 0) {
      __builtin_amdgcn_s_setprio(1);
      if (live_prev) pv(prev);
      if (live) qk(cur);
      __builtin_amdgcn_s_setprio(0);
    } else if (live_prev) {
      softmax((t - 1) * BN);
    }
    block_sync_lds();
    if (grp == 0) {
      if (live) softmax(t * BN);
    } else {
      __builtin_amdgcn_s_setprio(1);
      if (live_prev) pv(prev);
      if (live) qk(cur);
      __builtin_amdgcn_s_setprio(0);
    }
    dma_wait_all();
    block_sync_lds();
    live_prev = live;
    slot_prev = slot;
    slot = slot_next;
  }
  {
    const unsigned char* prev = lds + slot_prev * SLOT_B;
    if (grp == 0) {
      if (live_prev) pv(prev);
    } else if (live_prev) {
      softmax((n_tiles - 1) * BN);
    }
    block_sync_lds();
    if (grp == 1 && live_prev) pv(prev);
  }

  if (!wave_active) return;
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
  const int n_pairs = a.B * a.Hkv * a.head_chunks;
  dim3 grid((unsigned)(n_pairs * a.n_pb));
  dim3 block((unsigned)(nwaves * 64));
  const size_t smem = 2 * 2 * 64 * D * sizeof(T);  // 2 buffers x (K + V) tiles
  hipLaunchKernelGGL((prefill_kernel<T, D>), grid, block, smem, stream, a);
  return hipGetLastError();
}

template <typename T, int D>
hipError_t launch_pp(const PrefillArgs& a, hipStream_t stream) {
  const int n_pairs = a.B * a.Hkv * a.head_chunks;
  dim3 grid((unsigned)(n_pairs * a.n_pb));
  const size_t smem = (size_t)kPpSlots * 2 * 64 * D * sizeof(T);  // ring of (K + V) tiles
  hipLaunchKernelGGL((prefill_pp_kernel<T, D>), grid, dim3(512), smem, stream, a);
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
  // D = 64 (16-bit): ping-pong kernel, two groups of 4 waves, 64 rows per
  // wave; D = 128: one group of 4 waves, 32 rows per wave.
  const bool pp = head_dim == 64 && dtype != MI_DTYPE_F32;
  const int rows_per_block = pp ? 2 * 64 * pj : 32 * prefill_row_blocks<128>() * pj;
  a.n_pb = (int32_t)((seq_len + rows_per_block - 1) / rows_per_block);
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
    e = pp ? launch_pp<bf16_t, 64>(a, st) : launch<bf16_t, 128>(a, nwaves, st);
  else
    e = pp ? launch_pp<f16_t, 64>(a, st) : launch<f16_t, 128>(a, nwaves, st);
  if (e != hipSuccess) {
    set_last_error("attn_prefill: launch failed: %s", hipGetErrorString(e));
    return (int32_t)e;
  }
  return MI_OK;
}
