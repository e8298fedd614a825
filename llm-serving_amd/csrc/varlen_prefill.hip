// Packed varlen causal prefill attention on gfx950 bf16/fp16 MFMA.
//
// Replaces FlashVarlen.prefill_varlen's FA2 call (reference model/attention/varlen.py:
// 317-357): causal attention inside each cu_seqlens segment of a packed (total, H, D)
// token axis, GQA head h -> KV head h / (H / H_kv), softmax scale applied to the fp32
// scores. FlashAttention-2 style: one pass over K/V tiles with an fp32 online softmax.
//
// MI355X shape of the computation:
//   * a workgroup (4 waves) owns 64 query rows of one head of one packed segment. Wave w
//     takes query block w & 1 (32 rows) and key half w >> 1 of every 64-key tile, so the
//     serial chain of the longest causal tile is half its keys; the two key halves of a
//     query block are folded at the end through LDS (log-sum-exp merge);
//   * K and V tiles are double-buffered in LDS: the next tile's global loads are issued
//     before the current tile's MFMAs and land in registers, which are written to the
//     other buffer afterwards, so one barrier per tile remains. K is stored row-major; V
//     is stored transposed (V^T[d][key]) through a 4x8 register transpose and 8-byte LDS
//     writes, which is the operand layout the PV product needs;
//   * scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16 (A = K from
//     LDS, B = Q held in VGPRs for the whole loop). In the 32x32 accumulator layout each
//     lane then owns one query column, so the row max needs one cross-lane exchange
//     (lane ^ 32) and the row sum none until the end;
//   * O^T = V^T P^T with the same MFMA: P^T comes straight from the score registers
//     (packed to bf16), the A operand is two 8-byte LDS reads per lane, and the key order
//     inside a 16-key MFMA step is permuted identically on both operands to match the
//     score accumulator layout;
//   * causal tiles above the diagonal are never loaded; the diagonal tile is masked;
//   * grid = (head, schedule entry), entries ordered heaviest-first; heads are permuted so
//     the query heads of one KV head are dispatched to the same XCD and its K/V tiles are
//     served from that XCD's L2.
#include <algorithm>
#include <climits>
#include <type_traits>
#include <vector>

#include "common.h"

namespace miattn {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));

constexpr int kBQ = 64;  // query rows per workgroup (two blocks of 32)
constexpr int kXcds = 8; // MI355X: 8 XCDs, workgroups dispatched round-robin over them
// Schedule layout (int32 words): {n_work, n_merge, n_partials, layout = head_dim << 8 |
// query rows per tile}, then n_work work entries and n_merge merge entries of two words
// each (see mi_varlen_schedule). 128-row tiles run the ring kernel, 64-row tiles the
// register-staged kernel.
constexpr int kSchedHeader = 4;
// The ring kernel is chosen when the longest segment reaches this many tokens: measured on
// MI355X (H16/H_kv8/D128 bf16, causal) the duo kernel is faster up to 6144 tokens (30.0
// against 39.3 us at 2048, 84.4 against 87.0 us at 4096, 187 against 195 us at 6144, and
// 42.0 against 31.7 us on the config-3 batch); the ring kernel's 128-row tiles are 2%
// faster at 8192 and 4% at 16384 tokens.
constexpr int kRingMinLen = 8192;
// The tall kernel is chosen (head_dim 64/128) when the longest segment reaches this many
// tokens and its schedule deals the batch out without splitting any tile: measured on
// MI355X (H16/H_kv8/D128 bf16, causal), 8 x 1536 tokens 105.0 against 107.6 us for the duo
// kernel, 8 x 2048 168.4 against 177.3, 4 x 4096 292.8 against 309.0, 8192 272.7 against
// 295.4 (ring 305.9), 16384 1046.5 against 1134.3 (ring 1155.6); 16 x 1024 112.3 against
// 110.1. Where its schedule has to split tiles to fill the chip (2 x 2048: 70.7 against
// 47.1 us; the config-3 batch: 44.4 against 32.2) the other kernels stay the choice.
constexpr int kTallMinLen = 1536;
#ifndef MIATTN_PREFILL_SPLIT
#define MIATTN_PREFILL_SPLIT 1
#endif

// K/V tiles in flight in registers while a tile is computed: 1 (tile it+1) or 2 (it+1 and
// it+2; twice the staging registers).
#ifndef MIATTN_PREFILL_DEPTH
#define MIATTN_PREFILL_DEPTH 1
#endif
constexpr int kDepth = MIATTN_PREFILL_DEPTH;

__device__ __forceinline__ floatx16 zero16() {
  floatx16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

template <typename T>
__device__ __forceinline__ floatx16 mfma32(const uint4& a, const uint4& b, const floatx16& c) {
  if constexpr (std::is_same<T, bf16_t>::value) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(halfx8, a),
                                                  __builtin_bit_cast(halfx8, b), c, 0, 0, 0);
  }
}

// Two fp32 values -> one word of two 16-bit values, round to nearest even; one
// v_cvt_pk_bf16_f32 on gfx950 for bf16.
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (std::is_same<T, bf16_t>::value) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
  } else {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    const f16x2_t v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, v);
  }
}

// V^T tile: D rows of BK keys (BK/8 slots of 16 B), no padding. Within each 16-key
// MFMA step the 4-key groups are stored in the order [0, 2, 1, 3], so the 8 keys one lane
// feeds to the PV MFMA (keys 4g..4g+3 and 8+4g..8+4g+3 of the step, the score
// accumulator's layout) are one contiguous 16-byte slot; slots are XOR-swizzled by row so
// the transposing 8-byte writes are at most 2-way bank-conflicted and the 16-byte operand
// reads are conflict-free.
template <int BK>
__device__ __forceinline__ int vt_offset(int d, int grp) {  // element offset of a 4-key group
  const int gp = (grp & ~3) | ((grp & 1) << 1) | ((grp >> 1) & 1);
  const int slot = (gp >> 1) ^ ((d ^ (d >> 3)) & 7);
  return d * BK + slot * 8 + (gp & 1) * 4;
}

// NKS waves share each query block, each taking 32 keys of a BK = 32*NKS tile, so the
// serial chain of the longest causal tile is L / (32*NKS) tiles. NKS = 2 (4 waves, two
// 64-key LDS buffers, 2 workgroups per CU at D = 128) measured faster on config 3 than
// NKS = 4 (8 waves, 128-key tiles, one workgroup per CU: 57.6 vs 39.5 us per layer),
// because two independent workgroups overlap each other's barrier and staging phases.
#ifndef MIATTN_PREFILL_NKS
#define MIATTN_PREFILL_NKS 2
#endif
template <int D>
struct Tiles {
  static constexpr int NKS = D <= 128 ? MIATTN_PREFILL_NKS : 2;  // key splits per tile
  static constexpr int THREADS = 64 * 2 * NKS;  // 2 query blocks x NKS key splits
  static constexpr int BK = 32 * NKS;           // keys per tile
  static constexpr int KST = D + 8;             // K tile row stride (elements): 16 B skew
  static constexpr int KTILE = BK * KST;        // elements
  static constexpr int VTILE = D * BK;
  static constexpr int BUF = KTILE + VTILE;
  static constexpr int KCH = BK * D / 8 / THREADS;                 // 16-byte K chunks per thread
  static constexpr int VPAIRS = (BK / 4) * (D / 8);                // (4 keys x 8 d) blocks of V
  static constexpr int VPT = (VPAIRS + THREADS - 1) / THREADS;     // blocks per thread
  static_assert(KCH >= 1 && (BK * D / 8) % THREADS == 0, "K staging assumes whole chunks");
};

template <typename T, int D>
__global__ __launch_bounds__(Tiles<D>::THREADS, D <= 128 && Tiles<D>::NKS == 2 ? 2 : 1) void varlen_prefill_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    T* __restrict__ out, const int32_t* __restrict__ cu, const int32_t* __restrict__ sched,
    int H, int H_kv, int G, float scale_log2, int causal) {
  using Tl = Tiles<D>;
  constexpr int kThreads = Tl::THREADS, kBK = Tl::BK, NKS = Tl::NKS;
  constexpr int KS = D / 16;  // MFMA k-steps over D for S^T
  constexpr int DB = D / 32;  // 32-row blocks of D for O^T
  constexpr int KST = Tl::KST;
  __shared__ __align__(16) uint16_t lds[2 * Tl::BUF];

  // Head permutation: x -> h so that x % 8 (the XCD) selects a block of consecutive heads.
  const int x = blockIdx.x;
  const int h = (H % kXcds == 0) ? (x % kXcds) * (H / kXcds) + x / kXcds : x;
  const int kvh = h / G;
  const int entry = sched[2 * blockIdx.y];  // (seq, tile); this kernel's entries are never split
  const int seq = int(uint32_t(entry) >> 16);
  const int tile = entry & 0xffff;
  const int seq0 = cu[seq];
  const int L = cu[seq + 1] - seq0;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int qb = wave & 1;    // query block of this wave
  const int kh = wave >> 1;   // key split (32 keys) of every tile
  const int g = lane >> 5;    // k-group of the MFMA operands
  const int col = lane & 31;  // query column owned by this lane
  const int qrow0 = tile * kBQ + qb * 32;
  const int qi = qrow0 + col;  // local query index

  const int64_t q_row = int64_t(H) * D;
  const int64_t kv_row = int64_t(H_kv) * D;

  // Q^T as the B operand: lane holds Q[qi][ks*16 + 8g .. +8] for every k-step.
  uint4 qB[KS];
  {
    const int qc = qi < L ? qi : L - 1;
    const T* qp = q + int64_t(seq0 + qc) * q_row + h * D + g * 8;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qB[ks] = load16(qp + ks * 16);
  }

  // Loop-invariant LDS offsets of this lane's V^T operand slots (keys kh*32 + 16t +
  // {4g..4g+3, 8+4g..8+4g+3} of D row db*32 + col; see vt_offset).
  int vt_rd[DB][2];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
#pragma unroll
    for (int t = 0; t < 2; ++t) vt_rd[db][t] = vt_offset<kBK>(db * 32 + col, kh * 8 + t * 4 + g);
  }

  const int q_end = min(L, tile * kBQ + kBQ);
  const int n_it = causal ? (q_end + kBK - 1) / kBK : (L + kBK - 1) / kBK;

  // ---- tile staging: global -> registers (issued early) -> LDS (after the MFMAs)
  uint4 kreg[kDepth][Tl::KCH];
  uint4 vreg[kDepth][Tl::VPT][4];
  // K/V tiles are read with buffer loads: one scalar resource per tile whose base is the
  // tile's first token and whose size ends at the segment's last token, so each lane's
  // byte offset is a constant for the whole loop and keys past the segment read as zero
  // (range-checked by the hardware; they are masked out of the softmax anyway).
  const int row_b = int(kv_row) * 2;  // bytes per packed token (all KV heads)
  int koff[Tl::KCH];
#pragma unroll
  for (int c = 0; c < Tl::KCH; ++c) {
    const int idx = c * kThreads + tid;
    const int key = idx / (D / 8), cc = idx - key * (D / 8);
    koff[c] = key * row_b + kvh * D * 2 + cc * 16;
  }
  int voff[Tl::VPT];
#pragma unroll
  for (int p = 0; p < Tl::VPT; ++p) {
    const int pr = p * kThreads + tid;
    const int kq = pr / (D / 8), dq = pr - kq * (D / 8);
    voff[p] = kq * 4 * row_b + kvh * D * 2 + dq * 16;
  }
  auto tile_rsrc = [&](const T* base, int key0) {
    return __builtin_amdgcn_make_buffer_rsrc(
        const_cast<T*>(base + int64_t(seq0 + key0) * kv_row), (short)0, (L - key0) * row_b,
        0x00020000);
  };
  // The register set is a compile-time index: a runtime index would make the compiler
  // select between the sets right after each load and wait for the data there.
  auto load_tile = [&](int it, auto set_c) {
    constexpr int set = decltype(set_c)::value;
    const int key0 = it * kBK;
    const auto rk = tile_rsrc(k, key0);
    const auto rv = tile_rsrc(v, key0);
#pragma unroll
    for (int c = 0; c < Tl::KCH; ++c) {
      kreg[set][c] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, koff[c], 0, 0));
    }
#pragma unroll
    for (int p = 0; p < Tl::VPT; ++p) {
      const int pr = p * kThreads + tid;
      if (Tl::VPAIRS % kThreads == 0 || pr < Tl::VPAIRS) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          vreg[set][p][j] = __builtin_bit_cast(
              uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, voff[p] + j * row_b, 0, 0));
        }
      }
    }
  };
  auto store_tile = [&](int buf, auto set_c) {
    constexpr int set = decltype(set_c)::value;
    uint16_t* Ks = lds + buf * Tl::BUF;
    uint16_t* Vt = Ks + Tl::KTILE;
#pragma unroll
    for (int c = 0; c < Tl::KCH; ++c) {
      const int idx = c * kThreads + tid;
      const int key = idx / (D / 8), cc = idx - key * (D / 8);
      *reinterpret_cast<uint4*>(&Ks[key * KST + cc * 8]) = kreg[set][c];
    }
#pragma unroll
    for (int p = 0; p < Tl::VPT; ++p) {
      const int pr = p * kThreads + tid;
      if (Tl::VPAIRS % kThreads == 0 || pr < Tl::VPAIRS) {
        const int kq = pr / (D / 8), dq = pr - kq * (D / 8);
        const uint4* vr = vreg[set][p];
        const uint32_t w[4][4] = {{vr[0].x, vr[0].y, vr[0].z, vr[0].w},
                                  {vr[1].x, vr[1].y, vr[1].z, vr[1].w},
                                  {vr[2].x, vr[2].y, vr[2].z, vr[2].w},
                                  {vr[3].x, vr[3].y, vr[3].z, vr[3].w}};
        // word m of key j holds d = 2m (low half) and 2m+1 (high half); V^T row d gets
        // the four keys' values of d as two words.
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const uint2 even = make_uint2((w[0][m] & 0xffffu) | (w[1][m] << 16),
                                        (w[2][m] & 0xffffu) | (w[3][m] << 16));
          const uint2 odd = make_uint2((w[0][m] >> 16) | (w[1][m] & 0xffff0000u),
                                       (w[2][m] >> 16) | (w[3][m] & 0xffff0000u));
          const int d0 = dq * 8 + 2 * m;
          *reinterpret_cast<uint2*>(&Vt[vt_offset<kBK>(d0, kq)]) = even;
          *reinterpret_cast<uint2*>(&Vt[vt_offset<kBK>(d0 + 1, kq)]) = odd;
        }
      }
    }
  };

  floatx16 o[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i) o[i] = zero16();
  float m_i = -INFINITY;
  float l_i = 0.0f;

  // Tile it+1 and it+2 are in flight in the two register sets while tile it is computed
  // from LDS; tile it+1 is written to the other LDS buffer after the MFMAs.
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  load_tile(0, S0{});
  store_tile(0, S0{});
  // Consume the Q fragments here, before the loop: otherwise their loads can still be in
  // flight at the loop header, and the in-order load counter then makes every score MFMA
  // of every tile wait for that tile's K/V prefetch. (An empty asm that reads the
  // registers; the compiler places the wait for the Q loads in front of it.)
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) asm volatile("" ::"v"(qB[ks].x), "v"(qB[ks].y), "v"(qB[ks].z), "v"(qB[ks].w));
  if constexpr (kDepth == 2) {
    if (n_it > 1) load_tile(1, S1{});
    if (n_it > 2) load_tile(2, S0{});
  }
  __syncthreads();

  // One tile: compute tile `it` from LDS buffer it & 1 while tile it+1 (and, at depth 2,
  // it+2) is in flight in registers, then move tile it+1 into the other buffer. At depth 2
  // the register set (it+1) & 1 is then reused for tile it+3.
  auto step = [&](int it, auto set_c) {
    const bool more = it + 1 < n_it;
    if constexpr (kDepth == 1) {
      if (more) load_tile(it + 1, S0{});
    }
    const int kb0 = it * kBK + kh * 32;  // first key of this wave's split
    const bool live = kb0 < L && !(causal && kb0 > qrow0 + 31);
    if (live) {
      const uint16_t* Ks = lds + (it & 1) * Tl::BUF;
      const uint16_t* Vt = Ks + Tl::KTILE;
      // S^T[key][query] for the wave's 32 keys: all K fragments first, then the MFMAs.
      uint4 kf[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        kf[ks] = *reinterpret_cast<const uint4*>(&Ks[(kh * 32 + col) * KST + ks * 16 + g * 8]);
      }
      floatx16 sacc = zero16();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) sacc = mfma32<T>(kf[ks], qB[ks], sacc);
      // V^T fragments of the PV product, read now so they arrive during the softmax.
      uint4 vf[DB][2];
#pragma unroll
      for (int db = 0; db < DB; ++db) {
#pragma unroll
        for (int t = 0; t < 2; ++t) vf[db][t] = *reinterpret_cast<const uint4*>(&Vt[vt_rd[db][t]]);
      }
      // Online softmax for this lane's query column, in raw score units: the scale is
      // applied once to the max and folded into the exp2 argument (one FMA per score).
      // Only boundary tiles (segment end, causal diagonal) need the mask.
      const bool interior = kb0 + 31 < L && !(causal && kb0 + 31 > qrow0);
      if (!interior) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int key = kb0 + (j >> 2) * 8 + g * 4 + (j & 3);
          if (key >= L || (causal && key > qi)) sacc[j] = -INFINITY;
        }
      }
      float mloc = sacc[0];
#pragma unroll
      for (int j = 1; j < 16; ++j) mloc = fmaxf(mloc, sacc[j]);
      const float m_tile = max_halves(mloc) * scale_log2;
      const float m_new = fmaxf(m_i, m_tile);
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      // Rescale the accumulators only when some lane's running max moved (a wave-wide
      // vote); with a settled max the 4*DB*4 multiplies are skipped.
      if (__any(m_new != m_i)) {
        const float alpha = fast_exp2(m_i - m_use);
        l_i *= alpha;
#pragma unroll
        for (int i = 0; i < DB; ++i) o[i] *= alpha;
      }
      m_i = m_new;
      float lsum = 0.0f;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float p = fast_exp2(fmaf(sacc[j], scale_log2, -m_use));
        sacc[j] = p;
        lsum += p;
      }
      l_i += lsum;
      // P^T as the B operand: k-step t covers keys 16t..16t+15 and the lane's 8 values are
      // sacc[8t .. 8t+8] (keys 4g+0..3 and 8+4g+0..3 of that step).
      uint4 pB[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        pB[t] = make_uint4(pack2<T>(sacc[8 * t + 0], sacc[8 * t + 1]),
                           pack2<T>(sacc[8 * t + 2], sacc[8 * t + 3]),
                           pack2<T>(sacc[8 * t + 4], sacc[8 * t + 5]),
                           pack2<T>(sacc[8 * t + 6], sacc[8 * t + 7]));
      }
#pragma unroll
      for (int db = 0; db < DB; ++db) {
#pragma unroll
        for (int t = 0; t < 2; ++t) o[db] = mfma32<T>(vf[db][t], pB[t], o[db]);
      }
    }
    if (more) {
      if constexpr (kDepth == 1) {
        store_tile((it + 1) & 1, S0{});
      } else {
        store_tile((it + 1) & 1, set_c);
        if (it + 3 < n_it) load_tile(it + 3, set_c);
      }
    }
    __syncthreads();
  };
  if constexpr (kDepth == 1) {
    for (int it = 0; it < n_it; ++it) step(it, S0{});
  } else {
    for (int it = 0; it < n_it; it += 2) {
      step(it, S1{});
      if (it + 1 < n_it) step(it + 1, S0{});
    }
  }

  // Fold the NKS key splits of each query block: the waves with kh > 0 publish
  // (m, l, O^T) through LDS, the kh = 0 waves merge, normalise and store.
  const float l_tot = sum_halves(l_i);
  constexpr int NE = DB * 16 + 2;
  float* mbuf = reinterpret_cast<float*>(lds);  // [qb][kh-1][NE][64]
  if (kh > 0) {
    float* mine = mbuf + (qb * (NKS - 1) + kh - 1) * NE * 64;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int j = 0; j < 16; ++j) mine[(db * 16 + j) * 64 + lane] = o[db][j];
    }
    mine[(DB * 16) * 64 + lane] = m_i;
    mine[(DB * 16 + 1) * 64 + lane] = l_tot;
  }
  __syncthreads();
  if (kh > 0) return;
  const float* part = mbuf + qb * (NKS - 1) * NE * 64;
  float M = m_i;
#pragma unroll
  for (int sp = 0; sp < NKS - 1; ++sp) M = fmaxf(M, part[(sp * NE + DB * 16) * 64 + lane]);
  const float M_use = M == -INFINITY ? 0.0f : M;
  const float w0 = fast_exp2(m_i - M_use);
  float wsp[NKS - 1];
  float l_all = l_tot * w0;
#pragma unroll
  for (int sp = 0; sp < NKS - 1; ++sp) {
    wsp[sp] = fast_exp2(part[(sp * NE + DB * 16) * 64 + lane] - M_use);
    l_all = fmaf(part[(sp * NE + DB * 16 + 1) * 64 + lane], wsp[sp], l_all);
  }
  const float inv = 1.0f / fmaxf(l_all, 1e-30f);
  if (qi < L) {
    T* op = out + int64_t(seq0 + qi) * q_row + h * D;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      float r[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        float acc = o[db][j] * w0;
#pragma unroll
        for (int sp = 0; sp < NKS - 1; ++sp) acc = fmaf(part[(sp * NE + db * 16 + j) * 64 + lane], wsp[sp], acc);
        r[j] = acc * inv;
      }
      // lane owns query qi and, per 32-wide D block, d = (j/4)*8 + 4g + (j%4): four runs
      // of 4 consecutive elements.
#pragma unroll
      for (int jg = 0; jg < 4; ++jg) {
        const int d = db * 32 + jg * 8 + g * 4;
        const uint2 val = make_uint2(pack2<T>(r[jg * 4 + 0], r[jg * 4 + 1]),
                                     pack2<T>(r[jg * 4 + 2], r[jg * 4 + 3]));
        *reinterpret_cast<uint2*>(op + d) = val;
      }
    }
  }
}

// ---------------------------------------------------------------- ring kernel (D = 64, 128)
// Eight waves own 128 query rows (4 blocks of 32) x the two 32-key halves of every 64-key
// tile. K and V tiles stream from global memory straight into LDS (buffer_load_dwordx4 ...
// lds, no staging registers) through a ring of four stages, so tile it+2 is in flight
// while tile it is computed and the load latency is spread over two tiles of MFMA work.
// Each 16-byte chunk of a key row lands at slot chunk ^ sw(row) (see Ring::sw), which
// keeps the K operand reads and the transposed V reads free of LDS bank conflicts. V stays
// row-major in LDS; the PV operand V^T is read with ds_read_b64_tr_b16 (lane i of a 16-lane
// group receives element i%4 of the 8 bytes addressed by lanes 4j + i/4, j = 0..3), and
// the source rows are chosen so the operand's key order matches the score accumulator.
#ifndef MIATTN_PREFILL_STAGES
#define MIATTN_PREFILL_STAGES 4
#endif
#ifndef MIATTN_RING_SCHED
#define MIATTN_RING_SCHED 0
#endif
#ifndef MIATTN_PREFILL_QPW
#define MIATTN_PREFILL_QPW 1
#endif
template <int D>
struct Ring {
  static constexpr int QB = 4;                 // query blocks of 32 rows
  static constexpr int NKS = 2;                // 32-key halves of a tile
  // Query blocks per wave: every K and V^T operand a wave reads from LDS feeds QPW
  // blocks' MFMAs. QPW = 2 runs one wave per SIMD with the O accumulators in AGPRs.
  static constexpr int QPW = MIATTN_PREFILL_QPW;
  static constexpr int QPAIRS = QB / QPW;      // query-block groups
  static constexpr int WAVES = QPAIRS * NKS;
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int BQ = 32 * QB;           // query rows per workgroup
  static constexpr int BK = 32 * NKS;          // keys per tile
  static constexpr int ROWB = D * 2;           // bytes of one key row of one KV head
  static constexpr int NCH = D / 8;            // 16-byte chunks per row
  static constexpr int TILEB = BK * ROWB;      // K (or V) bytes per tile
  static constexpr int STAGEB = 2 * TILEB;     // K then V
  static constexpr int SEGS = STAGEB / 1024;   // 1 KiB wave-wide loads per stage
  static constexpr int LPW = SEGS / WAVES;     // of them per wave
  static constexpr int RPS = 1024 / ROWB;      // key rows per wave-wide load
  static constexpr int SWB = NCH == 16 ? 4 : NCH == 8 ? 3 : 2;  // log2(NCH)
  // LDS stages of the K/V ring: tile it+1 resident while tile it is computed, and
  // NST - 2 more in flight (5 x 32 KiB = the whole 160 KiB at head_dim 128).
  static constexpr int NST = MIATTN_PREFILL_STAGES;
  static_assert(NST == 4 || NST == 5, "ring depth");
  // Slot permutation of row r: its two low bits become the top bits of the slot index.
  // Bijective on r mod NCH, so 16 consecutive rows read at one chunk hit 16 slots (K
  // operand), and 4 consecutive rows x 4 chunks read by the transposed V loads hit 16
  // slots too.
  static __device__ __forceinline__ int sw(int r) {
    return ((r & 3) << (SWB - 2)) | ((r >> 2) & ((NCH >> 2) - 1));
  }
  static_assert(SEGS % WAVES == 0 && LPW % 2 == 0, "each wave loads whole K and V segments");
  static_assert(QB * D * 16 * 4 * 2 <= 2 * STAGEB, "key-half merge fits in two stages");
};

typedef __attribute__((address_space(3))) void lds_void_t;
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4_t lds_short4_t;

// 16 bytes per lane from a buffer straight into LDS: lane l of the wave writes bytes
// [16l, 16l + 16) after `dst` (the wave-uniform address goes through M0).
__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t rsrc, lds_void_t* dst, int voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, dst, 16, voffset, 0, 0, 0);
}
// the same with a wave-uniform byte offset in soffset (one lane-offset register serves
// every load of a tile)
__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t rsrc, lds_void_t* dst, int voffset,
                                                  int soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, dst, 16, voffset, soffset, 0, 0);
}

// s_waitcnt with vmcnt = N and lgkmcnt = 0 (expcnt left alone; gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | ((N >> 4) << 14));
}
// Workgroup barrier without the release/acquire fences of __syncthreads: those would wait
// for every LDS-bound load in flight, including the tile two steps ahead. The waits that
// matter are explicit (wait_vm_lgkm0) and the memory clobber keeps LDS accesses on their
// side of the barrier. Every wave loads a share of each tile (counted in vmcnt only), so
// at each barrier of the ring and duo kernels: (1) a tile read after it was waited for, by
// every wave, for that wave's own loads of it (vmcnt(N), N = loads issued after them; they
// retire in order); (2) a buffer refilled after it is no longer read by any wave before
// it (lgkmcnt(0) in the same wait). The duo kernel's head_dim 256 steps keep both rules
// over pairs of waves instead (pair_publish / pair_wait in that kernel).
__device__ __forceinline__ void bare_barrier() { asm volatile("s_barrier" ::: "memory"); }

template <typename T, int D>
__global__ __launch_bounds__(Ring<D>::THREADS, 1) void varlen_prefill_ring_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    T* __restrict__ out, const int32_t* __restrict__ cu, const int32_t* __restrict__ sched,
    float* __restrict__ partials, int H, int H_kv, int G, float scale_log2, int causal) {
  using R = Ring<D>;
  constexpr int KS = D / 16;  // MFMA k-steps over D for S^T
  constexpr int DB = D / 32;  // 32-row blocks of D for O^T
  constexpr int NCH = R::NCH, ROWB = R::ROWB, BK = R::BK, LPW = R::LPW, WAVES = R::WAVES;
  constexpr int QPW = R::QPW;
  // Separately declared stages: the compiler's wait insertion tells their LDS-bound loads
  // apart and never holds a read of one stage for the loads into another.
  constexpr int NST = R::NST;
  __shared__ __align__(16) uint8_t st0[R::STAGEB];
  __shared__ __align__(16) uint8_t st1[R::STAGEB];
  __shared__ __align__(16) uint8_t st2[R::STAGEB];
  __shared__ __align__(16) uint8_t st3[R::STAGEB];
  __shared__ __align__(16) uint8_t st4[NST > 4 ? R::STAGEB : 16];

  const int x = blockIdx.x;
  const int h = (H % kXcds == 0) ? (x % kXcds) * (H / kXcds) + x / kXcds : x;
  const int kvh = h / G;
  // work entry: (seq << 16 | tile, split << 28 | (n_split - 1) << 24 | partial slot)
  const int entry = sched[2 * blockIdx.y];
  const int piece = sched[2 * blockIdx.y + 1];
  const int seq = int(uint32_t(entry) >> 16);
  const int tile = entry & 0xffff;
  const int split = int(uint32_t(piece) >> 28);
  const int n_split = ((piece >> 24) & 15) + 1;
  const int slot = piece & 0xffffff;
  const int seq0 = cu[seq];
  const int L = cu[seq + 1] - seq0;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qp = wave % R::QPAIRS;  // this wave's group of QPW query blocks
  const int kh = wave / R::QPAIRS;  // key half of every tile
  const int g = lane >> 5;          // k-group of the MFMA operands
  const int col = lane & 31;        // query column owned by this lane (in each block)
  int qrow0[QPW], qi[QPW];
#pragma unroll
  for (int j = 0; j < QPW; ++j) {
    qrow0[j] = tile * R::BQ + (qp * QPW + j) * 32;
    qi[j] = qrow0[j] + col;
  }

  const int64_t q_row = int64_t(H) * D;
  const int64_t kv_row_b = int64_t(H_kv) * ROWB;

  const int q_end = min(L, tile * R::BQ + R::BQ);
  const int n_all = causal ? (q_end + BK - 1) / BK : (L + BK - 1) / BK;
  // This piece's key tiles [t_first, t_end): an even share of the tile's n_all.
  const int t_first = split * n_all / n_split;
  const int t_end = (split + 1) * n_all / n_split;
  const int n_it = t_end - t_first;

  uint4 qB[QPW][KS];
#pragma unroll
  for (int j = 0; j < QPW; ++j) {
    const int qc = qi[j] < L ? qi[j] : L - 1;
    const T* qp_ = q + int64_t(seq0 + qc) * q_row + h * D + g * 8;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qB[j][ks] = load16(qp_ + ks * 16);
  }

  // Loads of one tile: wave-wide load i of this wave fills 1 KiB segment j = wave + i *
  // WAVES of the stage (the first half of the segments is K, the second V). Lane t writes
  // bytes 16t.. of the segment: key row j' * RPS + t / NCH, slot t % NCH, which holds
  // chunk slot ^ sw(row) of that row.
  int dma_off[LPW];
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    const int jj = (wave + i * WAVES) % (R::SEGS / 2);
    const int r = jj * R::RPS + lane / NCH;
    // byte offset of this lane's 16 bytes from the tile's first token
    dma_off[i] = int(r * kv_row_b) + kvh * ROWB + (((lane % NCH) ^ R::sw(r)) << 4);
  }
  const char* kseg = reinterpret_cast<const char*>(k) + int64_t(seq0) * kv_row_b;
  const char* vseg = reinterpret_cast<const char*>(v) + int64_t(seq0) * kv_row_b;
  // One buffer resource per tile and tensor: base = the tile's first token, size = up to
  // the segment's end, so rows past the segment read as zero (range-checked in hardware;
  // they are masked out of the softmax) and the lane offsets above never change.
  auto tile_rsrc = [&](const char* seg, int t) {
    // tiles past this piece (issued by the last steps so every step issues alike) get an
    // empty range: they read as zero without touching memory
    const int rem = t < t_end ? L - t * BK : 0;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(seg + int64_t(t) * BK * kv_row_b), (short)0,
                                             rem > 0 ? int(rem * kv_row_b) : 0, 0x00020000);
  };
  auto stage_ptr = [&](auto s_c) -> uint8_t* {
    constexpr int s = decltype(s_c)::value;
    return s == 0 ? st0 : s == 1 ? st1 : s == 2 ? st2 : s == 3 ? st3 : st4;
  };
  auto issue = [&](int t, auto s_c) {
    uint8_t* dst = stage_ptr(s_c);
    const auto rk = tile_rsrc(kseg, t);
    const auto rv = tile_rsrc(vseg, t);
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      buffer_load_lds16(i < LPW / 2 ? rk : rv,
                        (lds_void_t*)((__attribute__((address_space(3))) uint8_t*)dst +
                                      (wave + i * WAVES) % (R::SEGS / 2) * 1024 + (i < LPW / 2 ? 0 : R::TILEB)),
                        dma_off[i]);
    }
  };

  // Loop-invariant LDS byte offsets of this lane's operands within a stage.
  int k_rd[KS];
  {
    const int r = kh * 32 + col;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) k_rd[ks] = r * ROWB + (((ks * 2 + g) ^ R::sw(r)) << 4);
  }
  // V^T operand (A of O^T = V^T P^T), k-step t of the wave's 32 keys: the lane's 8 k
  // positions are keys 16t + 4g + {0..3} and 16t + 8 + 4g + {0..3} (the score
  // accumulator's rows). Read 1 fetches the first four: source lane l addresses key
  // 16t + 4(l/32) + (l%16)/4, d = 32db + 16((l/16)%2) + 4(l%4) .. +3; read 2 is 8 keys on.
  int v_rd[DB][2][2];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int key = kh * 32 + 16 * t + 8 * hh + 4 * g + ((lane & 15) >> 2);
        const int d0 = db * 32 + ((lane >> 4) & 1) * 16 + 4 * (lane & 3);
        v_rd[db][t][hh] = R::TILEB + key * ROWB + (((d0 >> 3) ^ R::sw(key)) << 4) + ((d0 >> 2) & 1) * 8;
      }
    }
  }

  floatx16 o[QPW][DB];
  float m_i[QPW], l_i[QPW];
#pragma unroll
  for (int j = 0; j < QPW; ++j) {
#pragma unroll
    for (int i = 0; i < DB; ++i) o[j][i] = zero16();
    m_i[j] = -INFINITY;
    l_i[j] = 0.0f;
  }

  // One step's fused block: the V^T operands of tile t, the K fragments and score MFMAs of
  // tile t+1 (into `nxt`, every K fragment feeding all QPW blocks) and the online softmax
  // of tile t (from `cur`), which does not depend on them, in one branch-free block that
  // the scheduler interleaves MFMA / VALU. MASK drops keys past the segment end and above
  // the diagonal (the boundary tiles); interior tiles skip it.
  auto fused = [&](int t, auto s_c, auto s_next_c, floatx16 (&cur)[QPW], floatx16 (&nxt)[QPW], auto mask_c,
                   uint4 (&pB)[QPW][2], uint4 (&vf)[DB][2], float (&alpha)[QPW], bool (&moved)[QPW]) {
    constexpr bool kMask = decltype(mask_c)::value;
    const uint8_t* vbase = stage_ptr(s_c);
    const uint8_t* kbase = stage_ptr(s_next_c);
    uint4 kf[KS];
    auto read_v = [&]() {
#pragma unroll
      for (int db = 0; db < DB; ++db) {
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2) {
          const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_short4_t*)((__attribute__((address_space(3))) const uint8_t*)vbase + v_rd[db][t2][0]));
          const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_short4_t*)((__attribute__((address_space(3))) const uint8_t*)vbase + v_rd[db][t2][1]));
          const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
          vf[db][t2] = make_uint4(l2.x, l2.y, h2.x, h2.y);
        }
      }
    };
    auto read_k = [&]() {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kf[ks] = *reinterpret_cast<const uint4*>(kbase + k_rd[ks]);
    };
#if MIATTN_RING_SCHED == 0
    read_v();
    read_k();
#else
    read_k();
    read_v();
#endif
#pragma unroll
    for (int j = 0; j < QPW; ++j) {
      floatx16 sacc = zero16();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) sacc = mfma32<T>(kf[ks], qB[j][ks], sacc);
      nxt[j] = sacc;
    }

    const int kb0 = t * BK + kh * 32;
#pragma unroll
    for (int j = 0; j < QPW; ++j) {
      floatx16 sc = cur[j];
      if constexpr (kMask) {
        const int lim = (causal ? min(L, qi[j] + 1) : L) - kb0 - g * 4;  // key offsets < lim are valid
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          if ((e >> 2) * 8 + (e & 3) >= lim) sc[e] = -INFINITY;
        }
      }
      float mloc = sc[0];
#pragma unroll
      for (int e = 1; e < 16; ++e) mloc = fmaxf(mloc, sc[e]);
      const float m_tile = max_halves(mloc) * scale_log2;
      // Lazy rescaling: the reference max moves only when some query's tile max exceeds
      // it by more than 2^8 (log2 units); until then p = 2^(s - m) stays <= 256, exact to
      // the same relative precision in fp32 and in the 16-bit P operand, and O and l keep
      // one common reference, so the final O / l is unchanged.
      moved[j] = __any(m_tile > m_i[j] + 8.0f);
      const float m_new = moved[j] ? fmaxf(m_i[j], m_tile) : m_i[j];
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      alpha[j] = fast_exp2(m_i[j] - m_use);
      m_i[j] = m_new;
#pragma unroll
      for (int e = 0; e < 16; ++e) sc[e] = fast_exp2(fmaf(sc[e], scale_log2, -m_use));
      // the row sum from the fp32 probabilities, as in the duo kernel
      float ls = l_i[j] * alpha[j];
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2) {
        pB[j][t2] = make_uint4(pack2<T>(sc[8 * t2 + 0], sc[8 * t2 + 1]), pack2<T>(sc[8 * t2 + 2], sc[8 * t2 + 3]),
                               pack2<T>(sc[8 * t2 + 4], sc[8 * t2 + 5]), pack2<T>(sc[8 * t2 + 6], sc[8 * t2 + 7]));
#pragma unroll
        for (int e = 0; e < 8; ++e) ls += sc[8 * t2 + e];
      }
      l_i[j] = ls;
    }
#if MIATTN_RING_SCHED <= 1
    // LDS reads first (V^T operands, K fragments), some vector work to cover their latency,
    // then one score MFMA per group of vector instructions.
    __builtin_amdgcn_sched_group_barrier(0x0100, 4 * DB + KS, 0);
    __builtin_amdgcn_sched_group_barrier(0x0002, 12, 0);
#pragma unroll
    for (int ks = 0; ks < KS * QPW; ++ks) {
      __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x0002, kMask ? 10 : 6, 0);
    }
#elif MIATTN_RING_SCHED == 2
    // K fragments first, softmax work while they land, V^T reads, then one score MFMA per
    // group of vector instructions.
    __builtin_amdgcn_sched_group_barrier(0x0100, KS, 0);
    __builtin_amdgcn_sched_group_barrier(0x0002, 28, 0);
    __builtin_amdgcn_sched_group_barrier(0x0100, 4 * DB, 0);
#pragma unroll
    for (int ks = 0; ks < KS * QPW; ++ks) {
      __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x0002, kMask ? 8 : 5, 0);
    }
#endif
  };

  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  using S3 = std::integral_constant<int, 3>;
  using S4 = std::integral_constant<int, 4>;
  using Yes = std::true_type;
  using No = std::false_type;
  // Tiles 0..NST-2 in flight, 0 and 1 waited for; tile 0's scores go first.
  issue(t_first, S0{});
  issue(t_first + 1, S1{});
  issue(t_first + 2, S2{});
  if constexpr (NST > 4) issue(t_first + 3, S3{});
  // Q is consumed here so its loads are not outstanding inside the loop (the loop's
  // explicit waits count only tile loads).
#pragma unroll
  for (int j = 0; j < QPW; ++j) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      asm volatile("" ::"v"(qB[j][ks].x), "v"(qB[j][ks].y), "v"(qB[j][ks].z), "v"(qB[j][ks].w));
    }
  }
  wait_vm_lgkm0<(NST - 3) * LPW>();
  bare_barrier();
  floatx16 cur[QPW], nxt[QPW];  // scores of tile it, it+1
  {
    uint4 kf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kf[ks] = *reinterpret_cast<const uint4*>(st0 + k_rd[ks]);
#pragma unroll
    for (int j = 0; j < QPW; ++j) {
      cur[j] = zero16();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) cur[j] = mfma32<T>(kf[ks], qB[j][ks], cur[j]);
    }
  }

  // Step it (tile t = t_first + it in stage it % NST with its scores in hand; tile t+1 in
  // LDS; tiles t+2.. in flight): issue tile t+NST-1 into the stage tile t-1 used; fused
  // block (scores of tile t+1, softmax of tile t); rescale O if a running max moved; PV of
  // tile t; wait for this wave's loads of tile t+2; barrier. Tiles past the piece are
  // loaded too (inside the segment they are real keys, past it they read as zero) and the
  // scores of the tile after the piece are computed and never used, so no load or MFMA of
  // a step is conditional on the trip count.
  auto step = [&](int it, auto s_c) {
    constexpr int s = decltype(s_c)::value;
    const int t = t_first + it;
    issue(t + NST - 1, std::integral_constant<int, (s + NST - 1) % NST>{});
    // workgroup-uniform: every key of tile t is valid for every query row of the tile
    const bool interior = (t + 1) * BK <= L && (!causal || (t + 1) * BK - 1 <= tile * R::BQ);
    uint4 pB[QPW][2];
    uint4 vf[DB][2];
    float alpha[QPW];
    bool moved[QPW];
    if (interior) {
      fused(t, s_c, std::integral_constant<int, (s + 1) % NST>{}, cur, nxt, No{}, pB, vf, alpha, moved);
    } else {
      fused(t, s_c, std::integral_constant<int, (s + 1) % NST>{}, cur, nxt, Yes{}, pB, vf, alpha, moved);
    }
#pragma unroll
    for (int j = 0; j < QPW; ++j) {
      if (moved[j]) {
#pragma unroll
        for (int i = 0; i < DB; ++i) o[j][i] *= alpha[j];
      }
    }
#pragma unroll
    for (int j = 0; j < QPW; ++j) {
#pragma unroll
      for (int db = 0; db < DB; ++db) {
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2) o[j][db] = mfma32<T>(vf[db][t2], pB[j][t2], o[j][db]);
      }
      cur[j] = nxt[j];
    }
    if (it + 2 < n_it) wait_vm_lgkm0<(NST - 3) * LPW>(); else wait_vm_lgkm0<(NST - 2) * LPW>();
    bare_barrier();
  };
  int it = 0;
  for (; it + NST <= n_it; it += NST) {
    step(it, S0{});
    step(it + 1, S1{});
    step(it + 2, S2{});
    step(it + 3, S3{});
    if constexpr (NST > 4) step(it + 4, S4{});
  }
  if (it < n_it) step(it, S0{});
  if (it + 1 < n_it) step(it + 1, S1{});
  if (it + 2 < n_it) step(it + 2, S2{});
  if constexpr (NST > 4) {
    if (it + 3 < n_it) step(it + 3, S3{});
  }
  // Loads past the end may still be landing in the stages the merge below reuses.
  wait_vm_lgkm0<0>();
  bare_barrier();

  // Fold the two key halves of each query block: kh = 1 waves park (O^T, m, l) in the
  // stages (all tiles are consumed and no load is in flight), kh = 0 waves merge and store.
#pragma unroll
  for (int j = 0; j < QPW; ++j) {
    const int qb = qp * QPW + j;
    const float l_tot = sum_halves(l_i[j]);
    float* obuf = reinterpret_cast<float*>(qb < 2 ? st0 : st1) + (qb & 1) * (DB * 16 * 64);
    float* mlbuf = reinterpret_cast<float*>(st2) + qb * 2 * 64;
    if (kh > 0) {
#pragma unroll
      for (int db = 0; db < DB; ++db) {
#pragma unroll
        for (int e = 0; e < 16; ++e) obuf[(db * 16 + e) * 64 + lane] = o[j][db][e];
      }
      mlbuf[lane] = m_i[j];
      mlbuf[64 + lane] = l_tot;
    }
    l_i[j] = l_tot;
  }
  __syncthreads();
  if (kh > 0) return;
#pragma unroll
  for (int j = 0; j < QPW; ++j) {
    const int qb = qp * QPW + j;
    const float* obuf = reinterpret_cast<const float*>(qb < 2 ? st0 : st1) + (qb & 1) * (DB * 16 * 64);
    const float* mlbuf = reinterpret_cast<const float*>(st2) + qb * 2 * 64;
    const float m_p = mlbuf[lane];
    const float M = fmaxf(m_i[j], m_p);
    const float M_use = M == -INFINITY ? 0.0f : M;
    const float w0 = fast_exp2(m_i[j] - M_use);
    const float w1 = fast_exp2(m_p - M_use);
    const float l_all = fmaf(mlbuf[64 + lane], w1, l_i[j] * w0);
    if (n_split > 1) {
      // this piece's (O relative to M, M, l) for the merge launch; rows past the segment
      // are written too and never read
      float* pbase = partials + (int64_t(slot + split) * H + h) * (R::BQ * (D + 2));
      const int row = qb * 32 + col;
      float* prow = pbase + row * D;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
#pragma unroll
        for (int jg = 0; jg < 4; ++jg) {
          const int d = db * 32 + jg * 8 + g * 4;
          float4 v4;
          v4.x = fmaf(obuf[(db * 16 + jg * 4 + 0) * 64 + lane], w1, o[j][db][jg * 4 + 0] * w0);
          v4.y = fmaf(obuf[(db * 16 + jg * 4 + 1) * 64 + lane], w1, o[j][db][jg * 4 + 1] * w0);
          v4.z = fmaf(obuf[(db * 16 + jg * 4 + 2) * 64 + lane], w1, o[j][db][jg * 4 + 2] * w0);
          v4.w = fmaf(obuf[(db * 16 + jg * 4 + 3) * 64 + lane], w1, o[j][db][jg * 4 + 3] * w0);
          *reinterpret_cast<float4*>(prow + d) = v4;
        }
      }
      if (g == 0) *reinterpret_cast<float2*>(pbase + R::BQ * D + row * 2) = make_float2(M, l_all);
      continue;
    }
    const float inv = 1.0f / fmaxf(l_all, 1e-30f);
    if (qi[j] < L) {
      T* op = out + int64_t(seq0 + qi[j]) * q_row + h * D;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        float r[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) r[e] = fmaf(obuf[(db * 16 + e) * 64 + lane], w1, o[j][db][e] * w0) * inv;
#pragma unroll
        for (int jg = 0; jg < 4; ++jg) {
          const int d = db * 32 + jg * 8 + g * 4;
          const uint2 val = make_uint2(pack2<T>(r[jg * 4 + 0], r[jg * 4 + 1]),
                                       pack2<T>(r[jg * 4 + 2], r[jg * 4 + 3]));
          *reinterpret_cast<uint2*>(op + d) = val;
        }
      }
    }
  }
}

// Error word codes the prefill kernels report (the first one wins; the host clears it).
constexpr int kErrTallWait = 1;  // a tall owner gave up waiting for its producers
constexpr int kErrPairWait = 2;  // a head_dim 256 duo wave gave up waiting for its partner

__device__ __forceinline__ void report(int32_t* err, int code) {
  if (err != nullptr) atomicCAS(err, 0, code);
}

// ---------------------------------------------------------------- duo kernel (D = 64, 128)
// Persistent: the grid is two workgroups per CU, and each works through its own list of
// items (a 64-row query tile, or a key-range piece of one, of one head), which the host
// schedule deals out longest-first so every workgroup ends at about the same time, each
// KV head's items on the XCD whose L2 holds that head's K and V. Four waves own the
// tile's 64 query rows (two blocks of 32) x the two 32-key halves of every 64-key step;
// the two workgroups of a CU hide each other's barrier and epilogue phases. K and V go
// straight from memory into LDS (buffer_load_dwordx4 ... lds, 16-byte chunks swizzled per
// row, V^T operands read with ds_read_b64_tr_b16) through two rings of two 64-key buffers
// (64 KiB at head_dim 128, so two workgroups fit the 160 KiB LDS). Step it computes the
// softmax of tile t (scores in registers), the scores of tile t+1 (K(t+1) resident) and PV
// of tile t (V(t) resident) while K(t+2) and V(t+1) land in the buffers K(t) and V(t-1)
// left; one barrier per step. At an item's end the two key halves of each query block fold
// through the V ring, each wave normalising and storing half of the head dims, while the
// next item's Q and first two K tiles are already on their way.
template <int D>
struct Duo {
  static constexpr int WAVES = 4;             // 2 query blocks x 2 key halves
  static constexpr int THREADS = 64 * WAVES;
  // workgroups per CU: two at head_dim 64/128; one at 256 (128 KiB of K/V buffers, and the
  // 32 x 256 O^T accumulator and Q operands need the 512 registers of a lone wave per SIMD)
  static constexpr int PER_CU = D == 256 ? 1 : 2;
  static constexpr int BQ = 64;               // query rows per item
  static constexpr int BK = 64;               // keys per step
  static constexpr int ROWB = D * 2;          // bytes of one key row of one KV head
  static constexpr int NCH = D / 8;           // 16-byte chunks per row
  static constexpr int BUFB = BK * ROWB;      // bytes of one K (or V) buffer
  static constexpr int SEGS = BUFB / 1024;    // 1 KiB wave-wide loads per buffer
  static constexpr int LPW = SEGS / WAVES;    // of them per wave
  static constexpr int RPS = 1024 / ROWB;     // key rows per wave-wide load
  static constexpr int SWB = NCH >= 16 ? 4 : 3;
  // rows after which the swizzle repeats (it permutes the low SWB bits of the chunk index:
  // the 64 banks cover 256 bytes, so a 512-byte row's two halves alias)
  static constexpr int SW_PERIOD = 1 << SWB;
  // wave-wide loads i and i + LOAD_PERIOD of a wave land rows a whole swizzle period apart,
  // so their lane offsets differ by a constant
  static constexpr int LOAD_PERIOD = (WAVES * RPS) % SW_PERIOD == 0 ? 1 : SW_PERIOD / (WAVES * RPS);
  static constexpr int ITEM_WORDS = 4;        // {seq0, L, tile << 16 | split << 8 | n_split - 1, h << 24 | slot}
  // a workgroup's table entry: {first item word, item count, its first item's words, 0, 0},
  // so that a fresh workgroup reads its first item in the same round trip as its entry
  static constexpr int ENTRY_WORDS = 8;
  static_assert(D == 64 || D == 128 || D == 256, "duo kernel head dims");
  static_assert(SEGS % WAVES == 0 && LPW % LOAD_PERIOD == 0 && (WAVES * RPS * LOAD_PERIOD) % SW_PERIOD == 0,
                "whole loads per wave, swizzle periodic in the loads");
  static_assert(2 * (D / 32) * 16 * 64 * 4 <= 2 * BUFB, "fold fits the V ring");
  static constexpr __host__ __device__ int sw(int r) {
    return ((r & 3) << (SWB - 2)) | ((r >> 2) & ((1 << (SWB - 2)) - 1));
  }
};

// s_waitcnt lgkmcnt(0) alone (vmcnt and expcnt left at their maximum).
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14)); }

template <typename T, int D>
__global__ __launch_bounds__(Duo<D>::THREADS, Duo<D>::PER_CU) void varlen_prefill_duo_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    T* __restrict__ out, const int32_t* __restrict__ sched, float* __restrict__ partials, int H, int H_kv,
    int G, float scale_log2, int causal, int32_t* __restrict__ err, int spin_max) {
  using W = Duo<D>;
  constexpr int KS = D / 16;  // MFMA k-steps over D for S^T
  constexpr int DB = D / 32;  // 32-row blocks of D for O^T
  constexpr int BK = W::BK, BQ = W::BQ, ROWB = W::ROWB, LPW = W::LPW;
  // 512-byte aligned: at head_dim 256 the operand offsets are XOR-swizzled in bits 4-8
  __shared__ __align__(512) uint8_t kb0[W::BUFB];
  __shared__ __align__(512) uint8_t kb1[W::BUFB];
  __shared__ __align__(512) uint8_t vb0[W::BUFB];
  __shared__ __align__(512) uint8_t vb1[W::BUFB];
  __shared__ float mlx[2][2][2][64];  // [key half][query block][m, l][lane]

  // every argument is loaded with the schedule pointer (left alone, the compiler loads the
  // rest after the table entry: one or two more round trips before the first DMA); at
  // head_dim 256 the tensor pointers stay lazily loaded (held from the start they push the
  // lone wave's 512 registers into spills)
  if constexpr (D != 256) asm volatile("" ::"s"(q), "s"(k), "s"(v), "s"(out), "s"(partials));
  asm volatile("" ::"s"(H), "s"(H_kv), "s"(G), "s"(scale_log2), "s"(causal));
  // this workgroup's table entry: {first word of its item list, count, item 0's words}, all
  // loaded before the first wait (left alone, the compiler waits for the count's branch)
  const int32_t* entry = sched + kSchedHeader + W::ENTRY_WORDS * blockIdx.x;
  int first = entry[0], count = entry[1];
  int iw[W::ITEM_WORDS];
#pragma unroll
  for (int j = 0; j < W::ITEM_WORDS; ++j) iw[j] = entry[2 + j];
  static_assert(W::ITEM_WORDS == 4, "the pin below names four item words");
  asm volatile("" : "+s"(first), "+s"(count), "+s"(iw[0]), "+s"(iw[1]), "+s"(iw[2]), "+s"(iw[3]));
  if (count <= 0) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qb = wave & 1;   // query block
  const int kh = wave >> 1;  // key half of every step
  const int g = lane >> 5;
  const int col = lane & 31;
  const int64_t q_row = int64_t(H) * D;
  const int64_t kv_row_b = int64_t(H_kv) * ROWB;

  struct Item {
    int seq0, L, row0, split, n_split, slot, h, t_first, t_end;
  };
  // an item's words are loaded (scalar) while the previous item runs, decoded when needed
  // (item 0's came with the table entry)
  auto load_words = [&](int i) {
    const int32_t* w = sched + first + W::ITEM_WORDS * i;
#pragma unroll
    for (int j = 0; j < W::ITEM_WORDS; ++j) iw[j] = __builtin_amdgcn_readfirstlane(w[j]);
  };
  auto decode = [&]() {
    Item it;
    it.seq0 = iw[0];
    it.L = iw[1];
    it.row0 = int(uint32_t(iw[2]) >> 16) * BQ;
    it.split = (iw[2] >> 8) & 0xff;
    it.n_split = (iw[2] & 0xff) + 1;
    it.h = int(uint32_t(iw[3]) >> 24);
    it.slot = iw[3] & 0xffffff;
    const int q_end = min(it.L, it.row0 + BQ);
    const int n_all = causal ? (q_end + BK - 1) / BK : (it.L + BK - 1) / BK;
    it.t_first = it.split * n_all / it.n_split;
    it.t_end = (it.split + 1) * n_all / it.n_split;
    return it;
  };

  // Wave-wide load i of this wave fills 1 KiB segment wave + i * WAVES of a buffer: lane t
  // writes bytes 16t.. of it, i.e. key row (wave + i * WAVES) * RPS + t / NCH, slot t % NCH,
  // which holds chunk slot ^ sw(row) of that row; sw(row) repeats every LOAD_PERIOD loads,
  // so load i's lane offset is load i % LOAD_PERIOD's plus (i / LOAD_PERIOD) * WAVES * RPS *
  // LOAD_PERIOD rows. One buffer resource per tile: base = the tile's first token at the
  // item's KV head, range = the tile's rows inside the segment (rows past it read as zero; a
  // tile past the item reads nothing), so a step builds two resources and no per-load scalar
  // arithmetic.
  //
  // At head_dim 256 (one workgroup per CU, one wave per SIMD) the K/V tiles are loaded
  // pair-locally instead: the rows of key half kh come only from the two waves that read
  // them, (0, kh) and (1, kh), wave (qb, kh) taking segments kh * SEGS/2 + qb + 2i, so a
  // step ends with a sync of those two waves (pair_publish, pair_wait) instead of the workgroup
  // barrier that lock-steps all four (its sw(row) repeats every SW_PERIOD / (2 RPS) loads).
  constexpr bool kPairSync = D == 256;
  constexpr int LP = kPairSync ? W::SW_PERIOD / (2 * W::RPS) : W::LOAD_PERIOD;
  static_assert(!kPairSync || (LPW % LP == 0 && (W::SEGS / 2 * W::RPS) % W::SW_PERIOD == 0 &&
                               2 * LPW == W::SEGS / 2),
                "pair-local loads: whole swizzle periods, each pair covering its key half");
  auto seg_index = [&](int i) { return kPairSync ? kh * (W::SEGS / 2) + qb + 2 * i : wave + i * W::WAVES; };
  int dma_off[LP];
#pragma unroll
  for (int p = 0; p < LP; ++p) {
    const int r = seg_index(p) * W::RPS + lane / W::NCH;
    dma_off[p] = int(r * kv_row_b) + (((lane % W::NCH) ^ W::sw(r)) << 4);
  }
  const int dma_step = int((seg_index(LP) - seg_index(0)) * W::RPS * kv_row_b);
  auto issue = [&](const char* seg, const Item& it, int t, uint8_t* dst) {
    const int rows = t < it.t_end ? min(it.L - t * BK, BK) : 0;
    // the tile's byte offset as a 32 x 32 -> 64-bit unsigned product (t >= 0, and a tile's
    // bytes fit 32 bits, as its range below does): the signed 64-bit product took five
    // more scalar instructions per issue (29.6 against 29.8 us at head_dim 128, 37.1
    // against 37.7 at 256)
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(seg + uint64_t(uint32_t(t)) * uint32_t(BK * kv_row_b)), (short)0,
                                                      rows * int(kv_row_b), 0x00020000);
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      buffer_load_lds16(rs, (lds_void_t*)((__attribute__((address_space(3))) uint8_t*)dst + seg_index(i) * 1024),
                        dma_off[i % LP] + (i / LP) * dma_step);
    }
  };
  // Pair sync (head_dim 256): once its own loads of the step's tiles have landed and its
  // reads of the shared rows are done (the caller's wait, before the step's last MFMAs), a
  // wave publishes its step count in LDS (pair_publish); at the end of the step it waits
  // until its partner's count has caught up (pair_wait). Both waves of a pair run the same
  // steps, so the counts meet; the wait gives up after spin_max polls and reports that
  // through the error word (the launch then ends normally, its output not to be trusted).
  __shared__ int pflag[W::WAVES];
  int gstep = 0;
  auto pair_publish = [&]() {
    ++gstep;
    asm volatile("" ::: "memory");
    __hip_atomic_store(&pflag[wave], gstep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    asm volatile("" ::: "memory");
  };
  auto pair_wait = [&]() {
    asm volatile("" ::: "memory");
    int seen = 0;
    for (int spin = 0; spin < spin_max; ++spin) {
      seen = __builtin_amdgcn_readfirstlane(
          __hip_atomic_load(&pflag[wave ^ 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
      if (seen >= gstep) break;  // (polled without s_sleep: 43.7 against 46.3 us with it)
    }
    if (seen < gstep && lane == 0) report(err, kErrPairWait);
    asm volatile("" ::: "memory");
  };
  if constexpr (kPairSync) {
    if (tid < W::WAVES) pflag[tid] = 0;  // read after the first item's barrier
  }
  // the item's K and V at its segment's first token and its KV head
  auto seg_of = [&](const T* base, const Item& it) {
    return reinterpret_cast<const char*>(base) + int64_t(it.seq0) * kv_row_b + (it.h / G) * ROWB;
  };
  // An item's Q tile goes into LDS like a K tile (same swizzled rows, whole 16-byte chunks
  // along each row, each row loaded once per workgroup), into V buffer 1, which is idle
  // from the end of an item's fold until the next item's second step; rows past the
  // segment read as zero. Its operand reads are the K reads shifted by (qb - kh) x 32 rows
  // (sw(r) depends on r mod SW_PERIOD, which divides 32, only).
  // The lane offsets are rebuilt per call from an opaque copy of the lane id (kept live
  // through the item loop they would be spilled).
  const int64_t q_row_b = q_row * int64_t(sizeof(T));
  auto issue_q = [&](const Item& it) {
    int ql = lane;
    asm volatile("" : "+v"(ql));
    int qdma_off[LP];
#pragma unroll
    for (int p = 0; p < LP; ++p) {
      const int r = (wave + p * W::WAVES) * W::RPS + ql / W::NCH;
      qdma_off[p] = int(r * q_row_b) + (((ql % W::NCH) ^ W::sw(r)) << 4);
    }
    const int qdma_step = int(W::WAVES * W::RPS * LP * q_row_b);
    const int rows = min(it.L - it.row0, BQ);
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(reinterpret_cast<const char*>(q) + int64_t(it.seq0 + it.row0) * q_row_b + it.h * ROWB),
        (short)0, rows * int(q_row_b), 0x00020000);
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      buffer_load_lds16(rs, (lds_void_t*)((__attribute__((address_space(3))) uint8_t*)vb1 + (wave + i * W::WAVES) * 1024),
                        qdma_off[i % LP] + (i / LP) * qdma_step);
    }
  };
  static_assert(BQ == BK, "a Q tile has the layout of a K tile");
  uint4 qB[KS];

  // LDS byte offsets of this lane's operands within a buffer (as in the ring kernel): K
  // fragment of k-step ks, and the two transposed reads of each V^T operand (the second
  // 16-key k-step sits 16 rows on, which keeps sw(key), so it is a constant offset). At
  // head_dim 256 they are derived per read from three bases instead of held (32 registers
  // the lone wave per SIMD cannot spare): chunk (2 ks + g) ^ sw(r) = (g ^ sw(r)) ^ 2 ks, and
  // chunk (4 db + x) ^ sw(key) = (x ^ sw(key)) ^ 4 db, the k-step and block bits disjoint from
  // the row bits.
  constexpr bool kXorOff = D == 256;
  int k_rd[kXorOff ? 1 : KS];
  int v_rd[kXorOff ? 1 : DB][2];
  {
    const int r = kh * 32 + col;
#pragma unroll
    for (int ks = 0; ks < (kXorOff ? 1 : KS); ++ks) k_rd[ks] = r * ROWB + (((ks * 2 + g) ^ W::sw(r)) << 4);
  }
#pragma unroll
  for (int db = 0; db < (kXorOff ? 1 : DB); ++db) {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int key = kh * 32 + 8 * hh + 4 * g + ((lane & 15) >> 2);
      const int d0 = db * 32 + ((lane >> 4) & 1) * 16 + 4 * (lane & 3);
      v_rd[db][hh] = key * ROWB + (((d0 >> 3) ^ W::sw(key)) << 4) + ((d0 >> 2) & 1) * 8;
    }
  }
  static_assert(!kXorOff || (ROWB % 512 == 0 && W::SWB == 4), "XOR offsets: chunk bits 4-8 free of row bits");
  // (the bases pass through an empty asm at each use site's step: otherwise the compiler
  // hoists all the XORed offsets out of the loop and spills them)
  int kx = k_rd[0], vx0 = v_rd[0][0], vx1 = v_rd[0][1];
  auto fresh_bases = [&]() {
    if constexpr (kXorOff) {
      kx = k_rd[0];
      vx0 = v_rd[0][0];
      vx1 = v_rd[0][1];
      asm volatile("" : "+v"(kx), "+v"(vx0), "+v"(vx1));
    }
  };
  auto koff = [&](int ks) { return kXorOff ? (kx ^ (ks << 5)) : k_rd[ks]; };
  auto voff = [&](int db, int hh) { return kXorOff ? ((hh ? vx1 : vx0) ^ (db << 6)) : v_rd[db][hh]; };
  static_assert(W::sw(16) == W::sw(0) && W::sw(17) == W::sw(1), "16-row shift keeps the swizzle");

  // first item: Q, K(t0), K(t0+1) and V(t0) in flight (later items get them from the
  // previous item's epilogue)
  Item it = decode();
  const char* kseg = seg_of(k, it);
  const char* vseg = seg_of(v, it);
  issue_q(it);
  issue(kseg, it, it.t_first, kb0);
  issue(kseg, it, it.t_first + 1, kb1);
  issue(vseg, it, it.t_first, vb0);

  for (int idx = 0; idx < count; ++idx) {
    const int L = it.L;
    const int qi = it.row0 + qb * 32 + col;
    const int n_it = it.t_end - it.t_first;
    if (idx + 1 < count) load_words(idx + 1);  // used by this item's epilogue
    // Q, K(t0), K(t0+1) (and the previous item's output stores) complete
    wait_vm_lgkm0<0>();
    bare_barrier();
    floatx16 cur;
    {
      const uint8_t* qbuf = vb1 + (qb - kh) * 32 * ROWB;
      fresh_bases();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) qB[ks] = *reinterpret_cast<const uint4*>(qbuf + koff(ks));
      uint4 kf[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kf[ks] = *reinterpret_cast<const uint4*>(kb0 + koff(ks));
      cur = zero16();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) cur = mfma32<T>(kf[ks], qB[ks], cur);
    }
    wait_lgkm0();
    bare_barrier();  // every wave has read K(t0) before step 0 refills its buffer (and Q before step 1)

    floatx16 o[DB];
#pragma unroll
    for (int i = 0; i < DB; ++i) o[i] = zero16();
    float m_i = -INFINITY;
    float l_i = 0.0f;
    uint4 pB[2];  // P of the previous tile, whose PV runs in this step

    auto read_vt = [&](const uint8_t* vb, uint4 (&vf)[DB][2]) {
#pragma unroll
      for (int db = 0; db < DB; ++db) {
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2) {
          const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_short4_t*)((__attribute__((address_space(3))) const uint8_t*)vb + voff(db, 0) + t2 * 16 * ROWB));
          const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_short4_t*)((__attribute__((address_space(3))) const uint8_t*)vb + voff(db, 1) + t2 * 16 * ROWB));
          const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
          vf[db][t2] = make_uint4(l2.x, l2.y, h2.x, h2.y);
        }
      }
    };
    // Step sidx (tile t = t_first + sidx): softmax of tile t (its scores in registers), the
    // scores of tile t+1 (K(t+1) in kb_next) and PV of tile t-1 (V(t-1) in vb_prev, P(t-1)
    // from the previous step), so every MFMA of the step is independent of the step's
    // softmax; K(t+2) goes to kb_free (K(t)'s buffer) and V(t) to vb_free (V(t-2)'s). The
    // first step of an item has no PV (kPV false) and issues no V: V(t0) was issued into
    // V buffer 0 together with the item's Q. Every step runs the masked softmax: an
    // unmasked copy for interior tiles pushes the kernel past its 256 registers.
    auto step = [&](int sidx, uint8_t* kb_next, uint8_t* kb_free, const uint8_t* vb_prev, uint8_t* vb_free,
                    auto pv_c) {
      constexpr bool kPV = decltype(pv_c)::value;
      const int t = it.t_first + sidx;
      issue(kseg, it, t + 2, kb_free);
      if constexpr (kPV) issue(vseg, it, t, vb_free);  // V(t0) came with the item's Q
      // Higher wave priority from here to the end-of-step wait: when the two waves sharing a
      // SIMD (one per workgroup) both have work, the one in its MFMA/softmax section issues
      // first, which keeps the matrix pipe fed (3-4% faster than equal priorities).
      __builtin_amdgcn_s_setprio(1);
      // At head_dim 256 the K and V^T operands are read and used in NH = 2 parts (k-steps,
      // head-dim blocks), so that only half of them hold registers at once.
      constexpr int NH = D == 256 ? 2 : 1;
      constexpr int KSH = KS / NH, DBH = DB / NH;
      fresh_bases();
      uint4 kf[KSH];
      uint4 vf[DBH][2];
      auto read_part = [&](int hf) {
#pragma unroll
        for (int i = 0; i < KSH; ++i) kf[i] = *reinterpret_cast<const uint4*>(kb_next + koff(hf * KSH + i));
        if constexpr (kPV) {
#pragma unroll
          for (int i = 0; i < DBH; ++i) {
            const int db = hf * DBH + i;
#pragma unroll
            for (int t2 = 0; t2 < 2; ++t2) {
              const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                  (lds_short4_t*)((__attribute__((address_space(3))) const uint8_t*)vb_prev + voff(db, 0) + t2 * 16 * ROWB));
              const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                  (lds_short4_t*)((__attribute__((address_space(3))) const uint8_t*)vb_prev + voff(db, 1) + t2 * 16 * ROWB));
              const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
              vf[i][t2] = make_uint4(l2.x, l2.y, h2.x, h2.y);
            }
          }
        }
      };
      read_part(0);
      // online softmax of tile t (raw score units, scale folded into the exp2 argument),
      // lazy rescaling as in the ring kernel
      floatx16 sc = cur;
      // workgroup-uniform: only a tile that reaches past the segment end or the diagonal
      // needs the mask
      if ((t + 1) * BK > L || (causal && (t + 1) * BK - 1 > it.row0)) {
        // at head_dim 256 the lane's query row and key group are rebuilt here from the lane
        // id: held through the item loop they were spilled, and the scratch reload's wait
        // (loads retire in order) also waited for the step's K/V loads just issued
        int lim;  // key offsets < lim are valid
        if constexpr (D == 256) {
          const int ml = __lane_id();
          lim = (causal ? min(L, it.row0 + qb * 32 + (ml & 31) + 1) : L) - (t * BK + kh * 32) - (ml >> 5) * 4;
        } else {
          lim = (causal ? min(L, qi + 1) : L) - (t * BK + kh * 32) - g * 4;
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          if ((e >> 2) * 8 + (e & 3) >= lim) sc[e] = -INFINITY;
        }
      }
      float mloc = sc[0];
#pragma unroll
      for (int e = 1; e < 16; ++e) mloc = fmaxf(mloc, sc[e]);
      const float m_tile = max_halves(mloc) * scale_log2;
      // Each query row (lanes l and l ^ 32 hold the same one, and max_halves gave both the
      // same m_tile) moves its own reference max; the wave-wide vote only decides whether
      // the O rescale after the MFMAs runs, so the exponentials do not wait for a VALU ->
      // SALU -> VALU round trip (1.3% at head_dim 128). A row that did not move gets alpha
      // = 1 exactly, so its O is unchanged by the rescale.
      const bool mv = m_tile > m_i + 8.0f;
      const float m_new = mv ? m_tile : m_i;
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      const float alpha = fast_exp2(m_i - m_use);
      m_i = m_new;
#pragma unroll
      for (int e = 0; e < 16; ++e) sc[e] = fast_exp2(fmaf(sc[e], scale_log2, -m_use));
      const bool moved = __any(mv);
      // The row sum is taken from the fp32 probabilities, before their rounding for the PV
      // MFMA, as flash attention does. Summing the rounded ones (8 dot2) instead lowered the
      // end-to-end greedy agreement with the CPU seat path (closed case 252 against 254 of
      // 260 steps exact, trace case 1142 against 1153 of 1168), all fp32 near-ties.
      // At head_dim 256 the sum is a tree (four levels, not a chain of 16 dependent adds):
      // 37.9 against 38.4 us. At head_dim 64/128 it stays a chain: there the tree is within
      // noise and its other rounding moved the closed greedy gate (253 against 254 of 260
      // steps exact, every miss an fp32 near-tie).
      float lsum;
      if constexpr (D == 256) {
        const float q0 = (sc[0] + sc[1]) + (sc[2] + sc[3]), q1 = (sc[4] + sc[5]) + (sc[6] + sc[7]);
        const float q2 = (sc[8] + sc[9]) + (sc[10] + sc[11]), q3 = (sc[12] + sc[13]) + (sc[14] + sc[15]);
        lsum = fmaf(l_i, alpha, (q0 + q1) + (q2 + q3));
      } else {
        lsum = l_i * alpha;
#pragma unroll
        for (int e = 0; e < 16; ++e) lsum += sc[e];
      }
      // P(t) packed here, in the block of this step's MFMAs, and pinned with the row sum:
      // left alone the compiler sinks the exponentials past the end of the step, beside the
      // PV MFMAs that read P, where nothing hides them (2-3% of the kernel), and keeps the
      // fp32 probabilities live across the step's MFMAs for the sum (head_dim 256: 50.4
      // against 38.2 us)
      uint4 pN[2];
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2) {
        pN[t2] = make_uint4(pack2<T>(sc[8 * t2 + 0], sc[8 * t2 + 1]), pack2<T>(sc[8 * t2 + 2], sc[8 * t2 + 3]),
                            pack2<T>(sc[8 * t2 + 4], sc[8 * t2 + 5]), pack2<T>(sc[8 * t2 + 6], sc[8 * t2 + 7]));
      }
      asm volatile("" : "+v"(pN[0].x), "+v"(pN[0].y), "+v"(pN[0].z), "+v"(pN[0].w),
                        "+v"(pN[1].x), "+v"(pN[1].y), "+v"(pN[1].z), "+v"(pN[1].w), "+v"(lsum));
      l_i = lsum;
      floatx16 nxt = zero16();
      auto mfma_part = [&](int hf) {
#pragma unroll
        for (int i = 0; i < KSH; ++i) nxt = mfma32<T>(kf[i], qB[hf * KSH + i], nxt);
        if constexpr (kPV) {
#pragma unroll
          for (int i = 0; i < DBH; ++i) {
#pragma unroll
            for (int t2 = 0; t2 < 2; ++t2) o[hf * DBH + i] = mfma32<T>(vf[i][t2], pB[t2], o[hf * DBH + i]);
          }
        }
      };
      mfma_part(0);
      if constexpr (NH != 1) {
        // the first half's K fragment reads, 20 vector instructions of the softmax while they
        // land (28: 38.2 us), its V^T reads (37.4 against 37.6 us left free), then its 16 MFMAs each
        // followed by up to 8 vector instructions (37.1 against 37.6 us at head_dim 256; 4:
        // 37.9, 6: 37.7, 10: 37.2, 12: 37.2, 16: 39.2)
        __builtin_amdgcn_sched_group_barrier(0x0100, KSH, 0);
        __builtin_amdgcn_sched_group_barrier(0x0002, 20, 0);
        __builtin_amdgcn_sched_group_barrier(0x0100, 4 * DBH, 0);
#pragma unroll
        for (int i = 0; i < KSH + 2 * DBH; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x0002, 8, 0);
        }
      }
      if constexpr (NH == 1) {
        // K fragments first, softmax work while the reads land, V^T reads, then one MFMA per
        // group of vector instructions
        __builtin_amdgcn_sched_group_barrier(0x0100, KS, 0);
        __builtin_amdgcn_sched_group_barrier(0x0002, 20, 0);
        if constexpr (kPV) __builtin_amdgcn_sched_group_barrier(0x0100, 4 * DB, 0);
#pragma unroll
        for (int i = 0; i < (kPV ? 2 : 1) * KS; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x0002, kPV ? 5 : 9, 0);
        }
      } else {
        // the second half scheduled freely against the first half's MFMAs: behind a
        // sched_barrier the compiler read its fragments one at a time, each waited for
        // before its MFMA (43.9 against 43.4 us at head_dim 256)
        read_part(1);
        if constexpr (kPairSync) {
          // this wave's loads of the step have landed and its reads of the shared rows are
          // done: published before the half's MFMAs, so the partner waits less (41.8 against
          // 42.2 us published at the end of the step)
          wait_vm_lgkm0<0>();
          pair_publish();
        }
        mfma_part(1);
      }
      // O (with PV(t-1) added) moves to tile t's reference max
      if (moved) {
#pragma unroll
        for (int i = 0; i < DB; ++i) o[i] *= alpha;
      }
      pB[0] = pN[0];
      pB[1] = pN[1];
      cur = nxt;
      __builtin_amdgcn_s_setprio(0);
      wait_vm_lgkm0<0>();
      if constexpr (kPairSync) {
        pair_wait();
      } else {
        bare_barrier();
      }
    };
    using NoPV = std::false_type;
    using PV = std::true_type;
    step(0, kb1, kb0, vb1, vb0, NoPV{});
    int sidx = 1;
    for (; sidx + 2 <= n_it; sidx += 2) {
      step(sidx, kb0, kb1, vb0, vb1, PV{});
      step(sidx + 1, kb1, kb0, vb1, vb0, PV{});
    }
    if (sidx < n_it) step(sidx, kb0, kb1, vb0, vb1, PV{});
    // PV of the last tile, whose V landed in buffer (n_it - 1) & 1
    auto drain = [&](const uint8_t* vb) {
      fresh_bases();
      uint4 vf[DB][2];
      read_vt(vb, vf);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2) o[db] = mfma32<T>(vf[db][t2], pB[t2], o[db]);
      }
    };
    if ((n_it - 1) & 1) {
      drain(vb1);
    } else {
      drain(vb0);
    }

    // the next item's first two K tiles, in flight during this item's epilogue (its Q tile
    // follows once the fold has released V buffer 1)
    const Item cur_it = it;
    const bool more = idx + 1 < count;
    if (more) {
      it = decode();
      kseg = seg_of(k, it);
      vseg = seg_of(v, it);
      issue(kseg, it, it.t_first, kb0);
      issue(kseg, it, it.t_first + 1, kb1);
    }
    wait_lgkm0();
    bare_barrier();  // every wave has read the last V tile before the fold reuses its buffer

    // Fold the two key halves: wave (qb, kh) finalises head-dim blocks [kh * DB/2, (kh+1) *
    // DB/2) of its query block and hands its other blocks to its partner through V buffer
    // qb, as [e][lane] floats (conflict-free). Each query block's code names its buffer at
    // compile time, so the compiler sees that the fold does not touch the K buffers the
    // next item's loads are filling and does not wait for them.
    constexpr int HB = DB / 2;  // head-dim blocks each wave finalises
    // The epilogue's addresses are rebuilt here from an opaque copy of the lane id: computed
    // once before the item loop they would stay live through it and be spilled, and a
    // scratch reload waits (in order) for the next item's loads just issued.
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int e_col = ln & 31, e_g = ln >> 5;
    const float l_tot = sum_halves(l_i);
    mlx[kh][qb][0][ln] = m_i;
    mlx[kh][qb][1][ln] = l_tot;
    static_assert(DB * 16 * 64 * 4 <= W::BUFB, "a query block's fold fits one V buffer");
    // KH (this wave's key half) is a template argument so that every o[] index below is a
    // compile-time constant (a run-time block choice compiles to a chain of branches).
    auto fold_out = [&](uint8_t* fbuf_bytes, auto kh_c) {
      constexpr int KH = decltype(kh_c)::value;
      float* fbuf = reinterpret_cast<float*>(fbuf_bytes);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        if (db / HB == KH) continue;  // kept
#pragma unroll
        for (int e = 0; e < 16; ++e) fbuf[(db * 16 + e) * 64 + ln] = o[db][e];
      }
      wait_lgkm0();
      bare_barrier();
      const float m_o = mlx[KH ^ 1][qb][0][ln];
      const float l_o = mlx[KH ^ 1][qb][1][ln];
      const float M = fmaxf(m_i, m_o);
      const float M_use = M == -INFINITY ? 0.0f : M;
      const float w_me = fast_exp2(m_i - M_use);
      const float w_o = fast_exp2(m_o - M_use);
      const float l_all = fmaf(l_o, w_o, l_tot * w_me);
      const float inv = 1.0f / fmaxf(l_all, 1e-30f);
      // The normalised output goes out through LDS: the first 32 x HB * 64 bytes of this
      // wave's kept blocks in fbuf (read just above, by this wave only) take it as
      // [query row][HB * 32 dims] bf16 with 16-byte chunk c of row r at c ^ (r % NC), and
      // are read back 16 bytes per lane along the row, so each global store writes whole
      // 128-byte lines (stored straight from the MFMA layout, every lane's 8 bytes would
      // touch another row: 32 lines per instruction). The stores carry the nontemporal
      // hint: the output is not read again here, and in the XCD's L2 it would displace the
      // K and V that the following items re-read.
      constexpr int NC = HB * 4;  // 16-byte chunks of a staged row
      uint8_t* stg = fbuf_bytes + KH * HB * 16 * 64 * 4;
      // every kept block is combined before any is staged: the staging area overlaps the
      // blocks (from the second one on, when a wave keeps more than two)
      float r[HB][16];
#pragma unroll
      for (int hb = 0; hb < HB; ++hb) {
        const int db = KH * HB + hb;
#pragma unroll
        for (int e = 0; e < 16; ++e) r[hb][e] = fmaf(fbuf[(db * 16 + e) * 64 + ln], w_o, o[db][e] * w_me);
      }
#pragma unroll
      for (int hb = 0; hb < HB; ++hb) {
        const int db = KH * HB + hb;
        if (cur_it.n_split <= 1) {
#pragma unroll
          for (int jg = 0; jg < 4; ++jg) {
            // written as floats: the same bytes, in a type the compiler's LDS alias tracking
            // keeps apart from the next item's K loads in flight (it would wait for them)
            const int pos = (hb * 4 + jg) ^ (e_col & (NC - 1));
            float* f = fbuf + (KH * HB * 16 * 64 * 4 + e_col * (NC * 16) + pos * 16 + e_g * 8) / 4;
            f[0] = __builtin_bit_cast(float, pack2<T>(r[hb][jg * 4 + 0] * inv, r[hb][jg * 4 + 1] * inv));
            f[1] = __builtin_bit_cast(float, pack2<T>(r[hb][jg * 4 + 2] * inv, r[hb][jg * 4 + 3] * inv));
          }
        } else {
          // this piece's (O relative to M, M, l) for the merge launch; rows past the segment
          // are written too and never read
          float* pbase = partials + (int64_t(cur_it.slot + cur_it.split) * H + cur_it.h) * (BQ * (D + 2));
          const int row = qb * 32 + e_col;
#pragma unroll
          for (int jg = 0; jg < 4; ++jg) {
            const int d = db * 32 + jg * 8 + e_g * 4;
            *reinterpret_cast<float4*>(pbase + row * D + d) =
                make_float4(r[hb][jg * 4 + 0], r[hb][jg * 4 + 1], r[hb][jg * 4 + 2], r[hb][jg * 4 + 3]);
          }
          if (KH == 0 && hb == 0 && e_g == 0) *reinterpret_cast<float2*>(pbase + BQ * D + row * 2) = make_float2(M, l_all);
        }
      }
      if (cur_it.n_split <= 1) {
        // NC lanes per staged row, 64 / NC rows per wave-wide store
        const int c = ln & (NC - 1);
#pragma unroll
        for (int i = 0; i < NC / 2; ++i) {
          const int rr = i * (64 / NC) + ln / NC;
          const uint4 val = *reinterpret_cast<const uint4*>(stg + rr * (NC * 16) + ((c ^ (rr & (NC - 1))) << 4));
          const int qrow = cur_it.row0 + qb * 32 + rr;
          if (qrow < cur_it.L) {
            store16_nt(out + int64_t(cur_it.seq0 + qrow) * q_row + cur_it.h * D + KH * HB * 32 + c * 8, val);
          }
        }
      }
    };
    using K0 = std::integral_constant<int, 0>;
    using K1 = std::integral_constant<int, 1>;
    if (qb == 0) {
      if (kh == 0) fold_out(vb0, K0{}); else fold_out(vb0, K1{});
    } else {
      if (kh == 0) fold_out(vb1, K0{}); else fold_out(vb1, K1{});
    }
    wait_lgkm0();
    bare_barrier();  // the V ring and mlx are read before the next item refills them
    if (more) {
      issue_q(it);
      issue(vseg, it, it.t_first, vb0);
    }
  }
}

// ------------------------------------------------------------------ tall kernel
// Persistent kernel of 128-row items in which every wave owns 32 query rows over all 64
// keys of a step: wave w takes query block w, computes S^T for both 32-key blocks of the
// step and PV over its 64 keys, so no two waves share a query row and an item ends without
// a key-half fold. Each K/V tile in LDS feeds 128 query rows (the duo kernel's feed 64)
// and a batch has half as many items. Two workgroups per CU (two waves per SIMD).
//
// An item whose key range is longer than the schedule's cap is cut into pieces that run
// on different workgroups at the same time. Every piece except the one holding the
// diagonal (the owner) is a producer: it writes its (O, m, l) partial with device-scope
// stores, waits for them to be acknowledged and bumps the item's counter. The owner, after
// its own steps, waits until the counter reaches its producer count, folds the partials
// into its state, writes the output and takes its count back off the counter, so every
// counter is zero again when the launch ends. A workgroup's item list never has an owner
// before a producer and a producer never waits, so every wait ends while the grid is
// resident (one launch of at most two workgroups per CU); the wait is bounded all the
// same, and a wait that gives up is reported through the error word.
template <int D>
struct Tall {
  static constexpr int WAVES = 4;             // query blocks of 32 rows, one per wave
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int PER_CU = 2;
  static constexpr int BQ = 32 * WAVES;       // query rows per item
  static constexpr int BK = 64;               // keys per step
  static constexpr int ROWB = D * 2;          // bytes of one row of one head
  static constexpr int NCH = D / 8;           // 16-byte chunks per row
  static constexpr int BUFB = BK * ROWB;      // bytes of one K (or V) buffer
  static constexpr int SEGS = BUFB / 1024;    // 1 KiB wave-wide loads per buffer
  static constexpr int LPW = SEGS / WAVES;    // of them per wave
  static constexpr int RPS = 1024 / ROWB;     // rows per wave-wide load
  static constexpr int SWB = NCH >= 16 ? 4 : 3;
  static constexpr int SW_PERIOD = 1 << SWB;
  // wave-wide loads i and i + LOAD_PERIOD of a wave land rows a whole swizzle period apart,
  // so their lane offsets differ by a constant
  static constexpr int LOAD_PERIOD = (WAVES * RPS) % SW_PERIOD == 0 ? 1 : SW_PERIOD / (WAVES * RPS);
  // {seq0, L, tile << 16 | head, t_first << 16 | t_end, role << 30 | n_prod << 24 | counter,
  //  partial slot (a producer's own; an owner's first producer's)}
  static constexpr int ITEM_WORDS = 6;
  static constexpr int ENTRY_WORDS = 2 + ITEM_WORDS;  // {first item word, count, item 0's words}
  // one piece's partial: O^T per query block as [block][16 groups of 4 head dims][64 lanes]
  // float4 (the accumulator layout, so the owner reads back exactly what each lane wrote),
  // then (m, l) per query row as [block][32 rows] float2
  static constexpr int PART_O = BQ * D;
  static constexpr int PART_FLOATS = PART_O + 2 * BQ;
  static constexpr int ROLE_WHOLE = 0, ROLE_PRODUCER = 1, ROLE_OWNER = 2;
  static_assert(D == 64 || D == 128, "tall kernel head dims");
  static_assert(SEGS % WAVES == 0 && LPW % LOAD_PERIOD == 0 && (WAVES * RPS * LOAD_PERIOD) % SW_PERIOD == 0,
                "whole loads per wave, the lane-offset pattern periodic in the loads");
  static_assert(2 * BUFB == BQ * ROWB, "a Q tile fills the two V buffers");
  static constexpr __host__ __device__ int sw(int r) {
    return ((r & 3) << (SWB - 2)) | ((r >> 2) & ((1 << (SWB - 2)) - 1));
  }
};

template <typename T, int D>
__global__ __launch_bounds__(Tall<D>::THREADS, Tall<D>::PER_CU) void varlen_prefill_tall_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v, T* __restrict__ out,
    const int32_t* __restrict__ sched, int32_t* __restrict__ counters, float* __restrict__ partials,
    int32_t* __restrict__ err, int H, int H_kv, int G, float scale_log2, int causal, int spin_max) {
  using W = Tall<D>;
  constexpr int KS = D / 16;  // MFMA k-steps over D for S^T
  constexpr int DB = D / 32;  // 32-row blocks of D for O^T
  constexpr int BK = W::BK, BQ = W::BQ, ROWB = W::ROWB, LPW = W::LPW;
  // two K and two V buffers; the Q tile's rows 0-63 go to V buffer 0 and rows 64-127 to V
  // buffer 1 (so do the staged output rows), which are separate arrays so that the compiler
  // sees that a load into one never aliases a read of the other
  __shared__ __align__(512) uint8_t kb0[W::BUFB];
  __shared__ __align__(512) uint8_t kb1[W::BUFB];
  __shared__ __align__(512) uint8_t vb0[W::BUFB];
  __shared__ __align__(512) uint8_t vb1[W::BUFB];
  static_assert(W::BUFB == 64 * ROWB && W::WAVES == 4, "a V buffer holds the rows of two query blocks");

  asm volatile("" ::"s"(q), "s"(k), "s"(v), "s"(out));
  asm volatile("" ::"s"(H), "s"(H_kv), "s"(G), "s"(scale_log2), "s"(causal));
  const int32_t* entry = sched + kSchedHeader + W::ENTRY_WORDS * blockIdx.x;
  int first = entry[0], count = entry[1];
  int iw[W::ITEM_WORDS];
#pragma unroll
  for (int j = 0; j < W::ITEM_WORDS; ++j) iw[j] = entry[2 + j];
  static_assert(W::ITEM_WORDS == 6, "the pin below names six item words");
  asm volatile("" : "+s"(first), "+s"(count), "+s"(iw[0]), "+s"(iw[1]), "+s"(iw[2]), "+s"(iw[3]), "+s"(iw[4]),
                    "+s"(iw[5]));
  if (count <= 0) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5;
  const int col = lane & 31;
  const int64_t q_row = int64_t(H) * D;
  const int64_t q_row_b = q_row * int64_t(sizeof(T));
  const int64_t kv_row_b = int64_t(H_kv) * ROWB;

  struct Item {
    int seq0, L, row0, h, t_first, t_end, role, n_prod, counter, slot;
  };
  auto load_words = [&](int i) {
    const int32_t* w = sched + first + W::ITEM_WORDS * i;
#pragma unroll
    for (int j = 0; j < W::ITEM_WORDS; ++j) iw[j] = __builtin_amdgcn_readfirstlane(w[j]);
  };
  auto decode = [&]() {
    Item it;
    it.seq0 = iw[0];
    it.L = iw[1];
    it.row0 = int(uint32_t(iw[2]) >> 16) * BQ;
    it.h = iw[2] & 0xffff;
    it.t_first = int(uint32_t(iw[3]) >> 16);
    it.t_end = iw[3] & 0xffff;
    it.role = int(uint32_t(iw[4]) >> 30);
    it.n_prod = (iw[4] >> 24) & 63;
    it.counter = iw[4] & 0xffffff;
    it.slot = iw[5];
    return it;
  };

  // Load i of this wave fills 1 KiB segment wave + i * WAVES of a buffer: lane t writes
  // bytes 16t.. of it, i.e. row (wave + i * WAVES) * RPS + t / NCH, slot t % NCH, which holds
  // chunk slot ^ sw(row); sw repeats every LOAD_PERIOD loads, so load i is load i % LP
  // shifted by (i / LP) * WAVES * RPS * LP rows (a scalar offset). One buffer resource per
  // tile: base = the tile's first token at the item's KV head, range = the tile's rows inside
  // the segment (rows past it read as zero).
  constexpr int LP = W::LOAD_PERIOD;
  int dma_off[LP];
#pragma unroll
  for (int p = 0; p < LP; ++p) {
    const int r = (wave + p * W::WAVES) * W::RPS + lane / W::NCH;
    dma_off[p] = int(r * kv_row_b) + (((lane % W::NCH) ^ W::sw(r)) << 4);
  }
  const int dma_step = int(W::WAVES * W::RPS * LP * kv_row_b);
  auto issue = [&](const char* seg, const Item& it, int t, uint8_t* dst) {
    const int rows = t < it.t_end ? min(it.L - t * BK, BK) : 0;
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(seg + uint64_t(uint32_t(t)) * uint32_t(BK * kv_row_b)), (short)0, rows * int(kv_row_b),
        0x00020000);
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      buffer_load_lds16(rs, (lds_void_t*)((__attribute__((address_space(3))) uint8_t*)dst + (wave + i * W::WAVES) * 1024),
                        dma_off[i % LP], (i / LP) * dma_step);
    }
  };
  auto seg_of = [&](const T* base, const Item& it) {
    return reinterpret_cast<const char*>(base) + int64_t(it.seq0) * kv_row_b + (it.h / G) * ROWB;
  };
  // The item's Q tile (128 rows, laid out like a K tile) fills both V buffers; rows past the
  // segment read as zero. Lane offsets rebuilt per call from an opaque copy of the lane id.
  auto issue_q = [&](const Item& it) {
    int ql = lane;
    asm volatile("" : "+v"(ql));
    int off[LP];
#pragma unroll
    for (int p = 0; p < LP; ++p) {
      const int r = (wave + p * W::WAVES) * W::RPS + ql / W::NCH;
      off[p] = int(r * q_row_b) + (((ql % W::NCH) ^ W::sw(r)) << 4);
    }
    const int step_b = int(W::WAVES * W::RPS * LP * q_row_b);
    const int rows = min(it.L - it.row0, BQ);
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(reinterpret_cast<const char*>(q) + int64_t(it.seq0 + it.row0) * q_row_b + it.h * ROWB),
        (short)0, rows * int(q_row_b), 0x00020000);
#pragma unroll
    for (int i = 0; i < 2 * LPW; ++i) {
      // segment wave + i * WAVES of the tile: V buffer 0 holds the first SEGS, buffer 1 the rest
      uint8_t* dst = i < LPW ? vb0 : vb1;
      buffer_load_lds16(rs, (lds_void_t*)((__attribute__((address_space(3))) uint8_t*)dst + (wave + (i % LPW) * W::WAVES) * 1024),
                        off[i % LP], (i / LP) * step_b);
    }
  };
  // this wave's query rows (wave * 32 .. +31 of the item) in a Q tile or a staged output:
  // V buffer wave >> 1
  uint8_t* const qrows = (wave < 2 ? vb0 : vb1) + (wave & 1) * 32 * ROWB;

  // LDS byte offsets of this lane's operands, derived per read from three bases (eight
  // K and eight V offsets held in registers push the four-wave kernel into spills): the K
  // (and Q) fragment of k-step ks of a 32-row block is chunk (2 ks + g) ^ sw(row) =
  // (g ^ sw(row)) ^ 2 ks of its row, i.e. kx ^ (ks << 5), block b b * 32 rows on (sw depends
  // on the row mod SW_PERIOD, which divides 32); the two transposed reads of V^T block db
  // are chunks (4 db + x) ^ sw(key) = (x ^ sw(key)) ^ 4 db, i.e. vx[hh] ^ (db << 6), and
  // 16-key k-step s4 sits 16 s4 rows on. The bases pass through an empty asm at each step
  // (otherwise the compiler hoists every XORed offset out of the loop and spills them).
  static_assert(ROWB % 256 == 0 || (ROWB == 128 && KS == 4 && DB == 2), "XOR offsets: chunk bits free of row bits");
  const int kx0 = col * ROWB + ((g ^ W::sw(col)) << 4);
  int vx0[2];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int key = 8 * hh + 4 * g + ((lane & 15) >> 2);
    const int d0 = ((lane >> 4) & 1) * 16 + 4 * (lane & 3);
    vx0[hh] = key * ROWB + (((d0 >> 3) ^ W::sw(key)) << 4) + ((d0 >> 2) & 1) * 8;
  }
  int kx = kx0, vx[2] = {vx0[0], vx0[1]};
  auto fresh_bases = [&]() {
    kx = kx0;
    vx[0] = vx0[0];
    vx[1] = vx0[1];
    asm volatile("" : "+v"(kx), "+v"(vx[0]), "+v"(vx[1]));
  };
  auto koff = [&](int ks) { return kx ^ (ks << 5); };
  static_assert(W::sw(16) == W::sw(0) && W::sw(32) == W::sw(0), "16- and 32-row shifts keep the swizzle");

  auto read_vt = [&](const uint8_t* vb, int db, int s4) {
    const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_short4_t*)((__attribute__((address_space(3))) const uint8_t*)vb + (vx[0] ^ (db << 6)) + s4 * 16 * ROWB));
    const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_short4_t*)((__attribute__((address_space(3))) const uint8_t*)vb + (vx[1] ^ (db << 6)) + s4 * 16 * ROWB));
    const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
    return make_uint4(l2.x, l2.y, h2.x, h2.y);
  };

  // first item: Q, K(t0) and K(t0+1) in flight (later items get them from the previous
  // item's last step and epilogue)
  Item it = decode();
  const char* kseg = seg_of(k, it);
  const char* vseg = seg_of(v, it);
  issue_q(it);
  issue(kseg, it, it.t_first, kb0);
  issue(kseg, it, it.t_first + 1, kb1);
  uint4 qB[KS];
  constexpr int RPI = 64 / W::NCH;       // rows per wave-wide 16-byte read of the staged output
  constexpr int kStores = 32 / RPI;     // output stores per wave per item
  bool stored = false;                   // the previous item left its output stores in flight

  for (int idx = 0; idx < count; ++idx) {
    const int L = it.L;
    const int n_it = it.t_end - it.t_first;
    const bool more = idx + 1 < count;
    if (more) load_words(idx + 1);
    // Q, K(t0), K(t0+1) landed. A whole or owner item before this one issued its output
    // stores after this item's Q loads, always kStores of them (range-checked, so rows past
    // the segment are dropped, not skipped): vmcnt(kStores) leaves them in flight.
    if (stored) {
      wait_vm_lgkm0<kStores>();
    } else {
      wait_vm_lgkm0<0>();
    }
    bare_barrier();
    floatx16 cur[2];
    {
      fresh_bases();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) qB[ks] = *reinterpret_cast<const uint4*>(qrows + koff(ks));
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        uint4 kf[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) kf[ks] = *reinterpret_cast<const uint4*>(kb0 + b * 32 * ROWB + koff(ks));
        cur[b] = zero16();
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) cur[b] = mfma32<T>(kf[ks], qB[ks], cur[b]);
      }
    }
    wait_lgkm0();
    bare_barrier();  // Q and K(t0) read by every wave: the V buffers and K buffer 0 are free

    floatx16 o[DB];
#pragma unroll
    for (int i = 0; i < DB; ++i) o[i] = zero16();
    float m_i = -INFINITY, l_i = 0.0f;
    uint4 pB[4];  // P of the previous tile (4 k-steps of 16 keys), whose PV runs in this step

    // Step sidx (tile t = t_first + sidx): softmax of tile t (scores in cur), the scores of
    // tile t+1 (K(t+1) in kb_next; kS) and PV of tile t-1 (V(t-1) in vb_prev; kPV), so every
    // MFMA of the step is independent of the step's softmax; K(t+2) goes to kb_free and V(t)
    // to vb_free. The last step of an item computes no scores; instead it starts the next
    // item's first two K tiles (both K buffers are free: K(t) was read in the step before).
    auto step = [&](int sidx, const uint8_t* kb_next, uint8_t* kb_free, const uint8_t* vb_prev, uint8_t* vb_free,
                    auto pv_c, auto s_c, const Item& nx, const char* nkseg) {
      constexpr bool kPV = decltype(pv_c)::value;
      constexpr bool kS = decltype(s_c)::value;
      const int t = it.t_first + sidx;
      issue(vseg, it, t, vb_free);
      if constexpr (kS) {
        if (t + 2 < it.t_end) issue(kseg, it, t + 2, kb_free);
      } else if (more) {
        // issued after V(t), so the step's end waits for V(t) (the drain's) and leaves these
        // in flight through the drain and the epilogue
        issue(nkseg, nx, nx.t_first, kb0);
        issue(nkseg, nx, nx.t_first + 1, kb1);
      }
      __builtin_amdgcn_s_setprio(1);
      fresh_bases();
      floatx16 sc[2] = {cur[0], cur[1]};
      // only a tile that reaches past the segment end or the item's first row needs the mask
      if ((t + 1) * BK > L || (causal && (t + 1) * BK - 1 > it.row0)) {
        const int qi = it.row0 + wave * 32 + col;
        const int lim0 = (causal ? min(L, qi + 1) : L) - t * BK - g * 4;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          const int lim = lim0 - b * 32;
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            if ((e >> 2) * 8 + (e & 3) >= lim) sc[b][e] = -INFINITY;
          }
        }
      }
      // Phase A: PV(t-1) on the matrix cores (four groups of four MFMAs, one per 16-key
      // k-step, each group's V^T operands read during the group before) while the row max
      // of tile t is formed. Phase B: the scores of tile t+1 (eight groups of two MFMAs, K
      // operands read a group ahead) while tile t's exponentials are taken, packed to 16
      // bits (the next step's PV operand) and summed. sched_barrier keeps each group's reads
      // ahead of the group before's MFMAs.
      float mx[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) mx[j] = fmaxf(fmaxf(sc[0][4 * j], sc[0][4 * j + 1]), fmaxf(sc[0][4 * j + 2], sc[0][4 * j + 3]));
      uint4 fa[DB], fb[DB];
      if constexpr (kPV) {
#pragma unroll
        for (int db = 0; db < DB; ++db) fa[db] = read_vt(vb_prev, db, 0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
          if (s4 + 1 < 4) {
#pragma unroll
            for (int db = 0; db < DB; ++db) fb[db] = read_vt(vb_prev, db, s4 + 1);
          }
#pragma unroll
          for (int db = 0; db < DB; ++db) o[db] = mfma32<T>(fa[db], pB[s4], o[db]);
          // a quarter of the row max's vector work between this group's MFMAs
#pragma unroll
          for (int j = 0; j < 4; ++j) mx[j] = fmaxf(mx[j], sc[1][4 * s4 + j]);
          if (s4 + 1 < 4) __builtin_amdgcn_sched_group_barrier(0x0100, 2 * DB, 0);
#pragma unroll
          for (int db = 0; db < DB; ++db) {
            __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x0002, 2, 0);
          }
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int db = 0; db < DB; ++db) fa[db] = fb[db];
        }
      } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) mx[e & 3] = fmaxf(mx[e & 3], sc[1][e]);
      }
      const float mloc = fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3]));
      const float m_tile = max_halves(mloc) * scale_log2;
      // per query row, as in the duo kernel: the vote only gates the O rescale
      const bool mv = m_tile > m_i + 8.0f;
      const float m_new = mv ? m_tile : m_i;
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      const float alpha = fast_exp2(m_i - m_use);
      m_i = m_new;
      const bool moved = __any(mv);
      float ls = l_i * alpha;
      // phase B, group q (of NG): K operands of group q+1 read, group q's PG MFMAs, and its
      // share of the exponentials (EPG of them, part of P's k-step (q * EPG) / 8)
      constexpr int PG = 2;                 // MFMAs per group
      constexpr int NG = 2 * KS / PG;       // groups
      constexpr int EPG = 32 / NG;          // exponentials per group
      uint4 ka[PG], kn[PG];
      if constexpr (kS) {
#pragma unroll
        for (int i = 0; i < PG; ++i) ka[i] = *reinterpret_cast<const uint4*>(kb_next + koff(i));
      }
      __builtin_amdgcn_sched_barrier(0);
      floatx16 acc[2];
      float p8[8];
#pragma unroll
      for (int qg = 0; qg < NG; ++qg) {
        const int b = (qg * PG) / KS, k0 = (qg * PG) % KS;
        if constexpr (kS) {
          if (qg + 1 < NG) {
            const int b1 = ((qg + 1) * PG) / KS, k1 = ((qg + 1) * PG) % KS;
#pragma unroll
            for (int i = 0; i < PG; ++i) kn[i] = *reinterpret_cast<const uint4*>(kb_next + b1 * 32 * ROWB + koff(k1 + i));
          }
          if (k0 == 0) acc[b] = zero16();
#pragma unroll
          for (int i = 0; i < PG; ++i) acc[b] = mfma32<T>(ka[i], qB[k0 + i], acc[b]);
        }
        const int s4 = (qg * EPG) / 8, j0 = (qg * EPG) % 8;
        const floatx16& src = sc[s4 >> 1];
#pragma unroll
        for (int j = 0; j < EPG; ++j) p8[j0 + j] = fast_exp2(fmaf(src[8 * (s4 & 1) + j0 + j], scale_log2, -m_use));
        if (j0 + EPG == 8) {
          pB[s4] = make_uint4(pack2<T>(p8[0], p8[1]), pack2<T>(p8[2], p8[3]), pack2<T>(p8[4], p8[5]),
                              pack2<T>(p8[6], p8[7]));
          // pinned here, in this group: left alone the compiler sinks the exponentials into
          // the next step, beside the PV MFMAs that read P
#pragma unroll
          for (int e = 0; e < 8; ++e) ls += p8[e];  // the row sum from the fp32 values, as in the duo kernel
          asm volatile("" : "+v"(pB[s4].x), "+v"(pB[s4].y), "+v"(pB[s4].z), "+v"(pB[s4].w), "+v"(ls));
        }
        if constexpr (kS) {
          if (qg + 1 < NG) __builtin_amdgcn_sched_group_barrier(0x0100, PG, 0);
#pragma unroll
          for (int i = 0; i < PG; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x0002, 4, 0);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < PG; ++i) ka[i] = kn[i];
      }
      l_i = ls;
      if constexpr (kS) {
        cur[0] = acc[0];
        cur[1] = acc[1];
      }
      // O (with PV(t-1) added) moves to tile t's reference max
      if (moved) {
#pragma unroll
        for (int i = 0; i < DB; ++i) o[i] *= alpha;
      }
      __builtin_amdgcn_s_setprio(0);
      if (!kS && more) {
        wait_vm_lgkm0<2 * LPW>();
      } else {
        wait_vm_lgkm0<0>();
      }
      bare_barrier();
    };
    auto drain = [&](const uint8_t* vb) {
      fresh_bases();
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
#pragma unroll
        for (int db = 0; db < DB; ++db) o[db] = mfma32<T>(read_vt(vb, db, s4), pB[s4], o[db]);
      }
    };
    const Item cur_it = it;
    Item nx = it;
    const char* nkseg = kseg;
    if (more) {
      nx = decode();
      nkseg = seg_of(k, nx);
    }
    using No = std::false_type;
    using Yes = std::true_type;
    if (n_it == 1) {
      step(0, kb1, kb0, vb1, vb0, No{}, No{}, nx, nkseg);
      drain(vb0);
    } else {
      step(0, kb1, kb0, vb1, vb0, No{}, Yes{}, nx, nkseg);
      int sidx = 1;
      for (; sidx + 2 < n_it; sidx += 2) {
        step(sidx, kb0, kb1, vb0, vb1, Yes{}, Yes{}, nx, nkseg);
        step(sidx + 1, kb1, kb0, vb1, vb0, Yes{}, Yes{}, nx, nkseg);
      }
      if (sidx + 1 < n_it) {
        step(sidx, kb0, kb1, vb0, vb1, Yes{}, Yes{}, nx, nkseg);
        ++sidx;
      }
      // sidx == n_it - 1: the last step, then PV of the last tile (V in buffer sidx & 1)
      if (sidx & 1) {
        step(sidx, kb0, kb1, vb0, vb1, Yes{}, No{}, nx, nkseg);
        drain(vb1);
      } else {
        step(sidx, kb1, kb0, vb1, vb0, Yes{}, No{}, nx, nkseg);
        drain(vb0);
      }
    }
    it = nx;
    kseg = nkseg;
    vseg = seg_of(v, it);

    // ---- epilogue of cur_it
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int e_col = ln & 31, e_g = ln >> 5;
    float l_tot = sum_halves(l_i);
    // this wave's slice of a piece's partial
    auto part_rsrc = [&](int slot) {
      return __builtin_amdgcn_make_buffer_rsrc(partials + int64_t(slot) * W::PART_FLOATS, (short)0,
                                               W::PART_FLOATS * 4, 0x00020000);
    };
    constexpr int kSc1 = 16;  // device-scope cache policy: written through / read from the coherent level
    if (cur_it.role == W::ROLE_PRODUCER) {
      const auto rs = part_rsrc(cur_it.slot);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int grp = db * 4 + j;
          const u32x4_nt val = {__float_as_uint(o[db][4 * j + 0]), __float_as_uint(o[db][4 * j + 1]),
                                __float_as_uint(o[db][4 * j + 2]), __float_as_uint(o[db][4 * j + 3])};
          __builtin_amdgcn_raw_buffer_store_b128(val, rs, ((wave * (DB * 4) + grp) * 64 + ln) * 16, 0, kSc1);
        }
      }
      if (e_g == 0) {
        const u32x2_t ml = {__float_as_uint(m_i), __float_as_uint(l_tot)};
        __builtin_amdgcn_raw_buffer_store_b64(ml, rs, (W::PART_O + (wave * 32 + e_col) * 2) * 4, 0, kSc1);
      }
      stored = false;
      wait_vm_lgkm0<0>();  // this wave's partial is at the coherent level
      bare_barrier();      // ... and every wave's
      if (tid == 0) __hip_atomic_fetch_add(counters + cur_it.counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      if (cur_it.role == W::ROLE_OWNER) {
        // wait for the producers' count (bounded), then fold each partial in
        int seen = 0;
        for (int spin = 0; spin < spin_max; ++spin) {
          seen = __builtin_amdgcn_readfirstlane(
              __hip_atomic_load(counters + cur_it.counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
          if (seen >= cur_it.n_prod) break;
          __builtin_amdgcn_s_sleep(2);
        }
        if (seen < cur_it.n_prod && ln == 0) report(err, kErrTallWait);
        for (int p = 0; p < cur_it.n_prod; ++p) {
          const auto rs = part_rsrc(cur_it.slot + p);
          const u32x2_t ml = __builtin_amdgcn_raw_buffer_load_b64(rs, (W::PART_O + (wave * 32 + e_col) * 2) * 4, 0, kSc1);
          u32x4_nt po[DB * 4];
#pragma unroll
          for (int grp = 0; grp < DB * 4; ++grp) {
            po[grp] = __builtin_amdgcn_raw_buffer_load_b128(rs, ((wave * (DB * 4) + grp) * 64 + ln) * 16, 0, kSc1);
          }
          const float m_p = __uint_as_float(ml.x), l_p = __uint_as_float(ml.y);
          const float M = fmaxf(m_i, m_p);
          const float M_use = M == -INFINITY ? 0.0f : M;
          const float w_me = fast_exp2(m_i - M_use);
          const float w_p = fast_exp2(m_p - M_use);
          l_tot = fmaf(l_p, w_p, l_tot * w_me);
          m_i = M;
#pragma unroll
          for (int db = 0; db < DB; ++db) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const u32x4_nt pv = po[db * 4 + j];
              o[db][4 * j + 0] = fmaf(__uint_as_float(pv.x), w_p, o[db][4 * j + 0] * w_me);
              o[db][4 * j + 1] = fmaf(__uint_as_float(pv.y), w_p, o[db][4 * j + 1] * w_me);
              o[db][4 * j + 2] = fmaf(__uint_as_float(pv.z), w_p, o[db][4 * j + 2] * w_me);
              o[db][4 * j + 3] = fmaf(__uint_as_float(pv.w), w_p, o[db][4 * j + 3] * w_me);
            }
          }
        }
      }
      const float inv = 1.0f / fmaxf(l_tot, 1e-30f);
      // every wave has read the last V tile: the V buffers take the staged output
      wait_lgkm0();
      bare_barrier();
      if (cur_it.role == W::ROLE_OWNER && tid == 0) {
        // every wave has seen the count: take it back off (a producer that arrives after a
        // give-up leaves the counter at zero too)
        __hip_atomic_fetch_add(counters + cur_it.counter, -cur_it.n_prod, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      // staged as [row][16-byte chunk c at c ^ (row % NCH)] in this wave's 32 rows of the V
      // buffers, then read back 16 bytes per lane along the rows and stored as whole lines
#pragma unroll
      for (int db = 0; db < DB; ++db) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int c = db * 4 + j;
          float* f = reinterpret_cast<float*>(qrows + e_col * ROWB + ((c ^ (e_col & (W::NCH - 1))) << 4) + e_g * 8);
          f[0] = __builtin_bit_cast(float, pack2<T>(o[db][4 * j + 0] * inv, o[db][4 * j + 1] * inv));
          f[1] = __builtin_bit_cast(float, pack2<T>(o[db][4 * j + 2] * inv, o[db][4 * j + 3] * inv));
        }
      }
      wait_lgkm0();
      uint4 val[kStores];
#pragma unroll
      for (int i = 0; i < kStores; ++i) {
        const int rr = i * RPI + ln / W::NCH;
        const int c = ln % W::NCH;
        val[i] = *reinterpret_cast<const uint4*>(qrows + rr * ROWB + ((c ^ (rr & (W::NCH - 1))) << 4));
      }
      wait_lgkm0();
      bare_barrier();  // every wave has read its staged rows: the V buffers take the next Q
      if (more) issue_q(it);
      // the output stores go after the next item's Q loads, so the wait for Q does not wait
      // for them; one resource over the item's rows inside the segment, so the stores of rows
      // past it are dropped by the range check and every wave issues exactly kStores
      {
        const auto rs = __builtin_amdgcn_make_buffer_rsrc(
            reinterpret_cast<char*>(out) + int64_t(cur_it.seq0 + cur_it.row0) * q_row_b + cur_it.h * ROWB, (short)0,
            min(cur_it.L - cur_it.row0, BQ) * int(q_row_b), 0x00020000);
        constexpr int kNt = 2;  // nontemporal: the output is not read again by this kernel
#pragma unroll
        for (int i = 0; i < kStores; ++i) {
          const int rr = i * RPI + ln / W::NCH;
          const int c = ln % W::NCH;
          const u32x4_nt w = {val[i].x, val[i].y, val[i].z, val[i].w};
          __builtin_amdgcn_raw_buffer_store_b128(w, rs, (wave * 32 + rr) * int(q_row_b) + c * 16, 0, kNt);
        }
      }
      stored = true;
      continue;
    }
    // producer: the V buffers are free once every wave has passed the barrier above
    if (more) issue_q(it);
  }
}

// Second launch for split query tiles, one workgroup per (head, merge entry, quarter of
// the tile's rows); each thread owns 32 columns of one row and folds that row over the
// pieces (log-sum-exp on the stored (M, l)), with every load of all pieces in flight at
// once, then normalises and writes. Merge entry: (seq << 16 | tile, n_split << 24 |
// first partial slot). BQ = query rows of the split kernel's tile.
constexpr int kMaxSplit = 4;
template <typename T, int D, int BQ>
__global__ __launch_bounds__(256) void varlen_prefill_merge_kernel(
    const int32_t* __restrict__ cu, const int32_t* __restrict__ merges,
    const float* __restrict__ partials, T* __restrict__ out, int H) {
  constexpr int CPR = D / 32;            // threads per row
  constexpr int RPB = 256 / CPR;         // rows per workgroup
  const int h = blockIdx.x;
  const int entry = merges[2 * blockIdx.y];
  const int info = merges[2 * blockIdx.y + 1];
  const int seq = int(uint32_t(entry) >> 16);
  const int tile = entry & 0xffff;
  const int n_split = int(uint32_t(info) >> 24);
  const int slot = info & 0xffffff;
  const int seq0 = cu[seq];
  const int L = cu[seq + 1] - seq0;
  const int row = blockIdx.z * RPB + threadIdx.x / CPR;
  const int qi = tile * BQ + row;
  if (row >= BQ || qi >= L) return;
  const int d0 = (threadIdx.x % CPR) * 32;
  const int64_t pstride = int64_t(H) * (BQ * (D + 2));  // between consecutive pieces
  const float* p0 = partials + (int64_t(slot) * H + h) * (BQ * (D + 2));
  float2 ml[kMaxSplit];
  float4 v[kMaxSplit][8];
#pragma unroll
  for (int s = 0; s < kMaxSplit; ++s) {
    const int sc = s < n_split ? s : n_split - 1;  // repeated pieces are weighted out below
    const float* ps = p0 + sc * pstride;
    ml[s] = *reinterpret_cast<const float2*>(ps + BQ * D + row * 2);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[s][e] = reinterpret_cast<const float4*>(ps + row * D + d0)[e];
  }
  float M = -INFINITY;
#pragma unroll
  for (int s = 0; s < kMaxSplit; ++s) M = s < n_split ? fmaxf(M, ml[s].x) : M;
  const float M_use = M == -INFINITY ? 0.0f : M;
  float acc[32];
#pragma unroll
  for (int e = 0; e < 32; ++e) acc[e] = 0.0f;
  float l = 0.0f;
#pragma unroll
  for (int s = 0; s < kMaxSplit; ++s) {
    const float w = s < n_split ? fast_exp2(ml[s].x - M_use) : 0.0f;
    l = fmaf(ml[s].y, w, l);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      acc[4 * e + 0] = fmaf(v[s][e].x, w, acc[4 * e + 0]);
      acc[4 * e + 1] = fmaf(v[s][e].y, w, acc[4 * e + 1]);
      acc[4 * e + 2] = fmaf(v[s][e].z, w, acc[4 * e + 2]);
      acc[4 * e + 3] = fmaf(v[s][e].w, w, acc[4 * e + 3]);
    }
  }
  const float inv = 1.0f / fmaxf(l, 1e-30f);
  T* op = out + int64_t(seq0 + qi) * H * D + h * D + d0;
#pragma unroll
  for (int e = 0; e < 32; e += 8) {
    *reinterpret_cast<uint4*>(op + e) =
        make_uint4(pack2<T>(acc[e] * inv, acc[e + 1] * inv), pack2<T>(acc[e + 2] * inv, acc[e + 3] * inv),
                   pack2<T>(acc[e + 4] * inv, acc[e + 5] * inv), pack2<T>(acc[e + 6] * inv, acc[e + 7] * inv));
  }
}

// Schedule layout word: kernel kind << 20 | head_dim << 8 | query rows per tile.
enum Kind { kStaged = MI_PREFILL_STAGED, kRing = MI_PREFILL_RING, kDuo = MI_PREFILL_DUO, kTall = MI_PREFILL_TALL };
constexpr int layout_word(int kind, int D, int rows) { return (kind << 20) | (D << 8) | rows; }
constexpr int layout_kind(int layout) { return layout >> 20; }
constexpr int layout_d(int layout) { return (layout >> 8) & 0xfff; }
constexpr int layout_rows(int layout) { return layout & 0xff; }
int kind_rows(int kind) {
  return kind == kRing ? Ring<128>::BQ : kind == kDuo ? Duo<128>::BQ : kind == kTall ? Tall<128>::BQ : kBQ;
}
// keys per schedule unit of work (a causal tile's cost is counted in these)
int kind_keys(int kind) { return kind == kDuo ? Duo<128>::BK : kind == kTall ? Tall<128>::BK : Ring<128>::BK; }
// workgroups one CU holds at once
int kind_per_cu(int kind, int D) {
  return kind == kDuo ? (D == 256 ? Duo<256>::PER_CU : Duo<128>::PER_CU)
         : kind == kTall ? Tall<128>::PER_CU : kind == kStaged ? 2 : 1;
}
static_assert(Ring<128>::BK == Tiles<256>::BK && Ring<64>::BK == Tiles<128>::BK, "64-key tiles");
static_assert(Duo<64>::BQ == Duo<128>::BQ && Duo<64>::BK == Duo<128>::BK, "duo tile shape");
static_assert(Tall<64>::BQ == Tall<128>::BQ && Tall<64>::BK == Tall<128>::BK &&
                  Tall<64>::ITEM_WORDS == Tall<128>::ITEM_WORDS, "tall tile shape");

// Polls a bounded wait makes before it gives up (a tall owner waiting for its producers, a
// head_dim 256 duo wave waiting for its partner): set by mi_prefill_wait_limit, read at each
// launch. Each tall poll sleeps ~0.1 us, so the default bounds a wait at ~0.1 s, far beyond
// any wait a correct launch makes (at most one producer piece's run time).
int g_wait_limit = 1 << 20;

// Bytes of the tall kernel's workspace ahead of the partials: one int32 counter per split
// item, rounded up to 256 bytes. They must be zero before the first launch; every launch
// leaves them zero.
size_t tall_counter_bytes(int n_counters) { return (size_t(n_counters) * 4 + 255) / 256 * 256; }
size_t tall_workspace_bytes(int n_counters, int n_partials, int D) {
  if (n_partials == 0) return 0;
  const size_t per = size_t(D == 64 ? Tall<64>::PART_FLOATS : Tall<128>::PART_FLOATS) * sizeof(float);
  return tall_counter_bytes(n_counters) + size_t(n_partials) * per;
}

template <typename T, int D>
int launch2(const void* q, const void* k, const void* v, void* out, const int32_t* cu,
            const int32_t* sched, int n_work, int n_merge, int kind, void* workspace, int H,
            int H_kv, float scale_log2, int causal, int32_t* err, hipStream_t s) {
  const int32_t* work = sched + kSchedHeader;
  float* partials = static_cast<float*>(workspace);
  if constexpr (D == 64 || D == 128) {
    if (kind == kTall) {
      // n_merge holds the split items' counter count; the counters lead the workspace
      int32_t* counters = static_cast<int32_t*>(workspace);
      float* tall_partials = workspace == nullptr ? nullptr
          : reinterpret_cast<float*>(static_cast<char*>(workspace) + tall_counter_bytes(n_merge));
      hipLaunchKernelGGL((varlen_prefill_tall_kernel<T, D>), dim3(n_work), dim3(Tall<D>::THREADS), 0, s,
                         static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
                         static_cast<T*>(out), sched, counters, tall_partials, err, H, H_kv, H / H_kv, scale_log2,
                         causal, g_wait_limit);
      return launch_status("mi_varlen_prefill");
    }
  }
  if constexpr (D == 64 || D == 128 || D == 256) {
    if (kind == kDuo || (D != 256 && kind == kRing)) {
      constexpr int kRowsPerBlock = 256 / (D / 32);
      if (kind == kRing) {
        if constexpr (D != 256) {
          hipLaunchKernelGGL((varlen_prefill_ring_kernel<T, D>), dim3(H, n_work), dim3(Ring<D>::THREADS), 0, s,
                             static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
                             static_cast<T*>(out), cu, work, partials, H, H_kv, H / H_kv, scale_log2, causal);
          if (n_merge > 0) {
            hipLaunchKernelGGL((varlen_prefill_merge_kernel<T, D, Ring<D>::BQ>),
                               dim3(H, n_merge, (Ring<D>::BQ + kRowsPerBlock - 1) / kRowsPerBlock), dim3(256), 0, s,
                               cu, work + 2 * n_work, static_cast<const float*>(partials), static_cast<T*>(out), H);
          }
        }
      } else if (kind == kDuo) {
        // n_work persistent workgroups; their table follows the header, the merge entries
        // follow the table
        hipLaunchKernelGGL((varlen_prefill_duo_kernel<T, D>), dim3(n_work), dim3(Duo<D>::THREADS), 0, s,
                           static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
                           static_cast<T*>(out), sched, partials, H, H_kv, H / H_kv, scale_log2, causal, err,
                           g_wait_limit);
        if (n_merge > 0) {
          hipLaunchKernelGGL((varlen_prefill_merge_kernel<T, D, Duo<D>::BQ>),
                             dim3(H, n_merge, (Duo<D>::BQ + kRowsPerBlock - 1) / kRowsPerBlock), dim3(256), 0, s,
                             cu, work + Duo<D>::ENTRY_WORDS * n_work, static_cast<const float*>(partials),
                             static_cast<T*>(out), H);
        }
      }
      return launch_status("mi_varlen_prefill");
    }
  }
  hipLaunchKernelGGL((varlen_prefill_kernel<T, D>), dim3(H, n_work), dim3(Tiles<D>::THREADS), 0, s,
                     static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
                     static_cast<T*>(out), cu, work, H, H_kv, H / H_kv, scale_log2, causal);
  return launch_status("mi_varlen_prefill");
}

template <typename T>
int launch1(int D, const void* q, const void* k, const void* v, void* out, const int32_t* cu,
            const int32_t* sched, int n_work, int n_merge, int kind, void* ws, int H,
            int H_kv, float sl2, int causal, int32_t* err, hipStream_t s) {
  switch (D) {
    case 64: return launch2<T, 64>(q, k, v, out, cu, sched, n_work, n_merge, kind, ws, H, H_kv, sl2, causal, err, s);
    case 128: return launch2<T, 128>(q, k, v, out, cu, sched, n_work, n_merge, kind, ws, H, H_kv, sl2, causal, err, s);
    case 256: return launch2<T, 256>(q, k, v, out, cu, sched, n_work, n_merge, kind, ws, H, H_kv, sl2, causal, err, s);
  }
  return fail(MI_ERR_UNSUPPORTED,
              "mi_varlen_prefill: head_dim %d is not supported by the HIP prefill kernel "
              "(supported: 64, 128, 256)",
              D);
}

// One schedule piece: a query tile's key range (w0 = seq << 16 | tile, w1 = split << 28 |
// (n_split - 1) << 24 | first partial slot), or a merge entry, with its cost in key tiles.
struct Piece { int work, w0, w1; };

// Persistent duo kernel schedule: {n_wg, n_merge, n_partials, layout}, then n_wg entries of
// Duo::ENTRY_WORDS {first item word, item count, the first item's words, 0, 0}, the n_merge
// merge entries, and the items, Duo::ITEM_WORDS words each. Items are (piece, head) pairs
// dealt out longest-first to the workgroup with the least work so far (LPT); when the launch
// fills the chip and the KV heads divide evenly over the XCDs, or the XCDs over the KV heads,
// the items of a KV head go to the workgroups of its XCD or block of XCDs (workgroup w runs on
// XCD w % kXcds), so its K and V stay in those XCDs' L2. An item costs its key tiles plus kItemOverhead for its
// prologue and epilogue: a workgroup's extra single-tile item takes about as long as five
// 64-key steps, and counting 8 balances best (config-3 batch 31.5 us against 32.2 us with
// 3, 31.8 with 12, 32.9 with 16; batches of equal or mid-length segments unchanged;
// rechecked on the current kernel: 28.2 us with 8 or 9, 28.9 with 5-7, 28.55 with 10). At
// head_dim 256 (one workgroup per CU, ~1.15 us steps, ~6 us per item's ends) 5: config-3
// lengths 40.3 us against 42.0 with 8, 40.8 with 2, 44.1 with 1 and 11, 40.2-40.4 with 3-6.
int duo_schedule(const int32_t* cu, const std::vector<Piece>& pieces, const std::vector<Piece>& merges,
                 int n_partials, int H, int H_kv, int D, int32_t* out, int capacity) {
  constexpr int kCUs = 256;
  const int kItemOverhead = D == 256 ? 5 : 8;
  const int kSlots = kCUs * kind_per_cu(kDuo, D);
  const int64_t n_items = int64_t(pieces.size()) * H;
  const int n_wg = int(std::min<int64_t>(kSlots, n_items));
  const int n_merge = int(merges.size());
  constexpr int EW = Duo<128>::ENTRY_WORDS, IW = Duo<128>::ITEM_WORDS;
  const int64_t words64 = kSchedHeader + EW * int64_t(n_wg) + 2 * int64_t(n_merge) + IW * n_items;
  if (words64 > INT32_MAX) return fail(MI_ERR_UNSUPPORTED, "mi_varlen_schedule: schedule too large");
  const int words = int(words64);
  if (out == nullptr) return words;
  if (capacity < words) return fail(MI_ERR_INVALID, "mi_varlen_schedule: capacity %d < %d words", capacity, words);
  // groups of workgroups that share an L2: one per XCD when the KV heads spread evenly
  // KV heads per XCD group: with H_kv a multiple of the XCD count each XCD takes the KV
  // heads kvh with kvh % kXcds == x; with H_kv a divisor of it each KV head takes a block of
  // kXcds / H_kv XCDs (at H_kv 2, XCDs 0-3 and 4-7), so an XCD's L2 holds one KV head's K/V
  const bool full = n_wg == kSlots;
  const int n_groups = !full ? 1 : H_kv % kXcds == 0 ? kXcds : kXcds % H_kv == 0 ? H_kv : 1;
  const int xcds_per_group = kXcds / n_groups;
  auto group_of_wg = [&](int w) { return (w % kXcds) / xcds_per_group; };
  const int G = H / H_kv;
  auto group_of_head = [&](int h) { return (h / G) % n_groups; };
  std::vector<std::vector<int>> lists(n_wg);
  std::vector<int64_t> load(n_wg, 0);
  for (int grp = 0; grp < n_groups; ++grp) {
    // workgroups of this group, as a min-heap on (load, id)
    std::vector<std::pair<int64_t, int>> heap;
    for (int w = 0; w < n_wg; ++w) {
      if (group_of_wg(w) == grp) heap.push_back({0, w});
    }
    auto cmp = [](const std::pair<int64_t, int>& a, const std::pair<int64_t, int>& b) { return a > b; };
    std::make_heap(heap.begin(), heap.end(), cmp);
    for (int p = 0; p < int(pieces.size()); ++p) {  // pieces are sorted longest-first
      for (int h = 0; h < H; ++h) {
        if (group_of_head(h) != grp) continue;
        std::pop_heap(heap.begin(), heap.end(), cmp);
        auto& top = heap.back();
        lists[top.second].push_back(p * H + h);
        top.first += pieces[p].work + kItemOverhead;
        std::push_heap(heap.begin(), heap.end(), cmp);
      }
    }
  }
  out[0] = n_wg;
  out[1] = n_merge;
  out[2] = n_partials;
  out[3] = layout_word(kDuo, D, Duo<128>::BQ);
  int32_t* table = out + kSchedHeader;
  int32_t* mw = table + EW * n_wg;
  for (const Piece& pc : merges) { *mw++ = pc.w0; *mw++ = pc.w1; }
  int item_word = int(mw - out);
  int32_t* iw = mw;
  for (int w = 0; w < n_wg; ++w) {
    int32_t* e = table + EW * w;
    std::fill(e, e + EW, 0);
    e[0] = item_word;
    e[1] = int(lists[w].size());
    for (size_t i = 0; i < lists[w].size(); ++i) {
      const int id = lists[w][i];
      const Piece& pc = pieces[id / H];
      const int h = id % H;
      const int seq = int(uint32_t(pc.w0) >> 16), tile = pc.w0 & 0xffff;
      const int split = int(uint32_t(pc.w1) >> 28), nsm1 = (pc.w1 >> 24) & 15, slot = pc.w1 & 0xffffff;
      iw[0] = cu[seq];
      iw[1] = cu[seq + 1] - cu[seq];
      iw[2] = int((uint32_t(tile) << 16) | (uint32_t(split) << 8) | uint32_t(nsm1));
      iw[3] = int((uint32_t(h) << 24) | uint32_t(slot));
      if (i == 0) std::copy(iw, iw + IW, e + 2);  // the first item, inline
      iw += IW;
      item_word += IW;
    }
  }
  return words;
}

// Tall kernel schedule: {n_workgroups, n_counters, n_partials, layout}, n_workgroups entries
// of Tall::ENTRY_WORDS {first item word, item count, the first item's six words}, then the
// items, Tall::ITEM_WORDS words each (see the kernel). 128-row query tiles of every segment
// count their 64-key steps; a tile x head whose steps exceed a cap C is cut into
// ceil(steps / C) key ranges of near-equal length, the last one (it holds the diagonal) the
// owner. Items are dealt longest-first to the least-loaded workgroup (LPT), the items of a
// KV head on the workgroups of its XCD (or block of XCDs) when the launch fills the chip, so
// its K and V stay in that L2. An item costs its steps plus kItemCost (its start and end), an
// owner kMergeCost more per producer; C is the cap, tried from kMinCap up to the longest
// tile, whose deal has the smallest most-loaded workgroup (ties: the larger cap, fewer
// pieces). Each workgroup's list then runs its producer pieces first, so no owner waits on a
// piece queued behind another owner.
#ifndef MIATTN_TALL_CAP
#define MIATTN_TALL_CAP 0  // > 0: a fixed piece cap in key steps instead of the search
#endif
#ifndef MIATTN_TALL_ITEM_COST
#define MIATTN_TALL_ITEM_COST 3
#endif
#ifndef MIATTN_TALL_MERGE_COST
#define MIATTN_TALL_MERGE_COST 2
#endif
int tall_schedule(const int32_t* cu, int n_seqs, int H, int H_kv, int D, int causal, int32_t* out, int capacity,
                  int* n_split_tiles = nullptr) {
  using W = Tall<128>;
  constexpr int kCUs = 256, kMinCap = 4, kMaxPieces = 32;
  constexpr int kItemCost = MIATTN_TALL_ITEM_COST, kMergeCost = MIATTN_TALL_MERGE_COST;
  const int slots = kCUs * W::PER_CU;
  struct TTile { int seq, tile, steps; };
  std::vector<TTile> tiles;
  int max_steps = 0;
  for (int s = 0; s < n_seqs; ++s) {
    const int L = cu[s + 1] - cu[s];
    const int n = (L + W::BQ - 1) / W::BQ;
    for (int t = 0; t < n; ++t) {
      const int end = std::min(L, (t + 1) * W::BQ);
      const int steps = causal ? (end + W::BK - 1) / W::BK : (L + W::BK - 1) / W::BK;
      tiles.push_back({s, t, steps});
      max_steps = std::max(max_steps, steps);
    }
  }
  if (max_steps > 65535) return fail(MI_ERR_UNSUPPORTED, "mi_varlen_schedule: segment too long for the tall kernel");
  if (H > 65535) return fail(MI_ERR_UNSUPPORTED, "mi_varlen_schedule: the tall kernel takes at most 65535 heads");
  struct TPiece { int tile, t0, t1, role, n_prod, cost; };
  const int G = H / H_kv;
  std::vector<TPiece> pieces;
  std::vector<std::vector<int>> lists;
  int n_wg = 0;
  auto cut = [&](int cap) {
    pieces.clear();
    for (int i = 0; i < int(tiles.size()); ++i) {
      const int S = tiles[i].steps;
      const int n = S > cap ? std::min(kMaxPieces, (S + cap - 1) / cap) : 1;
      for (int p = 0; p < n; ++p) {
        const int t0 = int(int64_t(p) * S / n), t1 = int(int64_t(p + 1) * S / n);
        const int role = n == 1 ? W::ROLE_WHOLE : p + 1 < n ? W::ROLE_PRODUCER : W::ROLE_OWNER;
        const int cost = (t1 - t0) + kItemCost + (role == W::ROLE_OWNER ? kMergeCost * (n - 1) : 0);
        pieces.push_back({i, t0, t1, role, n - 1, cost});
      }
    }
  };
  // deal (piece, head) items; returns the most-loaded workgroup's cost
  auto deal = [&]() -> int64_t {
    const int64_t n_items = int64_t(pieces.size()) * H;
    n_wg = int(std::min<int64_t>(slots, n_items));
    const bool full = n_wg == slots;
    const int n_groups = !full ? 1 : H_kv % kXcds == 0 ? kXcds : kXcds % H_kv == 0 ? H_kv : 1;
    const int xcds_per_group = kXcds / n_groups;
    std::vector<int> order(pieces.size());
    for (int i = 0; i < int(order.size()); ++i) order[i] = i;
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return pieces[a].cost > pieces[b].cost; });
    lists.assign(n_wg, {});
    int64_t worst = 0;
    for (int grp = 0; grp < n_groups; ++grp) {
      std::vector<std::pair<int64_t, int>> heap;
      for (int w = 0; w < n_wg; ++w) {
        if ((w % kXcds) / xcds_per_group == grp) heap.push_back({0, w});
      }
      auto cmp = [](const std::pair<int64_t, int>& a, const std::pair<int64_t, int>& b) { return a > b; };
      std::make_heap(heap.begin(), heap.end(), cmp);
      for (int p : order) {
        for (int h = 0; h < H; ++h) {
          if ((h / G) % n_groups != grp) continue;
          std::pop_heap(heap.begin(), heap.end(), cmp);
          auto& top = heap.back();
          lists[top.second].push_back(p * H + h);
          top.first += pieces[p].cost;
          worst = std::max(worst, top.first);
          std::push_heap(heap.begin(), heap.end(), cmp);
        }
      }
    }
    return worst;
  };
  int best_cap = max_steps;
  int64_t best = INT64_MAX;
  for (int cap = MIATTN_TALL_CAP > 0 ? std::min(MIATTN_TALL_CAP, max_steps) : std::min(kMinCap, max_steps);
       cap <= (MIATTN_TALL_CAP > 0 ? std::min(MIATTN_TALL_CAP, max_steps) : max_steps); ++cap) {
    cut(cap);
    const int64_t worst = deal();
    if (worst <= best) {
      best = worst;
      best_cap = cap;
    }
  }
  cut(best_cap);
  deal();
  // producers first in every list (stable), so a producer never waits behind an owner
  for (auto& lst : lists) {
    std::stable_partition(lst.begin(), lst.end(),
                          [&](int id) { return pieces[id / H].role == W::ROLE_PRODUCER; });
  }
  // counters (one per split tile x head) and partial slots (one per producer piece x head,
  // a tile's producers contiguous for each head)
  std::vector<int> tile_counter(tiles.size(), -1), tile_slot(tiles.size(), -1);
  int n_counters = 0, n_partials = 0;
  for (const TPiece& pc : pieces) {
    if (pc.role == W::ROLE_OWNER && tile_counter[pc.tile] < 0) {
      tile_counter[pc.tile] = n_counters;
      n_counters += H;
      tile_slot[pc.tile] = n_partials;
      n_partials += pc.n_prod * H;
    }
  }
  if (n_counters >= (1 << 24)) return fail(MI_ERR_UNSUPPORTED, "mi_varlen_schedule: too many split tiles");
  if (n_split_tiles != nullptr) *n_split_tiles = n_counters;
  constexpr int EW = W::ENTRY_WORDS, IW = W::ITEM_WORDS;
  const int64_t n_items = int64_t(pieces.size()) * H;
  const int64_t words64 = kSchedHeader + EW * int64_t(n_wg) + IW * n_items;
  if (words64 > INT32_MAX) return fail(MI_ERR_UNSUPPORTED, "mi_varlen_schedule: schedule too large");
  const int words = int(words64);
  if (out == nullptr) return words;
  if (capacity < words) return fail(MI_ERR_INVALID, "mi_varlen_schedule: capacity %d < %d words", capacity, words);
  out[0] = n_wg;
  out[1] = n_counters;
  out[2] = n_partials;
  out[3] = layout_word(kTall, D, W::BQ);
  int32_t* table = out + kSchedHeader;
  int item_word = kSchedHeader + EW * n_wg;
  int32_t* iw = out + item_word;
  for (int w = 0; w < n_wg; ++w) {
    int32_t* e = table + EW * w;
    std::fill(e, e + EW, 0);
    e[0] = item_word;
    e[1] = int(lists[w].size());
    for (size_t i = 0; i < lists[w].size(); ++i) {
      const int id = lists[w][i];
      const TPiece& pc = pieces[id / H];
      const int h = id % H;
      const TTile& tl = tiles[pc.tile];
      // a producer's slot: its tile's first slot for this head plus its index among the
      // tile's producers (pieces of a tile are consecutive, producers first)
      int slot = 0, counter = 0;
      if (pc.role != W::ROLE_WHOLE) {
        counter = tile_counter[pc.tile] + h;
        const int base = tile_slot[pc.tile] + h * pc.n_prod;
        int index = 0;
        if (pc.role == W::ROLE_PRODUCER) {
          for (int j = id / H - 1; j >= 0 && pieces[j].tile == pc.tile; --j) ++index;
        }
        slot = base + index;
      }
      iw[0] = cu[tl.seq];
      iw[1] = cu[tl.seq + 1] - cu[tl.seq];
      iw[2] = int((uint32_t(tl.tile) << 16) | uint32_t(h));
      iw[3] = int((uint32_t(pc.t0) << 16) | uint32_t(pc.t1));
      iw[4] = int((uint32_t(pc.role) << 30) | (uint32_t(pc.n_prod) << 24) | uint32_t(counter));
      iw[5] = slot;
      if (i == 0) std::copy(iw, iw + IW, e + 2);
      iw += IW;
      item_word += IW;
    }
  }
  return words;
}

size_t partial_bytes(int n_partials, int H, int D, int rows) {
  return size_t(n_partials) * H * rows * (D + 2) * sizeof(float);
}

}  // namespace
}  // namespace miattn

extern "C" int mi_varlen_schedule_for(const int32_t* host_cu_seqlens, int n_seqs, int H, int H_kv,
                                      int D, int causal, int kernel, int32_t* host_schedule,
                                      int capacity) {
  using namespace miattn;
  if (kernel < MI_PREFILL_AUTO || kernel > MI_PREFILL_TALL || kernel == 2) {
    return fail(MI_ERR_INVALID, "mi_varlen_schedule: unknown prefill kernel %d", kernel);
  }
  if (kernel == MI_PREFILL_TALL && D != 64 && D != 128) {
    return fail(MI_ERR_UNSUPPORTED, "mi_varlen_schedule: the tall kernel takes head_dim 64 or 128, got %d", D);
  }
  if (kernel == MI_PREFILL_RING && D != 64 && D != 128) {
    return fail(MI_ERR_UNSUPPORTED, "mi_varlen_schedule: the ring kernel takes head_dim 64 or 128, got %d", D);
  }
  if (kernel == MI_PREFILL_DUO && D != 64 && D != 128 && D != 256) {
    return fail(MI_ERR_UNSUPPORTED, "mi_varlen_schedule: the duo kernel takes head_dim 64, 128 or 256, got %d", D);
  }
  if (host_cu_seqlens == nullptr || n_seqs < 1 || n_seqs > 65535) {
    return fail(MI_ERR_INVALID, "mi_varlen_schedule: need 1..65535 segments, got %d", n_seqs);
  }
  if (H < 1 || H_kv < 1 || H % H_kv != 0) {
    return fail(MI_ERR_INVALID, "mi_varlen_schedule: n_head (%d) must be a multiple of n_kv_head (%d)",
                H, H_kv);
  }
  int max_len = 0;
  for (int s = 0; s < n_seqs; ++s) max_len = std::max(max_len, host_cu_seqlens[s + 1] - host_cu_seqlens[s]);
  if (kernel == MI_PREFILL_DUO && H > 255) {
    return fail(MI_ERR_UNSUPPORTED, "mi_varlen_schedule: the duo kernel takes at most 255 heads, got %d", H);
  }
  // By default head_dim 64 and 128 run the ring kernel when the longest segment reaches
  // kRingMinLen tokens and the persistent duo kernel otherwise, and head_dim 256 runs the
  // duo kernel; a batch of more heads than the duo kernel's item word holds (255) runs the
  // ring kernel (64, 128) or the register-staged kernel (256). The caller may name a kernel
  // instead.
  const bool duo_heads = H <= 255;
  for (int s = 0; s < n_seqs; ++s) {
    if (host_cu_seqlens[s + 1] - host_cu_seqlens[s] <= 0) {
      return fail(MI_ERR_INVALID, "mi_varlen_schedule: segment %d is empty", s);
    }
  }
  // by default head_dim 64/128 batches with a segment of kTallMinLen tokens or more run the
  // tall kernel when its schedule needs no split pieces
  bool tall_default = false;
  if (kernel == MI_PREFILL_AUTO && (D == 64 || D == 128) && max_len >= kTallMinLen && H <= 65535) {
    int n_split = -1;
    if (tall_schedule(host_cu_seqlens, n_seqs, H, H_kv, D, causal, nullptr, 0, &n_split) > 0 && n_split == 0) {
      tall_default = true;
    }
  }
  const int kind = kernel == MI_PREFILL_STAGED ? kStaged : kernel == MI_PREFILL_RING ? kRing
                 : kernel == MI_PREFILL_DUO ? kDuo : kernel == MI_PREFILL_TALL || tall_default ? kTall
                 : (D == 64 || D == 128) ? (max_len >= kRingMinLen || !duo_heads ? kRing : kDuo)
                 : D == 256 && duo_heads ? kDuo : kStaged;
  if (kind == kTall) {
    return tall_schedule(host_cu_seqlens, n_seqs, H, H_kv, D, causal, host_schedule, capacity);
  }
  const bool ring = kind != kStaged;  // one workgroup per CU, split-K capable
  const int RW = kind_rows(kind);
  const int BN = kind_keys(kind);
  struct Tile { int work, seq, tile; };
  std::vector<Tile> tiles;
  int64_t total = 0;
  for (int s = 0; s < n_seqs; ++s) {
    const int L = host_cu_seqlens[s + 1] - host_cu_seqlens[s];
    if (L <= 0) return fail(MI_ERR_INVALID, "mi_varlen_schedule: segment %d is empty", s);
    const int n = (L + RW - 1) / RW;
    if (n > 65535) return fail(MI_ERR_UNSUPPORTED, "mi_varlen_schedule: segment %d too long", s);
    for (int t = 0; t < n; ++t) {
      const int end = std::min(L, (t + 1) * RW);
      const int work = causal ? (end + BN - 1) / BN : (L + BN - 1) / BN;
      tiles.push_back({work, s, t});
      total += work;
    }
  }
  // Split-K for launches that cannot fill the MI355X's 256 CUs (fewer query tiles x heads
  // than CUs, one ring workgroup per CU): the long tiles' key ranges are cut so that no
  // piece exceeds the even share of the launch over the CUs, none drops below kMinPiece
  // key tiles, and no tile splits into more than kMaxSplit pieces. A launch that fills
  // the chip is not split: its pieces would only add per-workgroup start-up and merge
  // cost (measured slower on the config-3 batch, 46 + 8 us against 42 us unsplit).
  constexpr int kCUs = 256, kMinPiece = 8;
  const int slots = kCUs * kind_per_cu(kind, D);  // workgroups the chip runs at once
  const int64_t share = (total * H + slots - 1) / slots;
  const bool underfilled = int64_t(tiles.size()) * H < slots;
  const int cap = underfilled ? int(std::max<int64_t>(share, kMinPiece)) : INT32_MAX;
  std::vector<Piece> pieces, merges;
  int n_partials = 0;
  for (const Tile& t : tiles) {
    int ns = ring && MIATTN_PREFILL_SPLIT ? int((int64_t(t.work) + cap - 1) / cap) : 1;
    ns = std::max(1, std::min(ns, std::min(kMaxSplit, t.work)));
    const int w0 = (t.seq << 16) | t.tile;
    const int slot = ns > 1 ? n_partials : 0;
    for (int sp = 0; sp < ns; ++sp) {
      const int work = (sp + 1) * t.work / ns - sp * t.work / ns;
      pieces.push_back({work, w0, int((uint32_t(sp) << 28) | (uint32_t(ns - 1) << 24) | uint32_t(slot))});
    }
    if (ns > 1) {
      merges.push_back({t.work, w0, int((uint32_t(ns) << 24) | uint32_t(slot))});
      n_partials += ns;
    }
  }
  if (n_partials >= (1 << 24)) return fail(MI_ERR_UNSUPPORTED, "mi_varlen_schedule: too many split tiles");
  std::stable_sort(pieces.begin(), pieces.end(), [](const Piece& a, const Piece& b) { return a.work > b.work; });
  if (kind == kDuo) {
    return duo_schedule(host_cu_seqlens, pieces, merges, n_partials, H, H_kv, D, host_schedule, capacity);
  }
  const int n_work = int(pieces.size()), n_merge = int(merges.size());
  const int words = kSchedHeader + 2 * (n_work + n_merge);
  if (host_schedule != nullptr) {
    if (capacity < words) {
      return fail(MI_ERR_INVALID, "mi_varlen_schedule: capacity %d < %d words", capacity, words);
    }
    host_schedule[0] = n_work;
    host_schedule[1] = n_merge;
    host_schedule[2] = n_partials;
    host_schedule[3] = layout_word(kind, D, RW);
    int32_t* w = host_schedule + kSchedHeader;
    for (const Piece& pc : pieces) { *w++ = pc.w0; *w++ = pc.w1; }
    for (const Piece& pc : merges) { *w++ = pc.w0; *w++ = pc.w1; }
  }
  return words;
}

extern "C" int mi_varlen_schedule(const int32_t* host_cu_seqlens, int n_seqs, int H, int H_kv,
                                  int D, int causal, int32_t* host_schedule, int capacity) {
  return mi_varlen_schedule_for(host_cu_seqlens, n_seqs, H, H_kv, D, causal, MI_PREFILL_AUTO,
                                host_schedule, capacity);
}

extern "C" size_t mi_varlen_workspace_size(const int32_t* host_schedule, int H) {
  using namespace miattn;
  if (host_schedule == nullptr || H < 1) return 0;
  if (layout_kind(host_schedule[3]) == kTall) {
    return tall_workspace_bytes(host_schedule[1], host_schedule[2], layout_d(host_schedule[3]));
  }
  return partial_bytes(host_schedule[2], H, layout_d(host_schedule[3]), layout_rows(host_schedule[3]));
}

extern "C" int mi_prefill_wait_limit(int polls) {
  const int previous = miattn::g_wait_limit;
  if (polls >= 0) miattn::g_wait_limit = polls;
  return previous;
}

extern "C" int mi_varlen_prefill(const void* q, const void* k, const void* v, void* out,
                                 const int32_t* cu_seqlens, int n_seqs, int total_tokens,
                                 int max_seqlen, const int32_t* schedule, int n_work, int n_merge,
                                 int n_partials, int layout, int H, int H_kv, int D, float scale,
                                 int causal, int dtype, void* workspace, size_t workspace_bytes,
                                 int32_t* error_word, void* stream) {
  using namespace miattn;
  if (dtype != MI_BF16 && dtype != MI_F16) {
    return fail(MI_ERR_UNSUPPORTED,
                "mi_varlen_prefill: the MFMA prefill computes fp16/bf16 only (dtype code %d)", dtype);
  }
  if (H < 1 || H_kv < 1 || H % H_kv != 0) {
    return fail(MI_ERR_INVALID, "mi_varlen_prefill: n_head (%d) must be a multiple of n_kv_head (%d)",
                H, H_kv);
  }
  if (n_seqs < 1 || total_tokens < 1 || max_seqlen < 1 || n_work < 1 || n_work > 65535 ||
      n_merge < 0 || n_merge > 65535 || n_partials < 0) {
    return fail(MI_ERR_INVALID,
                "mi_varlen_prefill: bad sizes n_seqs=%d total=%d max_seqlen=%d work=%d merge=%d",
                n_seqs, total_tokens, max_seqlen, n_work, n_merge);
  }
  if (q == nullptr || k == nullptr || v == nullptr || out == nullptr || cu_seqlens == nullptr ||
      schedule == nullptr) {
    return fail(MI_ERR_INVALID, "mi_varlen_prefill: NULL pointer argument");
  }
  const int rows = layout_rows(layout);
  const int kind = layout_kind(layout);
  const bool split_capable = kind == kRing || kind == kDuo || kind == kTall;
  if (layout_d(layout) != D || kind < kStaged || kind > kTall || kind == 2 || rows != kind_rows(kind) ||
      (kind == kRing && D != 64 && D != 128) || (kind == kDuo && D != 64 && D != 128 && D != 256) ||
      (kind == kTall && D != 64 && D != 128) || (n_merge > 0) != (n_partials > 0) ||
      (n_merge > 0 && !split_capable)) {
    return fail(MI_ERR_INVALID, "mi_varlen_prefill: schedule (layout 0x%x) does not match head_dim %d",
                layout, D);
  }
  const size_t need = kind == kTall ? tall_workspace_bytes(n_merge, n_partials, D) : partial_bytes(n_partials, H, D, rows);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    return fail(MI_ERR_WORKSPACE, "mi_varlen_prefill: workspace of %zu bytes needed, got %zu", need,
                workspace == nullptr ? size_t(0) : workspace_bytes);
  }
  auto al = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  if (!al(q) || !al(k) || !al(v) || !al(out) || (need > 0 && !al(workspace))) {
    return fail(MI_ERR_UNSUPPORTED, "mi_varlen_prefill: q/k/v/out/workspace must be 16-byte aligned");
  }
  if (error_word != nullptr && reinterpret_cast<uintptr_t>(error_word) % 4 != 0) {
    return fail(MI_ERR_INVALID, "mi_varlen_prefill: error_word must be 4-byte aligned");
  }
  const float sl2 = float(double(scale) * 1.4426950408889634);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == MI_BF16) {
    return launch1<bf16_t>(D, q, k, v, out, cu_seqlens, schedule, n_work, n_merge, kind, workspace, H,
                           H_kv, sl2, causal, error_word, s);
  }
  return launch1<f16_t>(D, q, k, v, out, cu_seqlens, schedule, n_work, n_merge, kind, workspace, H,
                        H_kv, sl2, causal, error_word, s);
}
