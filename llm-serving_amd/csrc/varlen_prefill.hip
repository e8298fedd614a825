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
  const int entry = sched[blockIdx.y];
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
      const float m_tile = fmaxf(mloc, swap32(mloc)) * scale_log2;
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
  const float l_tot = l_i + swap32(l_i);
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

int rows_per_tile() { return kBQ; }

int keys_per_tile(int D) { return D <= 128 ? Tiles<128>::BK : Tiles<256>::BK; }

template <typename T, int D>
int launch2(const void* q, const void* k, const void* v, void* out, const int32_t* cu,
            const int32_t* sched, int n_tiles, int H, int H_kv, float scale_log2, int causal,
            hipStream_t s) {
  dim3 grid(H, n_tiles);
  hipLaunchKernelGGL((varlen_prefill_kernel<T, D>), grid, dim3(Tiles<D>::THREADS), 0, s,
                     static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
                     static_cast<T*>(out), cu, sched, H, H_kv, H / H_kv, scale_log2, causal);
  return launch_status("mi_varlen_prefill");
}

template <typename T>
int launch1(int D, const void* q, const void* k, const void* v, void* out, const int32_t* cu,
            const int32_t* sched, int n_tiles, int H, int H_kv, float sl2, int causal,
            hipStream_t s) {
  switch (D) {
    case 64: return launch2<T, 64>(q, k, v, out, cu, sched, n_tiles, H, H_kv, sl2, causal, s);
    case 128: return launch2<T, 128>(q, k, v, out, cu, sched, n_tiles, H, H_kv, sl2, causal, s);
    case 256: return launch2<T, 256>(q, k, v, out, cu, sched, n_tiles, H, H_kv, sl2, causal, s);
  }
  return fail(MI_ERR_UNSUPPORTED,
              "mi_varlen_prefill: head_dim %d is not supported by the HIP prefill kernel "
              "(supported: 64, 128, 256)",
              D);
}

}  // namespace
}  // namespace miattn

extern "C" int mi_varlen_schedule(const int32_t* host_cu_seqlens, int n_seqs, int H, int H_kv,
                                  int D, int causal, int32_t* host_schedule, int capacity) {
  using namespace miattn;
  if (host_cu_seqlens == nullptr || n_seqs < 1 || n_seqs > 65535) {
    return fail(MI_ERR_INVALID, "mi_varlen_schedule: need 1..65535 segments, got %d", n_seqs);
  }
  if (H < 1 || H_kv < 1 || H % H_kv != 0) {
    return fail(MI_ERR_INVALID, "mi_varlen_schedule: n_head (%d) must be a multiple of n_kv_head (%d)",
                H, H_kv);
  }
  const int RW = rows_per_tile();
  const int BN = keys_per_tile(D);
  struct Item { int work, seq, tile; };
  std::vector<Item> items;
  for (int s = 0; s < n_seqs; ++s) {
    const int L = host_cu_seqlens[s + 1] - host_cu_seqlens[s];
    if (L <= 0) return fail(MI_ERR_INVALID, "mi_varlen_schedule: segment %d is empty", s);
    const int tiles = (L + RW - 1) / RW;
    if (tiles > 65535) return fail(MI_ERR_UNSUPPORTED, "mi_varlen_schedule: segment %d too long", s);
    for (int t = 0; t < tiles; ++t) {
      const int end = std::min(L, (t + 1) * RW);
      const int work = causal ? (end + BN - 1) / BN : (L + BN - 1) / BN;
      items.push_back({work, s, t});
    }
  }
  std::stable_sort(items.begin(), items.end(),
                   [](const Item& a, const Item& b) { return a.work > b.work; });
  const int n = int(items.size());
  if (host_schedule != nullptr) {
    if (capacity < n) {
      return fail(MI_ERR_INVALID, "mi_varlen_schedule: capacity %d < %d tiles", capacity, n);
    }
    for (int i = 0; i < n; ++i) host_schedule[i] = (items[i].seq << 16) | items[i].tile;
  }
  return n;
}

extern "C" int mi_varlen_prefill(const void* q, const void* k, const void* v, void* out,
                                 const int32_t* cu_seqlens, int n_seqs, int total_tokens,
                                 int max_seqlen, const int32_t* tile_schedule, int n_tiles, int H,
                                 int H_kv, int D, float scale, int causal, int dtype,
                                 void* stream) {
  using namespace miattn;
  if (dtype != MI_BF16 && dtype != MI_F16) {
    return fail(MI_ERR_UNSUPPORTED,
                "mi_varlen_prefill: the MFMA prefill computes fp16/bf16 only (dtype code %d)", dtype);
  }
  if (H < 1 || H_kv < 1 || H % H_kv != 0) {
    return fail(MI_ERR_INVALID, "mi_varlen_prefill: n_head (%d) must be a multiple of n_kv_head (%d)",
                H, H_kv);
  }
  if (n_seqs < 1 || total_tokens < 1 || max_seqlen < 1 || n_tiles < 1 || n_tiles > 65535) {
    return fail(MI_ERR_INVALID, "mi_varlen_prefill: bad sizes n_seqs=%d total=%d max_seqlen=%d tiles=%d",
                n_seqs, total_tokens, max_seqlen, n_tiles);
  }
  if (q == nullptr || k == nullptr || v == nullptr || out == nullptr || cu_seqlens == nullptr ||
      tile_schedule == nullptr) {
    return fail(MI_ERR_INVALID, "mi_varlen_prefill: NULL pointer argument");
  }
  auto al = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  if (!al(q) || !al(k) || !al(v) || !al(out)) {
    return fail(MI_ERR_UNSUPPORTED, "mi_varlen_prefill: q/k/v/out must be 16-byte aligned");
  }
  const float sl2 = float(double(scale) * 1.4426950408889634);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == MI_BF16) {
    return launch1<bf16_t>(D, q, k, v, out, cu_seqlens, tile_schedule, n_tiles, H, H_kv, sl2,
                           causal, s);
  }
  return launch1<f16_t>(D, q, k, v, out, cu_seqlens, tile_schedule, n_tiles, H, H_kv, sl2,
                        causal, s);
}
