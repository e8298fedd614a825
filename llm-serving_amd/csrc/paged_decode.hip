// Block-table paged-decode GQA attention for gfx950.
//
// Replaces paged_decode / _paged_decode_kernel (reference model/triton_decode.py:250-328,
// :545-643). Same math: one query token per row, fp32 online softmax in the log2 domain
// with scale*log2(e), tail of the last page masked by `token < seqlen`, page walk clamped
// to max_blocks, out = acc / max(l, 1) so an empty row is exact zeros.
//
// Shape of the computation on MI355X:
//   * one workgroup per (split, KV-head group). At the Qwen3 shape the group is all 8 KV
//     heads, so a workgroup sweeps whole pages: one page of the (n_blocks, block_size,
//     H_kv, D) pool is 16 tokens x 8 heads x 256 B = 32 KiB of contiguous K (and the same
//     of V), read once from HBM in coalesced passes. Every query head of a KV head is
//     served by the lanes holding that KV head, so each K/V byte is read once (the
//     reference launches one program per query head and relies on the cache, :33-36);
//   * token-balanced split-K, planned on the device: every workgroup reads the row lengths,
//     sets chunk = ceil(sum(seqlen) / kTargetSplits) (rounded to a batch) and maps its
//     index to (row, split) through a prefix sum of the rows' split counts. Every split
//     therefore carries the same number of tokens however ragged the batch is, the grid
//     (kTargetSplits + B workgroups, sized without a host read of seqlen) fills the 256
//     CUs, and long rows (config 4) and short ones cost the same per token;
//   * lane layout: a (token, KV head) row of D elements is spread over LPR = D*esize/16
//     lanes holding 16 bytes each; a wave-wide 16-byte load covers 64/LPR rows and the
//     four waves of a workgroup cover NR = 4*64/LPR rows = TPL consecutive tokens of the
//     group's KVB heads. q.k is reduced over the LPR lanes with DPP/permlane butterflies;
//     each lane accumulates p*v for its own 16-byte slice of D;
//   * software pipeline: block-table entries are loaded two batches ahead and the K/V
//     registers of the next batch are loaded while the current batch is reduced, so every
//     wave keeps a batch of loads in flight;
//   * a row that fits in one split is finished in place; otherwise each split writes its
//     (m, l, acc) partial to the workspace and a second, small launch folds the partials
//     with a log-sum-exp merge. (An in-kernel "last split merges" counter needs an
//     agent-scope release per workgroup, which on the multi-XCD gfx950 writes back the
//     XCD's L2 each time; measured 3x slower than the extra launch on config 2 even with
//     a release-only fence, 122 vs 39 us per layer.)
//   * K/V are read with the nontemporal hint: each byte is used once, and keeping it out
//     of L2 lifted config 2 from 43.0 to 39.4 us and config 4 from 5.3 to 6.0 TB/s.
// HBM-bound: per (token, KV head) the kernel reads 2 * D * esize bytes of K+V.
#include <mutex>
#include <type_traits>

#include "common.h"

namespace miattn {
namespace {

struct DecodeArgs {
  int B, H, H_kv, G, kvb_log2, n_hchunks, bs_log2, max_blocks, target, slots;
  int64_t qs0, qs1, ks0, ks1, ks2, vs0, vs1, vs2, os0, os1, bts0;
  float scale_log2;
};

// Inputs of the fused form (mi_paged_decode_fused): each row's packed q/k/v projection
// ([q (H x D) | k (H_kv x D) | v (H_kv x D)] with row stride row_stride, as T values or as
// fp32 split-K partials [parts][B][row_stride]), the q/k RMSNorm weights, the RoPE tables
// (n_pos x D/2), each row's position and write slot.
struct FusedArgs {
  const void* qkv;
  int64_t row_stride, plane;
  int parts, slot_bits;
  const void* q_w;
  const void* k_w;
  const void* cos_tab;
  const void* sin_tab;
  int64_t n_pos, n_slots;
  const int64_t* pos;
  const void* slots;
  void* k_pool;  // the layer's pools (the kernel's k/v inputs), written at the new token's slot
  void* v_pool;
  float eps;
  int32_t* err;
};

#ifndef MIATTN_DECODE_THREADS
#define MIATTN_DECODE_THREADS 256
#endif
constexpr int kThreads = MIATTN_DECODE_THREADS;
constexpr int kWaves = kThreads / 64;

// Workgroups a launch aims for: 2 per CU of the 256-CU MI355X, all resident at once.
#ifndef MIATTN_DECODE_TARGET_SPLITS
#define MIATTN_DECODE_TARGET_SPLITS 512
#endif
constexpr int kTargetSplits = MIATTN_DECODE_TARGET_SPLITS;

// Upper bound on the KV heads one workgroup streams side by side.
#ifndef MIATTN_DECODE_KVB_MAX
#define MIATTN_DECODE_KVB_MAX 64
#endif

// Tokens per row state per batch, by query heads per lane: the next batch's K/V
// registers (2 * U * 16 B per lane) are live while the current batch is reduced.
#ifndef MIATTN_DECODE_UNROLL
#define MIATTN_DECODE_UNROLL 4
#endif
// With 4 or 8 query heads per lane each token costs as many dot products and reductions, and
// 2 tokens per batch measured faster than 4 at 4 heads (the Qwen3.5 shape, H 8 / H_kv 2 /
// D 256: 24.1 against 25.8 us per layer on config-2 lengths; 8 tokens: 36.8 us).
constexpr int unroll_for(int GB) {
  return GB <= 2 ? MIATTN_DECODE_UNROLL : 2;
}

template <typename T, int D, int GB>
struct Layout {
  static constexpr int esize = sizeof(T) == 4 ? 4 : 2;
  static constexpr int EPL = 16 / esize;  // elements per lane
  static constexpr int LPR = D / EPL;     // lanes per (token, KV head) row
  static constexpr int RPW = 64 / LPR;    // rows per wave-wide load
  static constexpr int NR = kWaves * RPW; // rows per workgroup-wide load
  static constexpr int U = unroll_for(GB);
  static_assert(LPR >= 1 && LPR <= 64 && (64 % LPR) == 0, "unsupported D/dtype");
};

// K/V are streamed once per launch: optionally read with the nontemporal hint so they do
// not displace the block tables, q and partials in L2.
#ifndef MIATTN_DECODE_NT
#define MIATTN_DECODE_NT 1
#endif
template <typename P>
__device__ __forceinline__ uint4 load_kv(const P* p) {
  if constexpr (MIATTN_DECODE_NT) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
  } else {
    return load16(p);
  }
}

// q.k over one lane's 16-byte slices of q and k, accumulated onto `acc` in order. 16-bit
// types use the packed dot2 instructions (v_dot2c_f32_bf16 / v_dot2c_f32_f16: two
// products of 16-bit inputs, exact in fp32, added in fp32), so k is never unpacked.
template <typename T>
__device__ __forceinline__ float dot16(const uint4& q, const uint4& k, float acc);
template <>
__device__ __forceinline__ float dot16<bf16_t>(const uint4& q, const uint4& k, float acc) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, q.x), __builtin_bit_cast(bf16x2, k.x), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, q.y), __builtin_bit_cast(bf16x2, k.y), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, q.z), __builtin_bit_cast(bf16x2, k.z), acc, false);
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, q.w), __builtin_bit_cast(bf16x2, k.w), acc, false);
}
template <>
__device__ __forceinline__ float dot16<f16_t>(const uint4& q, const uint4& k, float acc) {
  typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
  acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, q.x), __builtin_bit_cast(f16x2, k.x), acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, q.y), __builtin_bit_cast(f16x2, k.y), acc, false);
  acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, q.z), __builtin_bit_cast(f16x2, k.z), acc, false);
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, q.w), __builtin_bit_cast(f16x2, k.w), acc, false);
}
template <>
__device__ __forceinline__ float dot16<float>(const uint4& q, const uint4& k, float acc) {
  acc = fmaf(__uint_as_float(q.x), __uint_as_float(k.x), acc);
  acc = fmaf(__uint_as_float(q.y), __uint_as_float(k.y), acc);
  acc = fmaf(__uint_as_float(q.z), __uint_as_float(k.z), acc);
  return fmaf(__uint_as_float(q.w), __uint_as_float(k.w), acc);
}

// EPL fp32 values -> one 16-byte vector of T (round-to-nearest-even for 16-bit types).
template <typename T>
__device__ __forceinline__ uint4 pack16(const float* v) {
  if constexpr (sizeof(T) == 4) {
    return make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                      __float_as_uint(v[3]));
  } else {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      w[i] = uint32_t(from_f32<T>(v[2 * i]).bits) | (uint32_t(from_f32<T>(v[2 * i + 1]).bits) << 16);
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
}

__device__ __forceinline__ int clamp_len(int len, int capacity) {
  len = len < capacity ? len : capacity;  // page-walk clamp (reference :593)
  return len > 0 ? len : 0;
}

// Tokens per split for a batch holding `total` tokens (identical in both launches).
__device__ __forceinline__ int split_chunk(int total, int batch, int target) {
  int chunk = (total + target - 1) / target;
  chunk = (chunk + batch - 1) / batch * batch;
  return chunk > batch ? chunk : batch;
}

// Inclusive prefix sum over the 64 lanes of a wave, in DPP moves (no LDS round trips):
// shifts by 1, 2, 4 and 8 inside each row of 16 lanes (lanes shifted in from outside the
// row read 0), then lane 15 of rows 0 and 2 added into rows 1 and 3, and lane 31 into rows
// 2 and 3.
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);   // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);   // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);   // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);   // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15 -> rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31 -> rows 2, 3
  return v;
}

// This workgroup's piece of the token-balanced split: row b, split index within the row,
// the row's split count and the global index of its first split. Every wave derives it on
// its own from the row lengths (same inputs, same answer), so planning needs no LDS and no
// barrier; rows are taken 64 at a time, one per lane.
struct SplitInfo {
  int b, split, n_split, first, chunk, len;
};
__device__ __forceinline__ bool plan_split(const int32_t* __restrict__ seqlen, int B, int capacity,
                                           int batch, int target, int w, SplitInfo& si) {
  const int lane = __lane_id();
  // the first 64 rows' lengths are loaded once and serve both passes (one round trip for
  // batches of up to 64 rows)
  const int len_first = lane < B ? clamp_len(seqlen[lane], capacity) : 0;
  int total = __builtin_amdgcn_readlane(wave_inclusive_scan(len_first), 63);
  for (int r0 = 64; r0 < B; r0 += 64) {
    const int row = r0 + lane;
    const int len = row < B ? clamp_len(seqlen[row], capacity) : 0;
    total += __builtin_amdgcn_readlane(wave_inclusive_scan(len), 63);
  }
  const int chunk = split_chunk(total, batch, target);
  int base = 0;  // splits of the rows before this block of 64
  for (int r0 = 0; r0 < B; r0 += 64) {
    const int row = r0 + lane;
    const int len = r0 == 0 ? len_first : row < B ? clamp_len(seqlen[row], capacity) : 0;
    const int n = (len + chunk - 1) / chunk;
    const int incl = wave_inclusive_scan(n);
    const uint64_t owner = __ballot(w >= base + incl - n && w < base + incl);
    if (owner != 0) {
      const int o = __ffsll(static_cast<unsigned long long>(owner)) - 1;
      const int excl = __builtin_amdgcn_readlane(incl - n, o);
      si.b = r0 + o;
      si.split = w - base - excl;
      si.n_split = __builtin_amdgcn_readlane(n, o);
      si.first = base + excl;
      si.chunk = chunk;
      si.len = __builtin_amdgcn_readlane(len, o);  // the row's length, already in lane o
      return true;
    }
    base += __builtin_amdgcn_readlane(incl, 63);
  }
  return false;  // w is past the last split
}

// UP ("uniform pages"): every lane of a wave reads the same token of a workgroup-wide load
// (rows per wave <= KV heads per group, true at the Qwen3 shape), so the block-table
// entries are wave-uniform and read with scalar loads. Those are counted apart from the
// K/V vector loads, so the in-order vector-load counter tracks only K/V batches and the
// reduction of batch i never waits for batch i+1.
template <typename T, int D, int GB, bool UP, bool kFused>
__global__ __launch_bounds__(kThreads) void paged_decode_kernel(
    const T* __restrict__ q, const T* __restrict__ kc, const T* __restrict__ vc,
    const int32_t* __restrict__ block_table, const int32_t* __restrict__ seqlen,
    T* __restrict__ out, int32_t* __restrict__ ws_rows, float* __restrict__ ws_ml,
    float* __restrict__ ws_acc, DecodeArgs a, FusedArgs f) {
  using Lay = Layout<T, D, GB>;
  constexpr int EPL = Lay::EPL, LPR = Lay::LPR, RPW = Lay::RPW, NR = Lay::NR, U = Lay::U;
  extern __shared__ float smem[];  // parked row states: [TPL-1][KVB][GB] (m, l), then acc

  const int tid = threadIdx.x;
  const int KVB = 1 << a.kvb_log2;
  const int TPL = NR >> a.kvb_log2;  // tokens per workgroup-wide load
  const int batch = TPL * U;
  const int capacity = a.max_blocks << a.bs_log2;

  // ---- device-side split plan: total tokens -> chunk -> this workgroup's (row, split)
  SplitInfo si;
  if (!plan_split(seqlen, a.B, capacity, batch, a.target, blockIdx.x, si)) return;  // uniform
  const int b = si.b, split = si.split, n_split_b = si.n_split, first_slot = si.first;
  const int chunk = si.chunk;
  const int len = si.len;
  const int t_begin = split * chunk;
  const int t_end = min(len, t_begin + chunk);
  if (split == 0 && blockIdx.y == 0 && tid == 0) {
    ws_rows[2 * b] = first_slot;  // read by the merge launch (always, so never stale)
    ws_rows[2 * b + 1] = n_split_b;
  }

  const int grp = blockIdx.y / a.n_hchunks;  // KV-head group
  const int hch = blockIdx.y - grp * a.n_hchunks;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r = lane / LPR;          // row within the wave
  const int c = lane - r * LPR;      // 16-byte slice of D within the row
  const int R = wave * RPW + r;      // row state within the workgroup
  const int kvl = R & (KVB - 1);     // KV head within the group
  const int tsub = R >> a.kvb_log2;  // token within a workgroup-wide load
  const int kvh = grp * KVB + kvl;
  const int h0 = kvh * a.G + hch * GB;

  const int32_t* bt_row = block_table + b * a.bts0;
  const int bs_mask = (1 << a.bs_log2) - 1;
  const T* kbase = kc + kvh * a.ks2 + c * EPL;
  const T* vbase = vc + kvh * a.vs2 + c * EPL;
  // UP: every lane of a wave reads the same token, so the page/token part of an address is
  // wave-uniform (scalar registers) and each lane adds a constant 32-bit byte offset (the
  // host checks it fits): the loads take the scalar-base form with no per-load VALU math.
  const uint32_t klane = uint32_t((kvh * a.ks2 + c * EPL) * int64_t(sizeof(T)));
  const uint32_t vlane = uint32_t((kvh * a.vs2 + c * EPL) * int64_t(sizeof(T)));

  // Token u of a batch starting at t0; past t_end it falls back to t_begin (always valid)
  // and is masked out of the softmax.
  auto token = [&](int t0, int u) {
    const int tok = t0 + u * TPL + tsub;
    return tok < t_end ? tok : t_begin;
  };
  auto load_pages = [&](int t0, int (&pg)[U]) {
    if constexpr (UP) {
      const int ts = __builtin_amdgcn_readfirstlane(tsub);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        int tok = t0 + u * TPL + ts;
        tok = tok < t_end ? tok : t_begin;
        pg[u] = bt_row[tok >> a.bs_log2];
      }
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u) pg[u] = bt_row[token(t0, u) >> a.bs_log2];
    }
  };
  auto issue = [&](int t0, const int (&pg)[U], uint4 (&kr)[U], uint4 (&vr)[U]) {
    if constexpr (UP) {
      const int ts = __builtin_amdgcn_readfirstlane(tsub);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        int tok = t0 + u * TPL + ts;
        const int off = (tok < t_end ? tok : t_begin) & bs_mask;
        const char* page = reinterpret_cast<const char*>(kc + (int64_t(pg[u]) * a.ks0 + off * a.ks1));
        kr[u] = load_kv(page + klane);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        int tok = t0 + u * TPL + ts;
        const int off = (tok < t_end ? tok : t_begin) & bs_mask;
        const char* page = reinterpret_cast<const char*>(vc + (int64_t(pg[u]) * a.vs0 + off * a.vs1));
        vr[u] = load_kv(page + vlane);
      }
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int off = token(t0, u) & bs_mask;
        kr[u] = load_kv(kbase + int64_t(pg[u]) * a.ks0 + off * a.ks1);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int off = token(t0, u) & bs_mask;
        vr[u] = load_kv(vbase + int64_t(pg[u]) * a.vs0 + off * a.vs1);
      }
    }
    // keep each batch's loads together and in program order (see the pipeline below)
    __builtin_amdgcn_sched_barrier(0);
  };

  uint4 qr[GB];
  // Fused form: the row's new token (position len - 1, the last of the last split) has its
  // k and v computed here and kept in registers; the split's masked final batch reads them
  // instead of the pool, which this workgroup writes them to (no other workgroup reads
  // that token, so nothing waits for the write).
  int t_new = -1;
  uint4 k_new = make_uint4(0u, 0u, 0u, 0u), v_new = make_uint4(0u, 0u, 0u, 0u);
  // fused form, first half: every input load, none of them waiting on another (the row's
  // position and slot, its projection columns, the norm weights); the second half, after
  // the first K/V batches are issued, loads the RoPE rows at the position and computes.
  constexpr int kNX = GB + 2;  // q heads, then this lane's KV head's k and v
  float4 raw[kNX][2][2];       // [input][partial 0 / 1][elements 0-3 / 4-7]
  int64_t f_pb = 0, f_sl = -1;
  uint4 wq = make_uint4(0u, 0u, 0u, 0u), wk = wq, cv = wq, sv = wq;
  const bool last_split = t_end == len;
  auto col_of = [&](int ix) {
    return ix < GB ? (h0 + ix) * D : ix == GB ? (a.H + kvh) * D : (a.H + a.H_kv + kvh) * D;
  };
  if constexpr (!kFused) {
#pragma unroll
    for (int g = 0; g < GB; ++g) qr[g] = load16(q + b * a.qs0 + (h0 + g) * a.qs1 + c * EPL);
  } else {
    static_assert(D == 128 && EPL == 8 && LPR == 16, "fused form: head_dim 128, 16-bit types");
    f_pb = f.pos[b];
    f_sl = f.slot_bits == 32 ? int64_t(static_cast<const int32_t*>(f.slots)[b]) : static_cast<const int64_t*>(f.slots)[b];
    const int ps = f.parts > 0 ? f.parts : 1;
#pragma unroll
    for (int ix = 0; ix < kNX; ++ix) {
      if (ix >= GB && !last_split) break;
      const int64_t off = b * f.row_stride + col_of(ix) + c * EPL;
      if (f.parts == 0) {
        const uint4 w = load16(static_cast<const T*>(f.qkv) + off);
        raw[ix][0][0] = make_float4(__uint_as_float(w.x), __uint_as_float(w.y), __uint_as_float(w.z),
                                    __uint_as_float(w.w));
      } else {
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
          const float* fp = static_cast<const float*>(f.qkv) + int64_t(pp < ps ? pp : ps - 1) * f.plane + off;
          raw[ix][pp][0] = *reinterpret_cast<const float4*>(fp);
          raw[ix][pp][1] = *reinterpret_cast<const float4*>(fp + 4);
        }
      }
    }
    wq = load16(static_cast<const T*>(f.q_w) + c * EPL);
    wk = load16(static_cast<const T*>(f.k_w) + c * EPL);
    // the RoPE rows at the position the contract gives (len - 1), loaded without waiting for
    // pos[b]; a row whose pos differs is refused below and never uses them
    int64_t prow = int64_t(len) - 1;
    prow = prow < f.n_pos ? prow : f.n_pos - 1;
    prow = prow > 0 ? prow : 0;
    cv = load16(static_cast<const T*>(f.cos_tab) + prow * (D / 2) + (c & 7) * EPL);
    sv = load16(static_cast<const T*>(f.sin_tab) + prow * (D / 2) + (c & 7) * EPL);
  }
  // fused form, second half. q/k RMSNorm + RoPE, op by op as mi_qk_norm_rope_write
  // computes them, in this kernel's lane layout: a head row is one 16-lane DPP row, lane c
  // holding elements 8c .. 8c + 7. The sum of squares reproduces that kernel's 64-lane
  // butterfly exactly: its lane l holds rt(x_l^2) + rt(x_{l+64}^2), here the pair (lane c,
  // lane c + 8) forms those eight sums for l = 8(c mod 8) + j, the butterfly's levels 1-3
  // (l ^ 1, ^ 2, ^ 4) are the in-lane tree over j and its levels 4-6 (l ^ 8, ^ 16, ^ 32) the
  // 8-lane butterfly over c. The RoPE partner of element e (e +- 64) is lane c ^ 8's element j.
  auto fused_finish = [&]() {
    if constexpr (kFused) {
      const bool idle = f_sl == -1;
      const bool ok = !idle && f_pb >= 0 && f_pb < f.n_pos && f_sl >= 0 && f_sl < f.n_slots && f_pb == int64_t(len) - 1;
      if (!idle && !ok && split == 0 && blockIdx.y == 0 && tid == 0 && f.err != nullptr) atomicCAS(f.err, 0, b + 1);
      // input ix as T values (split-K partials summed in split order, rounded once)
      auto values = [&](int ix, float (&x)[EPL]) {
        if (f.parts == 0) {
          const uint4 w = make_uint4(__float_as_uint(raw[ix][0][0].x), __float_as_uint(raw[ix][0][0].y),
                                     __float_as_uint(raw[ix][0][0].z), __float_as_uint(raw[ix][0][0].w));
  #pragma unroll
          for (int j = 0; j < EPL; ++j) x[j] = Vec16<T>::get(w, j);
        } else {
          float s8[EPL] = {raw[ix][0][0].x, raw[ix][0][0].y, raw[ix][0][0].z, raw[ix][0][0].w,
                           raw[ix][0][1].x, raw[ix][0][1].y, raw[ix][0][1].z, raw[ix][0][1].w};
          if (f.parts > 1) {
            const float p1[EPL] = {raw[ix][1][0].x, raw[ix][1][0].y, raw[ix][1][0].z, raw[ix][1][0].w,
                                   raw[ix][1][1].x, raw[ix][1][1].y, raw[ix][1][1].z, raw[ix][1][1].w};
  #pragma unroll
            for (int j = 0; j < EPL; ++j) s8[j] += p1[j];
          }
          for (int pp = 2; pp < f.parts; ++pp) {
            const float* fp = static_cast<const float*>(f.qkv) + int64_t(pp) * f.plane + b * f.row_stride + col_of(ix) +
                              c * EPL;
  #pragma unroll
            for (int j = 0; j < EPL; ++j) s8[j] += fp[j];
          }
  #pragma unroll
          for (int j = 0; j < EPL; ++j) x[j] = rt<T>(s8[j]);
        }
      };
      auto norm_rope = [&](float (&x)[EPL], const uint4& w) {
        float v8[EPL];
  #pragma unroll
        for (int j = 0; j < EPL; ++j) {
          const float sq = rt<T>(x[j] * x[j]);
          v8[j] = sq + dpp<kDppRowRor8>(sq);
        }
        float ss = ((v8[0] + v8[1]) + (v8[2] + v8[3])) + ((v8[4] + v8[5]) + (v8[6] + v8[7]));
        ss = group_allreduce<8, SumOp>(ss);
        const float ms = rt<T>(ss * (1.0f / D));
        const float rms = rt<T>(sqrtf(rt<T>(ms + f.eps)));
        float y[EPL], o[EPL];
  #pragma unroll
        for (int j = 0; j < EPL; ++j) y[j] = rt<T>(rt<T>(x[j] / rms) * Vec16<T>::get(w, j));
  #pragma unroll
        for (int j = 0; j < EPL; ++j) {
          const float partner = dpp<kDppRowRor8>(y[j]);
          const float cs = Vec16<T>::get(cv, j), sn = Vec16<T>::get(sv, j);
          o[j] = c < 8 ? rt<T>(rt<T>(y[j] * cs) - rt<T>(partner * sn)) : rt<T>(rt<T>(partner * sn) + rt<T>(y[j] * cs));
        }
        return pack16<T>(o);
      };
      if (ok) {
  #pragma unroll
        for (int g = 0; g < GB; ++g) {
          float x[EPL];
          values(g, x);
          qr[g] = norm_rope(x, wq);
        }
      } else {
        // a row whose epilogue inputs are refused attends with q = 0, as the two-launch form
        // (mi_qk_norm_rope_write leaves zeros in q_out) does
  #pragma unroll
        for (int g = 0; g < GB; ++g) qr[g] = make_uint4(0u, 0u, 0u, 0u);
      }
      if (ok && last_split) {
        float xk[EPL], xv[EPL];
        values(GB, xk);
        values(GB + 1, xv);
        k_new = norm_rope(xk, wk);
        v_new = pack16<T>(xv);
        t_new = len - 1;
        if (tsub == t_new % TPL && hch == 0) {
          const int64_t blk = f_sl >> a.bs_log2, in_blk = f_sl & ((1 << a.bs_log2) - 1);
          store16(static_cast<T*>(f.k_pool) + blk * a.ks0 + in_blk * a.ks1 + kvh * a.ks2 + c * EPL, k_new);
          store16(static_cast<T*>(f.v_pool) + blk * a.vs0 + in_blk * a.vs1 + kvh * a.vs2 + c * EPL, v_new);
        }
      }
    }
  };

  float m[GB], l[GB], acc[GB][EPL];
#pragma unroll
  for (int g = 0; g < GB; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[g][e] = 0.0f;
  }

  // Online softmax over one batch of U tokens per row state. Only a split's last batch
  // can hold tokens past t_end, so the steady-state loop runs the unmasked form.
  auto compute = [&](int t0, const uint4 (&kr)[U], const uint4 (&vr)[U], auto masked) {
    __builtin_amdgcn_sched_barrier(0);
    float s[U][GB];
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int g = 0; g < GB; ++g) {
        uint4 kk = kr[u];
        if constexpr (kFused && decltype(masked)::value) {
          if (t0 + u * TPL + tsub == t_new) kk = k_new;
        }
        float dot = dot16<T>(qr[g], kk, 0.0f);
        dot = group_allreduce<LPR, SumOp>(dot);
        s[u][g] = dot * a.scale_log2;
        if constexpr (decltype(masked)::value) {
          if (t0 + u * TPL + tsub >= t_end) s[u][g] = -INFINITY;
        }
      }
    }
#pragma unroll
    for (int g = 0; g < GB; ++g) {
      float mb = s[0][g];
#pragma unroll
      for (int u = 1; u < U; ++u) mb = fmaxf(mb, s[u][g]);
      const float m_new = fmaxf(m[g], mb);
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      const float alpha = fast_exp2(m[g] - m_use);
      m[g] = m_new;
      float lsum_g = l[g] * alpha;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[g][e] *= alpha;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float p = fast_exp2(s[u][g] - m_use);
        lsum_g += p;
        uint4 vv = vr[u];
        if constexpr (kFused && decltype(masked)::value) {
          if (t0 + u * TPL + tsub == t_new) vv = v_new;
        }
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] = fmaf(p, Vec16<T>::get(vv, e), acc[g][e]);
      }
      l[g] = lsum_g;
    }
  };

  // Software pipeline with two statically named register sets (A, B) and the loop
  // unrolled by two: while batch i is reduced, batch i+1 is in flight, and the block-table
  // entries of the batch after are loaded one step ahead of its K/V. Inside the loop every
  // issue is unconditional (the bound guarantees the batch exists), so the compiler can
  // wait for exactly the batch being reduced; a copy between sets or a conditional issue
  // makes it wait for all loads in flight. Loads past t_end are harmless: token() clamps
  // them to t_begin, a valid token of this split (the plan gives no workgroup an empty
  // range), and compute() masks them out.
  const int n_b = (t_end - t_begin + batch - 1) / batch;
  int pgA[U], pgB[U];
  uint4 kA[U], vA[U], kB[U], vB[U];
  load_pages(t_begin, pgA);
  load_pages(t_begin + batch, pgB);
  if constexpr (UP) {
    // all 2U block-table loads go out before the first wait (left alone, the compiler
    // waits after each scalar load: 2U round trips before the first K/V load, not one)
    if constexpr (U == 4) {
      asm volatile("" : "+s"(pgA[0]), "+s"(pgA[1]), "+s"(pgA[2]), "+s"(pgA[3]), "+s"(pgB[0]),
                        "+s"(pgB[1]), "+s"(pgB[2]), "+s"(pgB[3]));
    } else if constexpr (U == 2) {
      asm volatile("" : "+s"(pgA[0]), "+s"(pgA[1]), "+s"(pgB[0]), "+s"(pgB[1]));
    }
  }
  issue(t_begin, pgA, kA, vA);
  issue(t_begin + batch, pgB, kB, vB);  // unconditional (see above); n_b >= 1 always
  load_pages(t_begin + 2 * batch, pgA);
  if constexpr (kFused) fused_finish();  // q (and the new token's k/v) while the batches land
  int i = 0;
  for (; i + 2 < n_b; i += 2) {
    const int t0 = t_begin + i * batch;
    compute(t0, kA, vA, std::false_type{});
    load_pages(t0 + 3 * batch, pgB);
    issue(t0 + 2 * batch, pgA, kA, vA);
    compute(t0 + batch, kB, vB, std::false_type{});
    load_pages(t0 + 4 * batch, pgA);
    issue(t0 + 3 * batch, pgB, kB, vB);
  }
  // One or two batches left: A holds batch i, B batch i+1 (past n_b B's loads were
  // clamped and are dropped). No issue is conditional, so nothing gets sunk into a branch.
  compute(t_begin + i * batch, kA, vA, std::true_type{});
  if (n_b - i == 2) compute(t_begin + (i + 1) * batch, kB, vB, std::true_type{});

  // Fold the TPL row states of each (KV head, query head, 16-byte slice) together: rows
  // with tsub > 0 park theirs in LDS, rows with tsub == 0 merge them in registers and write
  // whole 16-byte pieces of the output (or of the split's partial).
  if (TPL > 1) {
    float* sm_ml = smem;                             // [TPL-1][KVB][GB][2]
    float* sm_acc = smem + (((TPL - 1) * KVB * GB * 2 + 3) & ~3);  // 16 B aligned: [TPL-1][KVB][GB][LPR][EPL]
    if (tsub > 0) {
#pragma unroll
      for (int g = 0; g < GB; ++g) {
        const int slot = ((tsub - 1) * KVB + kvl) * GB + g;
        if (c == 0) *reinterpret_cast<float2*>(sm_ml + slot * 2) = make_float2(m[g], l[g]);
        float4* dst = reinterpret_cast<float4*>(sm_acc + (slot * LPR + c) * EPL);
#pragma unroll
        for (int e = 0; e < EPL; e += 4) dst[e / 4] = make_float4(acc[g][e], acc[g][e + 1], acc[g][e + 2], acc[g][e + 3]);
      }
    }
    __syncthreads();
    if (tsub > 0) return;  // no barrier follows
    for (int ts = 1; ts < TPL; ++ts) {
#pragma unroll
      for (int g = 0; g < GB; ++g) {
        const int slot = ((ts - 1) * KVB + kvl) * GB + g;
        const float2 ml2 = *reinterpret_cast<const float2*>(sm_ml + slot * 2);
        const float M = fmaxf(m[g], ml2.x);
        const float Mu = M == -INFINITY ? 0.0f : M;
        const float w0 = fast_exp2(m[g] - Mu), w1 = fast_exp2(ml2.x - Mu);
        m[g] = M;
        l[g] = fmaf(l[g], w0, ml2.y * w1);
        const float4* src = reinterpret_cast<const float4*>(sm_acc + (slot * LPR + c) * EPL);
#pragma unroll
        for (int e = 0; e < EPL; e += 4) {
          const float4 o = src[e / 4];
          acc[g][e + 0] = fmaf(acc[g][e + 0], w0, o.x * w1);
          acc[g][e + 1] = fmaf(acc[g][e + 1], w0, o.y * w1);
          acc[g][e + 2] = fmaf(acc[g][e + 2], w0, o.z * w1);
          acc[g][e + 3] = fmaf(acc[g][e + 3], w0, o.w * w1);
        }
      }
    }
  }

#pragma unroll
  for (int g = 0; g < GB; ++g) {
    const int h = h0 + g;
    if (n_split_b <= 1) {
      const float inv = 1.0f / fmaxf(l[g], 1.0f);
      float o[EPL];
#pragma unroll
      for (int e = 0; e < EPL; ++e) o[e] = acc[g][e] * inv;
      store16(out + b * a.os0 + h * a.os1 + c * EPL, pack16<T>(o));
    } else {
      // [head][slot]: the partials of one (row, head) are contiguous for the merge
      const int64_t ph = int64_t(h) * a.slots + first_slot + split;
      float4* dst = reinterpret_cast<float4*>(ws_acc + ph * D + c * EPL);
#pragma unroll
      for (int e = 0; e < EPL; e += 4) dst[e / 4] = make_float4(acc[g][e], acc[g][e + 1], acc[g][e + 2], acc[g][e + 3]);
      if (c == 0) *reinterpret_cast<float2*>(ws_ml + ph * 2) = make_float2(m[g], l[g]);
    }
  }
}

// Eight asm operands x[o] .. x[o + 7] with constraint C.
#define MI_PIN8(C, x, o)                                                                 \
  C(x[o]), C(x[o + 1]), C(x[o + 2]), C(x[o + 3]), C(x[o + 4]), C(x[o + 5]), C(x[o + 6]), \
      C(x[o + 7])

// Second launch, one workgroup per (query head, row), one thread per element of D:
// zero-length rows get exact zeros; rows split over several workgroups get the
// log-sum-exp merge of their partials, folded online (running max) 32 splits at a time --
// no LDS, no barrier. Three round trips: the arguments, then the row's length with its
// (first slot, split count) record written by the first launch, then the partials of up to
// 32 splits at once (lane j of each 32-lane half loads split j's (m, l), every thread the
// 32 elements of its d); rows of more than 32 splits take one more per 32. Single-split
// rows were finished by the first launch.
template <typename T, int D>
__global__ __launch_bounds__(256) void paged_decode_merge_kernel(
    const int32_t* __restrict__ seqlen, const int32_t* __restrict__ ws_rows,
    const float* __restrict__ ws_ml, const float* __restrict__ ws_acc, T* __restrict__ out,
    DecodeArgs a) {
  constexpr int kChunk = 32;  // one split per lane of a 32-lane half; the pin names 32
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int d = threadIdx.x;  // the launch has max(D, 64) threads: whole waves
  const int lane = d & 63;
  const int capacity = a.max_blocks << a.bs_log2;
  // the arguments on other kernarg lines than the row pointers' are loaded with those
  // (left alone, the compiler loads them after the row's record, each line a scalar-cache
  // miss of its own)
  asm volatile("" ::"s"(a.slots), "s"(a.os0), "s"(a.os1), "s"(capacity));
  // the row's length and its record go out together, one round trip (left alone, the
  // compiler loads the record only after the length's branch: two more)
  int len_raw = seqlen[b];
  int first = ws_rows[2 * b];
  int n_split = ws_rows[2 * b + 1];
  asm volatile("" : "+s"(len_raw), "+s"(first), "+s"(n_split));
  const int len = clamp_len(len_raw, capacity);
  T* orow = out + b * a.os0 + h * a.os1;
  if (len == 0) {
    if (d < D) orow[d] = from_f32<T>(0.0f);
    return;
  }
  if (n_split <= 1) return;
  // threads past D (D < 64) take part in the lane reductions and store nothing
  const int dl = d < D ? d : D - 1;
  const float* ml = ws_ml + (int64_t(h) * a.slots + first) * 2;  // [head][slot] layout
  const float* acc = ws_acc + (int64_t(h) * a.slots + first) * D + dl;
  float M = -INFINITY, Ls = 0.0f, As = 0.0f;
  for (int s0 = 0; s0 < n_split; s0 += kChunk) {
    const int js = s0 + (lane & (kChunk - 1));
    // past the row's last split the loads repeat it (valid memory); weighted out below
    const float2 mlj = *reinterpret_cast<const float2*>(ml + min(js, n_split - 1) * 2);
    float mx = mlj.x, lx = mlj.y;
    float v[kChunk];
#pragma unroll
    for (int j = 0; j < kChunk; ++j) v[j] = acc[int64_t(min(s0 + j, n_split - 1)) * D];
    // every load of the chunk is issued before the first wait
    asm volatile("" : "+v"(mx), "+v"(lx), MI_PIN8("+v", v, 0), MI_PIN8("+v", v, 8),
                      MI_PIN8("+v", v, 16), MI_PIN8("+v", v, 24));
    const bool valid = js < n_split;
    const float Mc = fmaxf(M, group_allreduce<kChunk, MaxOp>(valid ? mx : -INFINITY));
    const float Mu = Mc == -INFINITY ? 0.0f : Mc;
    const float r = fast_exp2(M - Mu);
    const float w = valid ? fast_exp2(mx - Mu) : 0.0f;  // split js's weight, in its lane
    Ls = fmaf(Ls, r, group_allreduce<kChunk, SumOp>(lx * w));
    As *= r;
#pragma unroll
    for (int j = 0; j < kChunk; ++j) {
      const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), j));
      As = fmaf(v[j], wj, As);
    }
    M = Mc;
  }
  if (d < D) orow[d] = from_f32<T>(As / fmaxf(Ls, 1.0f));
}
#undef MI_PIN8

int ilog2_exact(int x) {
  int lg = 0;
  while ((1 << lg) < x) ++lg;
  return (1 << lg) == x ? lg : -1;
}

bool supported_d(int D) { return D == 16 || D == 32 || D == 64 || D == 128 || D == 256; }

int esize_of(int dtype) { return dtype == MI_F32 ? 4 : (dtype == MI_F16 || dtype == MI_BF16) ? 2 : 0; }

int lowbit(int x) { return x & -x; }

// Launch geometry, computed identically by the workspace query and the launcher.
struct Plan {
  int GB, n_hchunks, KVB, kvb_log2, n_groups, NR, TPL, U, target, slots;
  size_t rows_bytes, ml_bytes, acc_bytes;
  size_t smem_bytes;
};

Plan make_plan(int B, int H, int H_kv, int D, int block_size, int max_blocks, int dtype) {
  Plan p{};
  const int es = esize_of(dtype);
  const int lpr = D * es / 16;
  p.NR = kWaves * (64 / lpr);
  const int G = H / H_kv;
  // Query heads per lane: the largest of 8/4/2/1 dividing G whose LDS merge buffer fits
  // in 64 KiB.
  p.GB = 1;
  for (int gb = 8; gb >= 1; gb /= 2) {
    if (G % gb == 0 && size_t(p.NR) * gb * (D + 2) * 4 <= 65536) {
      p.GB = gb;
      break;
    }
  }
  p.n_hchunks = G / p.GB;
  p.KVB = lowbit(H_kv) < p.NR ? lowbit(H_kv) : p.NR;
  p.KVB = p.KVB < MIATTN_DECODE_KVB_MAX ? p.KVB : MIATTN_DECODE_KVB_MAX;
  p.kvb_log2 = ilog2_exact(p.KVB);
  p.n_groups = H_kv / p.KVB;
  p.TPL = p.NR / p.KVB;
  p.U = unroll_for(p.GB);
  // Each of the n_groups * n_hchunks workgroup columns splits the same token ranges, so
  // the split target is shared out among them. Splits never exceed target + B: chunk >=
  // total / target, and each row adds at most one partial split.
  const int cols = p.n_groups * p.n_hchunks;
  p.target = kTargetSplits / cols > 0 ? kTargetSplits / cols : 1;
  p.slots = p.target + B;
  // parked row states of the tsub > 0 rows: (m, l) pairs padded to 16 bytes, then acc
  const size_t parked = size_t(p.TPL - 1) * p.KVB * p.GB;
  p.smem_bytes = ((parked * 2 + 3) / 4 * 4 + parked * D) * sizeof(float);
  p.rows_bytes = (size_t(B) * 2 * sizeof(int32_t) + 255) / 256 * 256;
  p.ml_bytes = (size_t(p.slots) * H * 2 * sizeof(float) + 255) / 256 * 256;
  p.acc_bytes = size_t(p.slots) * H * D * sizeof(float);
  return p;
}

template <typename T, int D, int GB>
int launch_typed(const void* q, const void* kc, const void* vc, const int32_t* bt,
                 const int32_t* seqlen, void* out, int32_t* ws_rows, float* ws_ml,
                 float* ws_acc, const DecodeArgs& a, const Plan& p, const FusedArgs* fa, hipStream_t stream) {
  if (Layout<T, D, GB>::U != p.U || Layout<T, D, GB>::NR != p.NR) {
    return fail(MI_ERR_UNSUPPORTED, "mi_paged_decode: internal launch-geometry mismatch");
  }
  dim3 grid(p.slots, p.n_groups * p.n_hchunks);
  // Wave-uniform pages need every wave inside one token (RPW <= KVB) and the lane byte
  // offsets within 32 bits.
  const int64_t lane_span = (int64_t(a.H_kv) * std::max(a.ks2, a.vs2) + D) * int64_t(sizeof(T));
  const bool up = Layout<T, D, GB>::RPW <= p.KVB && a.ks2 >= 0 && a.vs2 >= 0 && lane_span < (int64_t(1) << 31);
  auto go = [&](auto up_c, auto fused_c) {
    hipLaunchKernelGGL((paged_decode_kernel<T, D, GB, decltype(up_c)::value, decltype(fused_c)::value>), grid,
                       dim3(kThreads), p.smem_bytes, stream, static_cast<const T*>(q), static_cast<const T*>(kc),
                       static_cast<const T*>(vc), bt, seqlen, static_cast<T*>(out), ws_rows, ws_ml, ws_acc, a,
                       fa != nullptr ? *fa : FusedArgs{});
  };
  using Yes = std::true_type;
  using No = std::false_type;
  if (fa != nullptr) {
    // the fused form exists for head_dim 128 in 16-bit types (the callers check)
    if constexpr (D == 128 && sizeof(T) == 2) {
      if (up) go(Yes{}, Yes{}); else go(No{}, Yes{});
    } else {
      return fail(MI_ERR_UNSUPPORTED, "mi_paged_decode_fused: no fused kernel for head_dim %d", D);
    }
  } else {
    if (up) go(Yes{}, No{}); else go(No{}, No{});
  }
  int rc = launch_status("mi_paged_decode (split kernel)");
  if (rc != MI_OK) return rc;
  const int threads = D > 64 ? D : 64;
  hipLaunchKernelGGL((paged_decode_merge_kernel<T, D>), dim3(a.H, a.B), dim3(threads), 0, stream,
                     seqlen, ws_rows, ws_ml, ws_acc, static_cast<T*>(out), a);
  return launch_status("mi_paged_decode (merge kernel)");
}

template <typename T, int D>
int dispatch_gb(const void* q, const void* kc, const void* vc, const int32_t* bt,
                const int32_t* seqlen, void* out, int32_t* ws_rows, float* ws_ml, float* ws_acc,
                const DecodeArgs& a, const Plan& p, const FusedArgs* fa, hipStream_t s) {
  switch (p.GB) {
    case 1: return launch_typed<T, D, 1>(q, kc, vc, bt, seqlen, out, ws_rows, ws_ml, ws_acc, a, p, fa, s);
    case 2: return launch_typed<T, D, 2>(q, kc, vc, bt, seqlen, out, ws_rows, ws_ml, ws_acc, a, p, fa, s);
    case 4: return launch_typed<T, D, 4>(q, kc, vc, bt, seqlen, out, ws_rows, ws_ml, ws_acc, a, p, fa, s);
    case 8: return launch_typed<T, D, 8>(q, kc, vc, bt, seqlen, out, ws_rows, ws_ml, ws_acc, a, p, fa, s);
  }
  return fail(MI_ERR_UNSUPPORTED, "mi_paged_decode: no kernel for %d heads per lane", p.GB);
}

template <typename T>
int dispatch_d(int D, const void* q, const void* kc, const void* vc, const int32_t* bt,
               const int32_t* seqlen, void* out, int32_t* ws_rows, float* ws_ml, float* ws_acc,
               const DecodeArgs& a, const Plan& p, const FusedArgs* fa, hipStream_t s) {
  switch (D) {
    case 16:
      if constexpr (sizeof(T) == 2) return dispatch_gb<T, 16>(q, kc, vc, bt, seqlen, out, ws_rows, ws_ml, ws_acc, a, p, fa, s);
      break;
    case 32: return dispatch_gb<T, 32>(q, kc, vc, bt, seqlen, out, ws_rows, ws_ml, ws_acc, a, p, fa, s);
    case 64: return dispatch_gb<T, 64>(q, kc, vc, bt, seqlen, out, ws_rows, ws_ml, ws_acc, a, p, fa, s);
    case 128: return dispatch_gb<T, 128>(q, kc, vc, bt, seqlen, out, ws_rows, ws_ml, ws_acc, a, p, fa, s);
    case 256: return dispatch_gb<T, 256>(q, kc, vc, bt, seqlen, out, ws_rows, ws_ml, ws_acc, a, p, fa, s);
  }
  return fail(MI_ERR_UNSUPPORTED,
              "mi_paged_decode: head_dim %d is not supported by the HIP decode kernel "
              "(supported: 32, 64, 128, 256; 16 for fp16/bf16)",
              D);
}

bool shape_ok(int B, int H, int H_kv, int D, int block_size, int max_blocks, int dtype) {
  return B > 0 && H > 0 && H_kv > 0 && H % H_kv == 0 && ilog2_exact(block_size) >= 0 &&
         max_blocks > 0 && esize_of(dtype) != 0 && supported_d(D) && !(D == 16 && dtype == MI_F32);
}

}  // namespace
}  // namespace miattn

extern "C" size_t mi_paged_decode_workspace_size(int B, int H, int H_kv, int D, int block_size,
                                                 int max_blocks, int dtype) {
  using namespace miattn;
  if (!shape_ok(B, H, H_kv, D, block_size, max_blocks, dtype)) return 0;
  const Plan p = make_plan(B, H, H_kv, D, block_size, max_blocks, dtype);
  return p.rows_bytes + p.ml_bytes + p.acc_bytes;
}

namespace miattn {
namespace {

// The body of both decode entry points; `workspace` is the caller's (mi_paged_decode) or
// this GPU's scratch array (mi_paged_decode_noalloc).
int paged_decode_entry(const void* q, const void* k_cache, const void* v_cache, const int32_t* block_table,
                       const int32_t* seqlen, void* out, int B, int H, int H_kv, int D, int block_size,
                       int max_blocks, const int64_t* strides, float scale, int dtype, void* workspace,
                       size_t workspace_bytes, void* stream, FusedArgs* fa = nullptr) {
  if (esize_of(dtype) == 0) return fail(MI_ERR_INVALID, "mi_paged_decode: unknown dtype %d", dtype);
  if (B < 0 || H < 1 || H_kv < 1 || H % H_kv != 0) {
    return fail(MI_ERR_INVALID, "mi_paged_decode: n_head (%d) must be a multiple of n_kv_head (%d)",
                H, H_kv);
  }
  const int bs_log2 = ilog2_exact(block_size);
  if (bs_log2 < 0) {
    return fail(MI_ERR_INVALID, "mi_paged_decode: block_size must be a power of two, got %d",
                block_size);
  }
  if (max_blocks < 1) return fail(MI_ERR_INVALID, "mi_paged_decode: max_blocks must be >= 1");
  if (!supported_d(D) || (D == 16 && dtype == MI_F32)) {
    return fail(MI_ERR_UNSUPPORTED,
                "mi_paged_decode: head_dim %d is not supported by the HIP decode kernel "
                "(supported: 32, 64, 128, 256; 16 for fp16/bf16)",
                D);
  }
  if (strides == nullptr) return fail(MI_ERR_INVALID, "mi_paged_decode: strides is NULL");
  if (B == 0) return MI_OK;
  if ((long long)max_blocks * block_size * B > 2147483647LL) {
    return fail(MI_ERR_UNSUPPORTED,
                "mi_paged_decode: B * max_blocks * block_size must stay below 2^31 tokens");
  }
  const int64_t* st = strides;
  // 16-byte vector access needs a contiguous head_dim and 16-byte aligned rows.
  const int es = esize_of(dtype);
  auto al = [&](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  const bool rows_ok = st[2] == 1 && st[6] == 1 && st[10] == 1 && st[13] == 1;
  const bool strides_ok = (st[0] * es) % 16 == 0 && (st[1] * es) % 16 == 0 &&
                          (st[3] * es) % 16 == 0 && (st[4] * es) % 16 == 0 &&
                          (st[5] * es) % 16 == 0 && (st[7] * es) % 16 == 0 &&
                          (st[8] * es) % 16 == 0 && (st[9] * es) % 16 == 0 &&
                          (st[11] * es) % 16 == 0 && (st[12] * es) % 16 == 0;
  if (!rows_ok || !strides_ok || !al(q) || !al(k_cache) || !al(v_cache) || !al(out)) {
    return fail(MI_ERR_UNSUPPORTED,
                "mi_paged_decode: q/k_cache/v_cache/out need a contiguous, 16-byte aligned head_dim "
                "(strides q=%lld,%lld,%lld k=%lld,%lld,%lld,%lld)",
                (long long)st[0], (long long)st[1], (long long)st[2], (long long)st[3],
                (long long)st[4], (long long)st[5], (long long)st[6]);
  }
  const Plan p = make_plan(B, H, H_kv, D, block_size, max_blocks, dtype);
  if (p.n_groups * p.n_hchunks > 65535 || B > 65535 || H > 65535) {
    return fail(MI_ERR_UNSUPPORTED, "mi_paged_decode: grid too large (B=%d, H=%d)", B, H);
  }
  const size_t need = p.rows_bytes + p.ml_bytes + p.acc_bytes;
  if (workspace == nullptr || workspace_bytes < need) {
    return fail(MI_ERR_WORKSPACE, "mi_paged_decode: workspace of %zu bytes < %zu needed",
                workspace_bytes, need);
  }
  if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0) {
    return fail(MI_ERR_WORKSPACE, "mi_paged_decode: workspace must be 16-byte aligned");
  }
  int32_t* ws_rows = static_cast<int32_t*>(workspace);
  float* ws_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) + p.rows_bytes);
  float* ws_acc = ws_ml + p.ml_bytes / sizeof(float);

  DecodeArgs a;
  a.B = B; a.H = H; a.H_kv = H_kv; a.G = H / H_kv; a.kvb_log2 = p.kvb_log2;
  a.n_hchunks = p.n_hchunks; a.bs_log2 = bs_log2;
  a.max_blocks = max_blocks; a.target = p.target; a.slots = p.slots;
  a.qs0 = st[0]; a.qs1 = st[1];
  a.ks0 = st[3]; a.ks1 = st[4]; a.ks2 = st[5];
  a.vs0 = st[7]; a.vs1 = st[8]; a.vs2 = st[9];
  a.os0 = st[11]; a.os1 = st[12];
  a.bts0 = st[14];
  a.scale_log2 = scale * 1.4426950408889634f;

  hipStream_t s = static_cast<hipStream_t>(stream);
  if (fa != nullptr) {
    fa->k_pool = const_cast<void*>(k_cache);
    fa->v_pool = const_cast<void*>(v_cache);
  }
  switch (dtype) {
    case MI_F32: return dispatch_d<float>(D, q, k_cache, v_cache, block_table, seqlen, out, ws_rows, ws_ml, ws_acc, a, p, fa, s);
    case MI_F16: return dispatch_d<f16_t>(D, q, k_cache, v_cache, block_table, seqlen, out, ws_rows, ws_ml, ws_acc, a, p, fa, s);
    case MI_BF16: return dispatch_d<bf16_t>(D, q, k_cache, v_cache, block_table, seqlen, out, ws_rows, ws_ml, ws_acc, a, p, fa, s);
  }
  return fail(MI_ERR_INVALID, "mi_paged_decode: unknown dtype %d", dtype);
}

}  // namespace
}  // namespace miattn

// Split-K scratch of mi_paged_decode_noalloc: one array per GPU, held until the process
// ends. Its name is a host-side stand-in; device code gets the address that
// hipGetSymbolAddress returns for the current device (decode_scratch below).
static __device__ __align__(256) unsigned char scratch[MI_DECODE_SCRATCH_BYTES];

namespace miattn {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_addr[kMaxDevices] = {};

// The current device's scratch address, looked up once per device with that device
// current (no allocation: the array is part of the loaded code object).
int decode_scratch(void** addr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(MI_ERR_LAUNCH, "mi_paged_decode_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) {
    return fail(MI_ERR_UNSUPPORTED, "mi_paged_decode_noalloc: device %d is past the %d this library tracks", dev,
                kMaxDevices);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_addr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      return fail(MI_ERR_LAUNCH, "mi_paged_decode_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                  hipGetErrorString(e));
    }
    g_scratch_addr[dev] = p;
  }
  *addr = g_scratch_addr[dev];
  return MI_OK;
}

}  // namespace
}  // namespace miattn

extern "C" int mi_paged_decode(const void* q, const void* k_cache, const void* v_cache,
                               const int32_t* block_table, const int32_t* seqlen, void* out, int B,
                               int H, int H_kv, int D, int block_size, int max_blocks,
                               const int64_t* strides, float scale, int dtype, void* workspace,
                               size_t workspace_bytes, void* stream) {
  return miattn::paged_decode_entry(q, k_cache, v_cache, block_table, seqlen, out, B, H, H_kv, D, block_size,
                                    max_blocks, strides, scale, dtype, workspace, workspace_bytes, stream);
}

extern "C" int mi_paged_decode_fused(const void* qkv, int64_t row_stride, int qkv_parts, const void* q_norm_w,
                                     const void* k_norm_w, const void* cos_tab, const void* sin_tab, int64_t n_pos,
                                     int rotary_dim, const int64_t* pos, const void* slot_ids, int slot_bits,
                                     void* k_cache, void* v_cache, const int32_t* block_table, const int32_t* seqlen,
                                     void* out, int B, int H, int H_kv, int D, int block_size, int max_blocks,
                                     int64_t n_slots, const int64_t* strides, float scale, float eps, int norm_mode,
                                     int dtype, void* workspace, size_t workspace_bytes, int32_t* error_word,
                                     void* stream) {
  using namespace miattn;
  if (dtype != MI_BF16 && dtype != MI_F16) {
    return fail(MI_ERR_UNSUPPORTED, "mi_paged_decode_fused: fp16/bf16 only, got dtype %d", dtype);
  }
  if (D != 128 || rotary_dim != D || norm_mode != 0) {
    return fail(MI_ERR_UNSUPPORTED,
                "mi_paged_decode_fused: head_dim 128 with whole-head RoPE and the Qwen3 norm only (got head_dim "
                "%d, rotary_dim %d, norm_mode %d); use mi_qk_norm_rope_write and mi_paged_decode",
                D, rotary_dim, norm_mode);
  }
  if (B < 0 || H < 1 || H_kv < 1 || H % H_kv != 0) {
    return fail(MI_ERR_INVALID, "mi_paged_decode_fused: n_head (%d) must be a multiple of n_kv_head (%d)", H, H_kv);
  }
  if (slot_bits != 32 && slot_bits != 64) {
    return fail(MI_ERR_INVALID, "mi_paged_decode_fused: slot_bits must be 32 or 64, got %d", slot_bits);
  }
  if (n_pos < 1 || n_slots < 1 || qkv_parts < 0) {
    return fail(MI_ERR_INVALID, "mi_paged_decode_fused: n_pos %lld, n_slots %lld, qkv_parts %d",
                (long long)n_pos, (long long)n_slots, qkv_parts);
  }
  if (row_stride < int64_t(H + 2 * H_kv) * D) {
    return fail(MI_ERR_INVALID, "mi_paged_decode_fused: row stride %lld < %d packed q/k/v elements",
                (long long)row_stride, (H + 2 * H_kv) * D);
  }
  if (qkv == nullptr || q_norm_w == nullptr || k_norm_w == nullptr || cos_tab == nullptr || sin_tab == nullptr ||
      pos == nullptr || slot_ids == nullptr) {
    return fail(MI_ERR_INVALID, "mi_paged_decode_fused: a required pointer is NULL");
  }
  const int64_t in_es = qkv_parts > 0 ? 4 : 2;
  auto al = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  if (!al(qkv) || (row_stride * in_es) % 16 != 0 || !al(q_norm_w) || !al(k_norm_w) || !al(cos_tab) || !al(sin_tab)) {
    return fail(MI_ERR_UNSUPPORTED,
                "mi_paged_decode_fused: qkv rows, norm weights and RoPE tables must be 16-byte aligned");
  }
  FusedArgs fa{};
  fa.qkv = qkv;
  fa.row_stride = row_stride;
  fa.plane = int64_t(B) * row_stride;
  fa.parts = qkv_parts;
  fa.slot_bits = slot_bits;
  fa.q_w = q_norm_w;
  fa.k_w = k_norm_w;
  fa.cos_tab = cos_tab;
  fa.sin_tab = sin_tab;
  fa.n_pos = n_pos;
  fa.n_slots = n_slots;
  fa.pos = pos;
  fa.slots = slot_ids;
  fa.eps = eps;
  fa.err = error_word;
  return paged_decode_entry(nullptr, k_cache, v_cache, block_table, seqlen, out, B, H, H_kv, D, block_size,
                            max_blocks, strides, scale, dtype, workspace, workspace_bytes, stream, &fa);
}

// The split-K partials need no clearing between calls: a row's (first slot, split count)
// record is written by its first split before the merge launch reads it, every partial the
// merge reads was written by this call's first launch, and rows of length 0 read nothing.
extern "C" int mi_paged_decode_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                       const int32_t* block_table, const int32_t* seqlen, void* out, int B,
                                       int H, int H_kv, int D, int block_size, int max_blocks,
                                       const int64_t* strides, float scale, int dtype, void* stream) {
  using namespace miattn;
  if (esize_of(dtype) != 0 && shape_ok(B, H, H_kv, D, block_size, max_blocks, dtype)) {
    const size_t need = mi_paged_decode_workspace_size(B, H, H_kv, D, block_size, max_blocks, dtype);
    if (need > MI_DECODE_SCRATCH_BYTES) {
      return fail(MI_ERR_WORKSPACE,
                  "mi_paged_decode_noalloc: this shape needs %zu bytes of split-K scratch, more than the %zu "
                  "bytes the library holds per GPU; use mi_paged_decode with a workspace",
                  need, size_t(MI_DECODE_SCRATCH_BYTES));
    }
  }
  void* ws = nullptr;
  const int rc = decode_scratch(&ws);
  if (rc != MI_OK) return rc;
  return paged_decode_entry(q, k_cache, v_cache, block_table, seqlen, out, B, H, H_kv, D, block_size, max_blocks,
                            strides, scale, dtype, ws, MI_DECODE_SCRATCH_BYTES, stream);
}
