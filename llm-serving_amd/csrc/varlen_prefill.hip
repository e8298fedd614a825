// Packed varlen causal prefill attention on gfx950 bf16/fp16 MFMA.
//
// Replaces FlashVarlen.prefill_varlen's FA2 call (reference model/attention/varlen.py:
// 317-357): causal attention inside each cu_seqlens segment of a packed (total, H, D)
// token axis, GQA head h -> KV head h / (H / H_kv), softmax scale applied to the fp32
// scores. FlashAttention-2 style: one pass over K/V tiles with an fp32 online softmax.
//
// MI355X shape of the computation:
//   * a workgroup (4 waves) owns one query tile of one packed segment for HPW query heads
//     that share a KV head; every wave owns 32 query rows of one head, so the K/V tile
//     staged in LDS is shared by all 4 waves (and by both GQA heads at Qwen3's 16/8);
//   * scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16 (A = K from
//     LDS, B = Q held in VGPRs for the whole loop). In the 32x32 accumulator layout each
//     lane then owns one query column, so the row max needs one cross-lane exchange
//     (lane ^ 32) and the row sum none until the end;
//   * O^T = V^T P^T with the same MFMA: P^T comes straight from the score registers
//     (packed to bf16), and V is stored transposed in LDS while it is staged, so the A
//     operand is two 8-byte LDS reads per lane; the key order inside a 16-key MFMA step
//     is permuted identically on both operands to match the score accumulator layout;
//   * causal tiles above the diagonal are never visited; the diagonal tile is masked;
//   * the grid is (head group, schedule entry): head groups are the fastest-varying
//     index, so with 8 head groups every tile of one KV head lands on the same XCD and
//     its K/V stay in that XCD's L2; schedule entries are ordered heaviest-first.
#include <algorithm>
#include <type_traits>
#include <vector>

#include "common.h"

namespace miattn {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));

constexpr int kThreads = 256;

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

template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return uint32_t(from_f32<T>(lo).bits) | (uint32_t(from_f32<T>(hi).bits) << 16);
}

// Rows of the query tile owned by one workgroup.
template <int HPW>
struct TileShape {
  static constexpr int WPH = 4 / HPW;  // waves per head
  static constexpr int RW = 32 * WPH;  // query rows per workgroup tile
};

template <int D>
struct KeyTile {
  static constexpr int BN = D <= 128 ? 64 : 32;  // keys per K/V tile
};

template <typename T, int D, int HPW>
__global__ __launch_bounds__(kThreads, 2) void varlen_prefill_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    T* __restrict__ out, const int32_t* __restrict__ cu, const int32_t* __restrict__ sched,
    int H, int H_kv, int G, float scale_log2, int causal) {
  constexpr int WPH = TileShape<HPW>::WPH;
  constexpr int RW = TileShape<HPW>::RW;
  constexpr int BN = KeyTile<D>::BN;
  constexpr int KST = D + 8;   // LDS row stride of the K tile (elements)
  constexpr int VST = BN + 8;  // LDS row stride of the transposed V tile
  constexpr int KS = D / 16;   // MFMA k-steps over D for S^T
  constexpr int MB = BN / 32;  // 32-key blocks per tile
  constexpr int TS = BN / 16;  // 16-key MFMA k-steps for O^T
  constexpr int DB = D / 32;   // 32-wide blocks of D for O^T
  __shared__ uint16_t Ks[BN * KST];
  __shared__ uint16_t Vt[D * VST];

  const int hg = blockIdx.x;
  const int entry = sched[blockIdx.y];
  const int seq = entry >> 16;
  const int tile = entry & 0xffff;
  const int seq0 = cu[seq];
  const int L = cu[seq + 1] - seq0;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = lane >> 5;     // which half of the wave (k-group of the MFMA operands)
  const int col = lane & 31;   // query column owned by this lane
  const int h = hg * HPW + wave / WPH;
  const int kvh = (hg * HPW) / G;
  const int qi = tile * RW + (wave % WPH) * 32 + col;  // local query index

  const int64_t q_row = int64_t(H) * D;
  const int64_t kv_row = int64_t(H_kv) * D;

  // Q^T as the B operand: lane holds Q[qi][ks*16 + 8g .. +8] for every k-step.
  uint4 qB[KS];
  {
    const int qc = qi < L ? qi : L - 1;
    const T* qp = q + (seq0 + qc) * q_row + h * D + g * 8;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qB[ks] = load16(qp + ks * 16);
  }

  floatx16 o[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i) o[i] = zero16();
  float m_i = -INFINITY;
  float l_i = 0.0f;

  const int tile_end = min(L, tile * RW + RW);
  const int n_kt = causal ? (tile_end + BN - 1) / BN : (L + BN - 1) / BN;
  const T* kseg = k + int64_t(seq0) * kv_row + kvh * D;
  const T* vseg = v + int64_t(seq0) * kv_row + kvh * D;

  for (int kt = 0; kt < n_kt; ++kt) {
    const int key0 = kt * BN;
    __syncthreads();
    // Stage K row-major: consecutive threads read consecutive 16-byte chunks of a row.
    for (int idx = threadIdx.x; idx < BN * D / 8; idx += kThreads) {
      const int key = idx / (D / 8);
      const int cch = idx - key * (D / 8);
      const int tok = key0 + key;
      const uint4 val = tok < L ? load16(kseg + tok * kv_row + cch * 8) : make_uint4(0, 0, 0, 0);
      *reinterpret_cast<uint4*>(&Ks[key * KST + cch * 8]) = val;
    }
    // Stage V transposed (Vt[d][key]): consecutive threads take consecutive keys so the
    // 2-byte LDS stores of one wave land on consecutive addresses.
    for (int idx = threadIdx.x; idx < BN * D / 8; idx += kThreads) {
      const int key = idx % BN;
      const int cch = idx / BN;
      const int tok = key0 + key;
      const uint4 val = tok < L ? load16(vseg + tok * kv_row + cch * 8) : make_uint4(0, 0, 0, 0);
      const uint32_t w[4] = {val.x, val.y, val.z, val.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        Vt[(cch * 8 + e) * VST + key] = uint16_t((w[e >> 1] >> ((e & 1) * 16)) & 0xffffu);
      }
    }
    __syncthreads();

    // S^T[key][query] for the MB 32-key blocks of the tile.
    floatx16 sacc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      sacc[mb] = zero16();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const uint4 a = *reinterpret_cast<const uint4*>(&Ks[(mb * 32 + col) * KST + ks * 16 + g * 8]);
        sacc[mb] = mfma32<T>(a, qB[ks], sacc[mb]);
      }
    }

    // Scale, mask, online softmax for this lane's query column.
    float mloc = -INFINITY;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int key = key0 + mb * 32 + (j >> 2) * 8 + g * 4 + (j & 3);
        const bool masked = key >= L || (causal && key > qi);
        const float s = masked ? -INFINITY : sacc[mb][j] * scale_log2;
        sacc[mb][j] = s;
        mloc = fmaxf(mloc, s);
      }
    }
    const float m_tile = fmaxf(mloc, swap32(mloc));
    const float m_new = fmaxf(m_i, m_tile);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = fast_exp2(m_i - m_use);
    m_i = m_new;
    float lsum = 0.0f;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float p = fast_exp2(sacc[mb][j] - m_use);
        sacc[mb][j] = p;
        lsum += p;
      }
    }
    l_i = l_i * alpha + lsum;
#pragma unroll
    for (int i = 0; i < DB; ++i) o[i] *= alpha;

    // P^T as the B operand of O^T += V^T P^T: k-step t covers keys 16t..16t+15 and the
    // lane's 8 values are sacc[t/2][(t%2)*8 .. +8] (keys 4g+0..3 and 8+4g+0..3).
    uint4 pB[TS];
#pragma unroll
    for (int t = 0; t < TS; ++t) {
      const int mb = t >> 1, jb = (t & 1) * 8;
      pB[t] = make_uint4(pack2<T>(sacc[mb][jb + 0], sacc[mb][jb + 1]),
                         pack2<T>(sacc[mb][jb + 2], sacc[mb][jb + 3]),
                         pack2<T>(sacc[mb][jb + 4], sacc[mb][jb + 5]),
                         pack2<T>(sacc[mb][jb + 6], sacc[mb][jb + 7]));
    }
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const uint16_t* vrow = &Vt[(db * 32 + col) * VST + g * 4];
#pragma unroll
      for (int t = 0; t < TS; ++t) {
        const uint2 lo = *reinterpret_cast<const uint2*>(vrow + t * 16);
        const uint2 hi = *reinterpret_cast<const uint2*>(vrow + t * 16 + 8);
        o[db] = mfma32<T>(make_uint4(lo.x, lo.y, hi.x, hi.y), pB[t], o[db]);
      }
    }
  }

  // Normalise and store: lane owns query qi and, per 32-wide D block, d values
  // (j/4)*8 + 4g + (j%4) -> four runs of 4 consecutive elements.
  const float l_tot = l_i + swap32(l_i);
  const float inv = 1.0f / fmaxf(l_tot, 1e-30f);
  if (qi < L) {
    T* op = out + (seq0 + qi) * q_row + h * D;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int jg = 0; jg < 4; ++jg) {
        const int d = db * 32 + jg * 8 + g * 4;
        const uint2 val = make_uint2(pack2<T>(o[db][jg * 4 + 0] * inv, o[db][jg * 4 + 1] * inv),
                                     pack2<T>(o[db][jg * 4 + 2] * inv, o[db][jg * 4 + 3] * inv));
        *reinterpret_cast<uint2*>(op + d) = val;
      }
    }
  }
}

int hpw_for(int G) { return (G % 4 == 0) ? 4 : (G % 2 == 0) ? 2 : 1; }

int rows_per_tile(int G) { return 32 * (4 / hpw_for(G)); }

int keys_per_tile(int D) { return D <= 128 ? 64 : 32; }

template <typename T, int D, int HPW>
int launch3(const void* q, const void* k, const void* v, void* out, const int32_t* cu,
            const int32_t* sched, int n_tiles, int H, int H_kv, float scale_log2, int causal,
            hipStream_t s) {
  dim3 grid(H / HPW, n_tiles);
  hipLaunchKernelGGL((varlen_prefill_kernel<T, D, HPW>), grid, dim3(kThreads), 0, s,
                     static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
                     static_cast<T*>(out), cu, sched, H, H_kv, H / H_kv, scale_log2, causal);
  return launch_status("mi_varlen_prefill");
}

template <typename T, int D>
int launch2(int hpw, const void* q, const void* k, const void* v, void* out, const int32_t* cu,
            const int32_t* sched, int n_tiles, int H, int H_kv, float sl2, int causal,
            hipStream_t s) {
  switch (hpw) {
    case 1: return launch3<T, D, 1>(q, k, v, out, cu, sched, n_tiles, H, H_kv, sl2, causal, s);
    case 2: return launch3<T, D, 2>(q, k, v, out, cu, sched, n_tiles, H, H_kv, sl2, causal, s);
    case 4: return launch3<T, D, 4>(q, k, v, out, cu, sched, n_tiles, H, H_kv, sl2, causal, s);
  }
  return fail(MI_ERR_UNSUPPORTED, "mi_varlen_prefill: bad heads-per-workgroup %d", hpw);
}

template <typename T>
int launch1(int D, int hpw, const void* q, const void* k, const void* v, void* out,
            const int32_t* cu, const int32_t* sched, int n_tiles, int H, int H_kv, float sl2,
            int causal, hipStream_t s) {
  switch (D) {
    case 64: return launch2<T, 64>(hpw, q, k, v, out, cu, sched, n_tiles, H, H_kv, sl2, causal, s);
    case 128: return launch2<T, 128>(hpw, q, k, v, out, cu, sched, n_tiles, H, H_kv, sl2, causal, s);
    case 256: return launch2<T, 256>(hpw, q, k, v, out, cu, sched, n_tiles, H, H_kv, sl2, causal, s);
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
  const int RW = rows_per_tile(H / H_kv);
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
  const int hpw = hpw_for(H / H_kv);
  const float sl2 = float(double(scale) * 1.4426950408889634);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == MI_BF16) {
    return launch1<bf16_t>(D, hpw, q, k, v, out, cu_seqlens, tile_schedule, n_tiles, H, H_kv, sl2,
                           causal, s);
  }
  return launch1<f16_t>(D, hpw, q, k, v, out, cu_seqlens, tile_schedule, n_tiles, H, H_kv, sl2,
                        causal, s);
}
