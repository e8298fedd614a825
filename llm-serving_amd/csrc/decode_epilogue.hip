// Decode-step attention epilogue of one layer, fused: per-head RMSNorm of q and k, NeoX
// RoPE at each row's position, q out contiguous for the paged decode, k and v scattered into
// the paged pool at each row's write slot.
//
// The reference runs these as separate tensor ops between the projections and the paged
// decode: q_norm / k_norm (RMSNorm, reference model/layers.py:342-350, applied at :193-194),
// apply_rotary_emb (:59-89, applied at :210-211), then PagedKV.write, whose slot scatter is
// mi_kv_slot_write (model/paged.py:503-520). At the decode shape (B = 32 rows, 16 + 8 + 8
// heads of 128) every one of those ops is a few microseconds of launch for kilobytes of
// data; here the whole epilogue is one launch.
//
// Arithmetic follows the reference's tensor ops step by step in the activation dtype: each
// elementwise result is rounded to the dtype as the op it restates would store it (x^2, the
// mean, mean + eps, its square root, x / rms, (x / rms) * w, and each product and sum of the
// rotation), with the mean's sum accumulated in fp32 as the reduction kernel does. The
// result equals the tensor-op chain's except where the fp32 sum's order moves a rounding
// boundary.
//
// With k_out / v_out the roped k and the v of each row are also written packed, (B, H_kv, D)
// contiguous, for a packed prefill's attention (the decode reads them from the pool).
//
// Two q/k norms: norm_mode 0 is the Qwen3 RMSNorm above (x / rms * w, op by op in T);
// norm_mode 1 is Qwen3.5's zero-centred norm (reference model/qwen35.py:67-89): x * (1 /
// sqrt(mean(x^2) + eps)) * (1 + w), all in fp32 and rounded to T once. RoPE rotates the first
// rotary_dim elements of each head (pairs (e, e + rotary_dim/2), NeoX halves of the rotated
// slice, reference model/layers.py:91-117) and passes the rest through; rotary_dim == D is
// the whole-head rotation of Qwen3, 64 of 256 is Qwen3.5's partial RoPE.
//
// Layout: one wave per (row, head) over q, k and v heads of a packed projection row
// [q (H x D) | k (H_kv x D) | v (H_kv x D)] (a longer row stride leaves room for further
// columns, such as Qwen3.5's output gate); lane l holds elements l, l + 64, ... (coalesced
// loads and stores); a rotation partner is in the same lane when rotary_dim/2 is a multiple
// of 64 and in lane l ^ 32 when it is 32. The projection rows are T, or fp32 split-K partial
// sums [parts][B][row_stride] of mi_rows_gemm, summed in split order and rounded once to T
// (the value the projection's own output would hold).
#include <type_traits>

#include "common.h"

namespace miattn {
namespace {

// Which q/k norm the epilogue applies (see the file comment).
enum NormMode { kNormQwen3 = 0, kNormZeroCentred = 1 };

template <typename T, int D, typename IdxT, int kU>
__global__ __launch_bounds__(256) void qk_norm_rope_write_kernel(
    const void* __restrict__ qkv, int64_t row_stride, int parts, int64_t plane, const T* __restrict__ q_w,
    const T* __restrict__ k_w, const T* __restrict__ cos_tab, const T* __restrict__ sin_tab, int64_t n_pos,
    int rotary, const int64_t* __restrict__ pos, const IdxT* __restrict__ slots, T* __restrict__ q_out,
    T* __restrict__ k_pool, T* __restrict__ v_pool, T* __restrict__ k_out, T* __restrict__ v_out, int B, int H,
    int H_kv, int64_t n_slots, float eps, int norm_mode, int32_t* __restrict__ err) {
  constexpr int NE = D / 64;  // elements per lane: lane l holds e = l + 64 j, j < NE
  const int lane = threadIdx.x & 63;
  const int head = blockIdx.y * (blockDim.x / 64) + (threadIdx.x >> 6);  // over q, k, v heads
  const int b = blockIdx.x;
  const int n_heads = H + 2 * H_kv;
  if (head >= n_heads || b >= B) return;  // wave-uniform
  // slot -1 marks a row with nothing to write this step (an idle or refused seat of a decode
  // step): skipped silently. Any other row whose position is outside the RoPE table or whose
  // slot is outside the pool is not written to the pool and is reported (row + 1) through
  // the error word. Either way the row's packed outputs (q_out, and k_out / v_out when given)
  // are zero-filled, so a consumer that reads every row reads defined values.
  const int64_t pb = pos[b];
  const IdxT slot = slots[b];
  const bool idle = slot == IdxT(-1);
  if (idle || pb < 0 || pb >= n_pos || !(slot >= 0 && int64_t(slot) < n_slots)) {
    if (!idle && lane == 0 && head == 0 && err != nullptr) atomicCAS(err, 0, b + 1);
    T* row = nullptr;
    if (head < H) {
      row = q_out + (int64_t(b) * H + head) * D;
    } else if (head < H + H_kv) {
      if (k_out != nullptr) row = k_out + (int64_t(b) * H_kv + (head - H)) * D;
    } else if (v_out != nullptr) {
      row = v_out + (int64_t(b) * H_kv + (head - H - H_kv)) * D;
    }
    if (row != nullptr) {
#pragma unroll
      for (int j = 0; j < NE; ++j) row[lane + 64 * j] = from_f32<T>(0.0f);
    }
    return;
  }
  const int64_t src = int64_t(b) * row_stride + int64_t(head) * D;
  // every load of this wave's inputs first, then the arithmetic (the rounding helper's empty
  // asm is a scheduling barrier)
  constexpr int kP = kU < 0 ? 1 : kU;
  PartSum<kP> raw[NE];
#pragma unroll
  for (int j = 0; j < NE; ++j) {
    const int e = lane + 64 * j;
    if constexpr (kU < 0) {
      raw[j].v[0] = to_f32(static_cast<const T*>(qkv)[src + e]);
    } else {
      raw[j].load(static_cast<const float*>(qkv) + src + e, parts, plane);
    }
  }
  // norm weights and this row's RoPE table entries (read here, used after the reduction);
  // the tables hold rotary/2 angles per position: element e < rotary uses angle e mod half
  const bool is_q = head < H;
  const int half = rotary >> 1;
  const T* w = is_q ? q_w : k_w;
  float wt[NE], cs[NE], sn[NE];
#pragma unroll
  for (int j = 0; j < NE; ++j) {
    const int e = lane + 64 * j;
    const int a = e < half ? e : (e < rotary ? e - half : 0);
    wt[j] = to_f32(w[e]);
    cs[j] = to_f32(cos_tab[pb * half + a]);
    sn[j] = to_f32(sin_tab[pb * half + a]);
  }
  float x[NE];
#pragma unroll
  for (int j = 0; j < NE; ++j) {
    if constexpr (kU < 0) x[j] = raw[j].v[0];
    else x[j] = rt<T>(raw[j].sum(parts));
  }

  if (head >= H + H_kv) {  // v head: copied as is (exact: x holds T values)
    const int vh = head - H - H_kv;
    T* dst = v_pool + (int64_t(slot) * H_kv + vh) * D;
    T* dst2 = v_out != nullptr ? v_out + (int64_t(b) * H_kv + vh) * D : nullptr;
#pragma unroll
    for (int j = 0; j < NE; ++j) {
      dst[lane + 64 * j] = from_f32<T>(x[j]);
      if (dst2 != nullptr) dst2[lane + 64 * j] = from_f32<T>(x[j]);
    }
    return;
  }

  float y[NE];  // normed head, T values
  if (norm_mode == kNormQwen3) {
    // x / sqrt(mean(x^2) + eps) * w, each op rounded to T, the squares summed in fp32
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NE; ++j) ss += rt<T>(x[j] * x[j]);
    ss = group_allreduce<64, SumOp>(ss);
    const float ms = rt<T>(ss * (1.0f / D));
    const float rms = rt<T>(sqrtf(rt<T>(ms + eps)));
#pragma unroll
    for (int j = 0; j < NE; ++j) y[j] = rt<T>(rt<T>(x[j] / rms) * wt[j]);
  } else {
    // zero-centred weight, all in fp32, rounded once: x * (1 / sqrt(mean(x^2) + eps)) * (1 + w)
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NE; ++j) ss += x[j] * x[j];
    ss = group_allreduce<64, SumOp>(ss);
    const float r = 1.0f / sqrtf(ss * (1.0f / D) + eps);
#pragma unroll
    for (int j = 0; j < NE; ++j) y[j] = rt<T>((x[j] * r) * (1.0f + wt[j]));
  }
  // NeoX RoPE over the first `rotary` elements: pairs (e, e + half); the partner is in this
  // lane at j ^ (half / 64) when half >= 64, else in lane ^ 32 (half = 32)
  float o[NE];
#pragma unroll
  for (int j = 0; j < NE; ++j) {
    const float across = swap32(y[j]);
    float partner = across;
    if constexpr (NE > 1) if (half == 64) partner = y[j ^ 1];
    if constexpr (NE > 2) if (half == 128) partner = y[j ^ 2];
    const int e = lane + 64 * j;
    if (e < half) {
      o[j] = rt<T>(rt<T>(y[j] * cs[j]) - rt<T>(partner * sn[j]));
    } else if (e < rotary) {
      o[j] = rt<T>(rt<T>(partner * sn[j]) + rt<T>(y[j] * cs[j]));
    } else {
      o[j] = y[j];
    }
  }

  T* dst;
  T* dst2 = nullptr;  // the packed k copy, when asked for
  if (is_q) {
    dst = q_out + (int64_t(b) * H + head) * D;
  } else {
    dst = k_pool + (int64_t(slot) * H_kv + (head - H)) * D;
    if (k_out != nullptr) dst2 = k_out + (int64_t(b) * H_kv + (head - H)) * D;
  }
#pragma unroll
  for (int j = 0; j < NE; ++j) {
    dst[lane + 64 * j] = from_f32<T>(o[j]);
    if (dst2 != nullptr) dst2[lane + 64 * j] = from_f32<T>(o[j]);
  }
}

// Launch arguments shared by every instantiation.
struct EpilogueArgs {
  const void* qkv; int64_t row_stride; int parts; const void* q_w; const void* k_w; const void* cos_tab;
  const void* sin_tab; int64_t n_pos; int rotary; const int64_t* pos; const void* slots; int slot_bits;
  void* q_out; void* k_pool; void* v_pool; void* k_out; void* v_out; int B; int H; int H_kv; int64_t n_slots;
  float eps; int norm_mode; int32_t* err; hipStream_t s;
};

template <typename T, int D>
int launch_d(const EpilogueArgs& a) {
  constexpr int kWaves = 4;
  const dim3 grid(a.B, (a.H + 2 * a.H_kv + kWaves - 1) / kWaves);
  const int64_t plane = int64_t(a.B) * a.row_stride;
  auto go = [&](auto idx_tag, auto unroll) {
    using IdxT = decltype(idx_tag);
    hipLaunchKernelGGL((qk_norm_rope_write_kernel<T, D, IdxT, decltype(unroll)::value>), grid, dim3(64 * kWaves), 0,
                       a.s, a.qkv, a.row_stride, a.parts, plane, static_cast<const T*>(a.q_w),
                       static_cast<const T*>(a.k_w), static_cast<const T*>(a.cos_tab),
                       static_cast<const T*>(a.sin_tab), a.n_pos, a.rotary, a.pos, static_cast<const IdxT*>(a.slots),
                       static_cast<T*>(a.q_out), static_cast<T*>(a.k_pool), static_cast<T*>(a.v_pool),
                       static_cast<T*>(a.k_out), static_cast<T*>(a.v_out), a.B, a.H, a.H_kv, a.n_slots, a.eps,
                       a.norm_mode, a.err);
  };
  auto by_slots = [&](auto unroll) {
    if (a.slot_bits == 32) go(int32_t{}, unroll); else go(int64_t{}, unroll);
  };
  switch (parts_unroll(a.parts)) {
    case -1: by_slots(std::integral_constant<int, -1>{}); break;
    case 2: by_slots(std::integral_constant<int, 2>{}); break;
    case 8: by_slots(std::integral_constant<int, 8>{}); break;
    default: by_slots(std::integral_constant<int, 0>{}); break;
  }
  return launch_status("mi_qk_norm_rope_write");
}

template <typename T>
int launch_t(int D, const EpilogueArgs& a) {
  switch (D) {
    case 64: return launch_d<T, 64>(a);
    case 128: return launch_d<T, 128>(a);
    case 256: return launch_d<T, 256>(a);
    default:
      return fail(MI_ERR_UNSUPPORTED, "mi_qk_norm_rope_write: head_dim %d is not supported (64, 128, 256)", D);
  }
}

}  // namespace
}  // namespace miattn

extern "C" int mi_qk_norm_rope_write(const void* qkv, int64_t row_stride, int qkv_parts, const void* q_norm_w,
                                     const void* k_norm_w, const void* cos_tab, const void* sin_tab,
                                     int64_t n_pos, int rotary_dim, const int64_t* pos, const void* slot_ids,
                                     int slot_bits, void* q_out, void* k_pool, void* v_pool, void* k_out,
                                     void* v_out, int B, int H, int H_kv, int D, int64_t n_slots, float eps,
                                     int norm_mode, int dtype, int32_t* error_word, void* stream) {
  using namespace miattn;
  if (B < 0 || H < 1 || H_kv < 1 || H % H_kv != 0) {
    return fail(MI_ERR_INVALID, "mi_qk_norm_rope_write: n_head (%d) must be a multiple of n_kv_head (%d)", H, H_kv);
  }
  if (slot_bits != 32 && slot_bits != 64) {
    return fail(MI_ERR_INVALID, "mi_qk_norm_rope_write: slot_bits must be 32 or 64, got %d", slot_bits);
  }
  if (n_pos < 1) return fail(MI_ERR_INVALID, "mi_qk_norm_rope_write: the RoPE table is empty");
  if (qkv_parts < 0) return fail(MI_ERR_INVALID, "mi_qk_norm_rope_write: qkv_parts %d < 0", qkv_parts);
  if (row_stride < int64_t(H + 2 * H_kv) * D) {
    return fail(MI_ERR_INVALID, "mi_qk_norm_rope_write: row stride %lld < %d packed q/k/v elements",
                (long long)row_stride, (H + 2 * H_kv) * D);
  }
  // the rotation partner of element e < rotary/2 is e + rotary/2: in the same lane when
  // rotary/2 is a multiple of 64, in lane ^ 32 when it is 32
  if (!(rotary_dim == 64 || rotary_dim == 128 || rotary_dim == 256) || rotary_dim > D) {
    return fail(MI_ERR_UNSUPPORTED, "mi_qk_norm_rope_write: rotary_dim %d must be 64, 128 or 256 and <= head_dim %d",
                rotary_dim, D);
  }
  if (norm_mode != 0 && norm_mode != 1) {
    return fail(MI_ERR_INVALID, "mi_qk_norm_rope_write: norm_mode %d is not 0 or 1", norm_mode);
  }
  if (qkv == nullptr || q_norm_w == nullptr || k_norm_w == nullptr || cos_tab == nullptr || sin_tab == nullptr ||
      pos == nullptr || slot_ids == nullptr || q_out == nullptr || k_pool == nullptr || v_pool == nullptr) {
    return fail(MI_ERR_INVALID, "mi_qk_norm_rope_write: NULL pointer argument");
  }
  if (B == 0) return MI_OK;
  const EpilogueArgs a{qkv, row_stride, qkv_parts, q_norm_w, k_norm_w, cos_tab, sin_tab, n_pos, rotary_dim, pos,
                       slot_ids, slot_bits, q_out, k_pool, v_pool, k_out, v_out, B, H, H_kv, n_slots, eps, norm_mode,
                       error_word, static_cast<hipStream_t>(stream)};
  switch (dtype) {
    case MI_BF16: return launch_t<bf16_t>(D, a);
    case MI_F16: return launch_t<f16_t>(D, a);
    case MI_F32: return launch_t<float>(D, a);
    default:
      return fail(MI_ERR_INVALID, "mi_qk_norm_rope_write: unknown dtype %d", dtype);
  }
}
