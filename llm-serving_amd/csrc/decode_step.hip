// Small per-layer ops of the decode step around the attention path, each fused into one
// launch: the residual add with the following RMSNorm, and SiLU(gate) * up.
//
// The reference's block is x = x + attn(norm1(x)); x = x + mlp(norm2(x)) (reference
// model/layers.py:365-367) with RMSNorm x / sqrt(mean(x^2) + eps) * w (:342-350) and the MLP
// down(silu(gate(x)) * up(x)) (:325-335), each a chain of tensor ops. At the decode shape
// (32 rows of 1024) every op is a few microseconds of launch for 64 KiB of data, so the
// step's time went to launches; here an add + norm is one launch and SiLU * up another.
//
// Arithmetic restates the tensor ops one by one in the activation dtype, as the attention
// epilogue does (csrc/decode_epilogue.hip): x + delta rounded, x^2 rounded, the mean of the
// rounded squares (fp32 sum times 1/N, rounded), + eps rounded, its square root rounded, x / rms
// rounded, times w rounded; silu(g) = g / (1 + exp(-g)) in fp32 rounded, times u rounded.
// Results equal the tensor-op chain's except where the fp32 sum's order moves a rounding
// boundary of the mean.
//
// The projection feeding each op (o_proj / down_proj into the add, gate_up into SiLU * up)
// may arrive as fp32 split-K partial sums [parts][rows][cols] of mi_rows_gemm: the op sums
// them in split order and rounds once to the activation dtype, the value the projection's
// own output would hold, before the chain above.
#include "common.h"

namespace miattn {
namespace {

// Round an fp32 result to T behind an empty asm, so the compiler cannot fold the op and
// the rounding into a native fp16 op of different rounding.
template <typename T>
__device__ __forceinline__ float rnd(float x) {
  asm volatile("" : "+v"(x));
  return to_f32(from_f32<T>(x));
}

// Element (row, col) of a projection output: T, or the rounded sum of fp32 partials.
template <typename T>
struct ProjIn {
  const void* p;
  int parts;      // 0: p is T [rows][cols]; n >= 1: p is fp32 [n][rows][cols]
  int64_t plane;  // rows * cols
  __device__ __forceinline__ float at(int64_t idx) const {
    if (parts == 0) return to_f32(static_cast<const T*>(p)[idx]);
    const float* f = static_cast<const float*>(p);
    float acc = f[idx];
    for (int s = 1; s < parts; ++s) acc += f[s * plane + idx];
    return rnd<T>(acc);
  }
};

constexpr int kNormThreads = 256;
constexpr int kNormMaxPerThread = 16;  // rows of up to 4096 elements stay in registers

// One workgroup per row: s = x + delta (or x), x_out = s, h_out = rmsnorm(s) * w.
template <typename T, bool kAdd>
__global__ __launch_bounds__(kNormThreads) void add_rms_norm_kernel(
    const T* x, ProjIn<T> delta, const T* __restrict__ w, T* x_out,  // x_out may alias x
    T* __restrict__ h_out, int cols, float eps) {
  __shared__ float part[kNormThreads / 64];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const T* xr = x + row * cols;
  float s[kNormMaxPerThread];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < kNormMaxPerThread; ++j) {
    const int i = tid + j * kNormThreads;
    s[j] = 0.0f;
    if (i < cols) {
      float v = to_f32(xr[i]);
      if constexpr (kAdd) v = rnd<T>(v + delta.at(row * cols + i));
      s[j] = v;
      ss += rnd<T>(v * v);
    }
  }
  ss = group_allreduce<64, SumOp>(ss);
  if ((tid & 63) == 0) part[tid >> 6] = ss;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int k = 0; k < kNormThreads / 64; ++k) total += part[k];
  const float ms = rnd<T>(total * (1.0f / float(cols)));  // the mean kernel scales by 1/N
  const float rms = rnd<T>(sqrtf(rnd<T>(ms + eps)));
#pragma unroll
  for (int j = 0; j < kNormMaxPerThread; ++j) {
    const int i = tid + j * kNormThreads;
    if (i < cols) {
      if constexpr (kAdd) {
        if (x_out != nullptr) x_out[row * cols + i] = from_f32<T>(s[j]);
      }
      h_out[row * cols + i] = from_f32<T>(rnd<T>(rnd<T>(s[j] / rms) * to_f32(w[i])));
    }
  }
}

// out[r, i] = silu(gu[r, i]) * gu[r, inter + i]
template <typename T>
__global__ __launch_bounds__(256) void silu_mul_kernel(ProjIn<T> gu, T* __restrict__ out, int inter) {
  const int64_t row = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= inter) return;
  const float g = gu.at(row * 2 * inter + i);
  const float u = gu.at(row * 2 * inter + inter + i);
  const float sg = rnd<T>(g / (1.0f + expf(-g)));
  out[row * inter + i] = from_f32<T>(rnd<T>(sg * u));
}

template <typename T>
int launch_norm(const void* x, const void* delta, int delta_parts, const void* w, void* x_out, void* h_out,
                int rows, int cols, float eps, hipStream_t s) {
  const dim3 grid(rows), block(kNormThreads);
  const ProjIn<T> d{delta, delta_parts, int64_t(rows) * cols};
  if (delta != nullptr) {
    hipLaunchKernelGGL((add_rms_norm_kernel<T, true>), grid, block, 0, s, static_cast<const T*>(x), d,
                       static_cast<const T*>(w), static_cast<T*>(x_out), static_cast<T*>(h_out), cols, eps);
  } else {
    hipLaunchKernelGGL((add_rms_norm_kernel<T, false>), grid, block, 0, s, static_cast<const T*>(x), d,
                       static_cast<const T*>(w), static_cast<T*>(nullptr), static_cast<T*>(h_out), cols, eps);
  }
  return launch_status("mi_add_rms_norm");
}

template <typename T>
int launch_silu(const void* gu, int gu_parts, void* out, int rows, int inter, hipStream_t s) {
  const dim3 grid((inter + 255) / 256, rows);
  const ProjIn<T> g{gu, gu_parts, int64_t(rows) * 2 * inter};
  hipLaunchKernelGGL((silu_mul_kernel<T>), grid, dim3(256), 0, s, g, static_cast<T*>(out), inter);
  return launch_status("mi_silu_mul");
}

}  // namespace
}  // namespace miattn

extern "C" int mi_add_rms_norm(const void* x, const void* delta, int delta_parts, const void* weight, void* x_out,
                               void* h_out, int rows, int cols, float eps, int dtype, void* stream) {
  using namespace miattn;
  if (rows < 0 || cols < 1) return fail(MI_ERR_INVALID, "mi_add_rms_norm: bad shape (%d, %d)", rows, cols);
  if (delta_parts < 0) return fail(MI_ERR_INVALID, "mi_add_rms_norm: delta_parts %d < 0", delta_parts);
  if (cols > kNormThreads * kNormMaxPerThread) {
    return fail(MI_ERR_UNSUPPORTED, "mi_add_rms_norm: rows of at most %d elements, got %d",
                kNormThreads * kNormMaxPerThread, cols);
  }
  if (x == nullptr || weight == nullptr || h_out == nullptr) return fail(MI_ERR_INVALID, "mi_add_rms_norm: NULL pointer");
  if (rows == 0) return MI_OK;
  if (rows > 2147483647 / cols) return fail(MI_ERR_UNSUPPORTED, "mi_add_rms_norm: too many elements");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case MI_BF16: return launch_norm<bf16_t>(x, delta, delta_parts, weight, x_out, h_out, rows, cols, eps, s);
    case MI_F16: return launch_norm<f16_t>(x, delta, delta_parts, weight, x_out, h_out, rows, cols, eps, s);
    case MI_F32: return launch_norm<float>(x, delta, delta_parts, weight, x_out, h_out, rows, cols, eps, s);
    default: return fail(MI_ERR_INVALID, "mi_add_rms_norm: unknown dtype %d", dtype);
  }
}

extern "C" int mi_silu_mul(const void* gate_up, int gate_up_parts, void* out, int rows, int inter, int dtype,
                           void* stream) {
  using namespace miattn;
  if (rows < 0 || inter < 1) return fail(MI_ERR_INVALID, "mi_silu_mul: bad shape (%d, %d)", rows, inter);
  if (gate_up_parts < 0) return fail(MI_ERR_INVALID, "mi_silu_mul: gate_up_parts %d < 0", gate_up_parts);
  if (gate_up == nullptr || out == nullptr) return fail(MI_ERR_INVALID, "mi_silu_mul: NULL pointer");
  if (rows == 0) return MI_OK;
  if (rows > 65535) return fail(MI_ERR_UNSUPPORTED, "mi_silu_mul: at most 65535 rows, got %d", rows);
  if (int64_t(rows) * 2 * inter > 2147483647LL) return fail(MI_ERR_UNSUPPORTED, "mi_silu_mul: too many elements");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case MI_BF16: return launch_silu<bf16_t>(gate_up, gate_up_parts, out, rows, inter, s);
    case MI_F16: return launch_silu<f16_t>(gate_up, gate_up_parts, out, rows, inter, s);
    case MI_F32: return launch_silu<float>(gate_up, gate_up_parts, out, rows, inter, s);
    default: return fail(MI_ERR_INVALID, "mi_silu_mul: unknown dtype %d", dtype);
  }
}
