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
#include <climits>
#include <type_traits>

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

// Element (row, col) of a projection output: T, or the rounded sum of fp32 partials
// (sum_parts<kU>).
template <typename T, int kU>
struct ProjIn {
  const void* p;
  int parts;      // kU = -1: p is T [rows][cols]; else p is fp32 [parts][rows][cols]
  int64_t plane;  // rows * cols
  // Raw loads of element idx (issued first) ...
  struct Raw {
    PartSum<(kU < 0 ? 1 : kU)> ps;
  };
  __device__ __forceinline__ void load(int64_t idx, Raw& r) const {
    if constexpr (kU < 0) {
      r.ps.v[0] = to_f32(static_cast<const T*>(p)[idx]);
    } else {
      r.ps.load(static_cast<const float*>(p) + idx, parts, plane);
    }
  }
  // ... and its value in T (the rounded sum of the partials).
  __device__ __forceinline__ float value(const Raw& r) const {
    if constexpr (kU < 0) {
      return r.ps.v[0];
    } else {
      return rnd<T>(r.ps.sum(parts));
    }
  }
};

constexpr int kNormThreads = 256;
constexpr int kNormMaxPerThread = 16;  // rows of up to 4096 elements stay in registers

// RMSNorm of one row held by a workgroup (PER elements per thread, PER * 256 >= cols; s and
// the norm weights wv already loaded): h_row = s / sqrt(mean(s^2) + eps) * w, rounded step by
// step, and x_row = s when x_row is not null.
template <typename T, int PER>
__device__ __forceinline__ void norm_row(const float (&s)[PER], const float (&wv)[PER], int cols, float eps,
                                         T* x_row, T* __restrict__ h_row) {
  __shared__ float part[kNormThreads / 64];
  const int tid = threadIdx.x;
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    if (tid + j * kNormThreads < cols) ss += rnd<T>(s[j] * s[j]);
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
  for (int j = 0; j < PER; ++j) {
    const int i = tid + j * kNormThreads;
    if (i < cols) {
      if (x_row != nullptr) x_row[i] = from_f32<T>(s[j]);
      h_row[i] = from_f32<T>(rnd<T>(rnd<T>(s[j] / rms) * wv[j]));
    }
  }
}

// One workgroup per row: s = x + delta (or x), x_out = s, h_out = rmsnorm(s) * w. Every load
// of the row (x, w and all delta partials) is issued before the first use, with indices past
// cols clamped to the row's last element (loaded, never used).
template <typename T, bool kAdd, int kU, int PER>
__global__ __launch_bounds__(kNormThreads) void add_rms_norm_kernel(
    const T* x, ProjIn<T, kU> delta, const T* __restrict__ w, T* x_out,  // x_out may alias x
    T* __restrict__ h_out, int cols, float eps) {
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const T* xr = x + row * cols;
  float s[PER], wv[PER];
  typename ProjIn<T, kU>::Raw dr[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int ic = min(tid + j * kNormThreads, cols - 1);
    s[j] = to_f32(xr[ic]);
    wv[j] = to_f32(w[ic]);
    if constexpr (kAdd) delta.load(row * cols + ic, dr[j]);
  }
  if constexpr (kAdd) {
#pragma unroll
    for (int j = 0; j < PER; ++j) s[j] = rnd<T>(s[j] + delta.value(dr[j]));
  }
  T* x_row = (kAdd && x_out != nullptr) ? x_out + row * cols : nullptr;
  norm_row<T, PER>(s, wv, cols, eps, x_row, h_out + row * cols);
}

// Start of a captured decode step, one workgroup per row: seqlen = pos + 1, the row's write
// slot table[pos / bs] * bs + pos % bs (reference model/paged.py:499-501), x = embed[token]
// (the embedding lookup) and h = rmsnorm(x) * w (layer 0's input norm).
// A row with a negative position is an idle seat of a serving batch: it is made inert for
// the step (below) without a report. A row is refused when its token is outside the
// vocabulary, its position is past the table's width, or the table entry for its position
// is negative (a row's table padded with -1 past its own blocks, so a row that runs past
// its own blocks is caught even inside a wider batch table); it is reported (row + 1)
// through the error word and made inert. Inert: slot -1 (the epilogue writes nothing for
// the row), seqlen 0 (its attention reads nothing and is zero) and x = h = 0; no other
// row's state is touched.
template <typename T, int PER>
__global__ __launch_bounds__(kNormThreads) void step_begin_kernel(
    const int64_t* __restrict__ tokens, const int64_t* __restrict__ pos, const int32_t* __restrict__ table,
    int64_t bt_stride, int block_size, int max_blocks, const T* __restrict__ embed, int64_t vocab,
    const T* __restrict__ w, int cols, float eps, int32_t* __restrict__ seqlen, int64_t* __restrict__ slots,
    T* __restrict__ x, T* __restrict__ h, int32_t* __restrict__ err) {
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t t = tokens[row];
  const int64_t p = pos[row];
  const bool idle = p < 0;
  const bool in_table = !idle && p / block_size < max_blocks;
  const int32_t page = in_table ? table[row * bt_stride + p / block_size] : -1;
  if (idle || t < 0 || t >= vocab || page < 0) {  // uniform over the workgroup
    if (tid == 0) {
      if (!idle && err != nullptr) atomicCAS(err, 0, row + 1);
      seqlen[row] = 0;
      slots[row] = -1;
    }
    for (int i = tid; i < cols; i += kNormThreads) {
      x[int64_t(row) * cols + i] = from_f32<T>(0.0f);
      h[int64_t(row) * cols + i] = from_f32<T>(0.0f);
    }
    return;
  }
  if (tid == 0) {
    seqlen[row] = int32_t(p + 1);
    slots[row] = int64_t(page) * block_size + p % block_size;
  }
  const T* er = embed + t * cols;
  float s[PER], wv[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int ic = min(tid + j * kNormThreads, cols - 1);
    s[j] = to_f32(er[ic]);
    wv[j] = to_f32(w[ic]);
  }
  norm_row<T, PER>(s, wv, cols, eps, x + int64_t(row) * cols, h + int64_t(row) * cols);
}

// out[r, i] = silu(gu[r, i]) * gu[r, inter + i]
template <typename T, int kU>
__global__ __launch_bounds__(256) void silu_mul_kernel(ProjIn<T, kU> gu, T* __restrict__ out, int inter) {
  const int64_t row = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= inter) return;
  typename ProjIn<T, kU>::Raw gr, ur;
  gu.load(row * 2 * inter + i, gr);
  gu.load(row * 2 * inter + inter + i, ur);
  const float g = gu.value(gr);
  const float u = gu.value(ur);
  const float sg = rnd<T>(g / (1.0f + expf(-g)));
  out[row * inter + i] = from_f32<T>(rnd<T>(sg * u));
}

template <typename T, int PER>
int launch_norm_per(const void* x, const void* delta, int delta_parts, const void* w, void* x_out, void* h_out,
                    int rows, int cols, float eps, hipStream_t s) {
  const dim3 grid(rows), block(kNormThreads);
  const int64_t plane = int64_t(rows) * cols;
  if (delta == nullptr) {
    hipLaunchKernelGGL((add_rms_norm_kernel<T, false, -1, PER>), grid, block, 0, s, static_cast<const T*>(x),
                       ProjIn<T, -1>{nullptr, 0, plane}, static_cast<const T*>(w), static_cast<T*>(nullptr),
                       static_cast<T*>(h_out), cols, eps);
  } else {
    auto go = [&](auto unroll) {
      constexpr int U = decltype(unroll)::value;
      hipLaunchKernelGGL((add_rms_norm_kernel<T, true, U, PER>), grid, block, 0, s, static_cast<const T*>(x),
                         ProjIn<T, U>{delta, delta_parts, plane}, static_cast<const T*>(w), static_cast<T*>(x_out),
                         static_cast<T*>(h_out), cols, eps);
    };
    switch (parts_unroll(delta_parts)) {
      case -1: go(std::integral_constant<int, -1>{}); break;
      case 2: go(std::integral_constant<int, 2>{}); break;
      case 8: go(std::integral_constant<int, 8>{}); break;
      default: go(std::integral_constant<int, 0>{}); break;
    }
  }
  return launch_status("mi_add_rms_norm");
}

template <typename T>
int launch_norm(const void* x, const void* delta, int delta_parts, const void* w, void* x_out, void* h_out,
                int rows, int cols, float eps, hipStream_t s) {
  if (cols <= 4 * kNormThreads) return launch_norm_per<T, 4>(x, delta, delta_parts, w, x_out, h_out, rows, cols, eps, s);
  if (cols <= 8 * kNormThreads) return launch_norm_per<T, 8>(x, delta, delta_parts, w, x_out, h_out, rows, cols, eps, s);
  return launch_norm_per<T, 16>(x, delta, delta_parts, w, x_out, h_out, rows, cols, eps, s);
}

template <typename T>
int launch_silu(const void* gu, int gu_parts, void* out, int rows, int inter, hipStream_t s) {
  const dim3 grid((inter + 255) / 256, rows);
  const int64_t plane = int64_t(rows) * 2 * inter;
  auto go = [&](auto unroll) {
    constexpr int U = decltype(unroll)::value;
    hipLaunchKernelGGL((silu_mul_kernel<T, U>), grid, dim3(256), 0, s, ProjIn<T, U>{gu, gu_parts, plane},
                       static_cast<T*>(out), inter);
  };
  switch (parts_unroll(gu_parts)) {
    case -1: go(std::integral_constant<int, -1>{}); break;
    case 2: go(std::integral_constant<int, 2>{}); break;
    case 8: go(std::integral_constant<int, 8>{}); break;
    default: go(std::integral_constant<int, 0>{}); break;
  }
  return launch_status("mi_silu_mul");
}

// ---------------------------------------------------------------- greedy pick
// torch.argmax over a row: the index of the largest value, the first one on ties, NaN above
// every number (the first NaN wins).
struct Best {
  float v;
  int i;
};
__device__ __forceinline__ bool better(float v, int i, const Best& b) {
  const bool nv = v != v, nb = b.v != b.v;
  if (nv != nb) return nv;
  if (!nv && v != b.v) return v > b.v;
  return i < b.i;
}

constexpr int kArgmaxThreads = 1024;

// Optional end of a greedy decode step (all null: plain argmax): tokens[r] = pick,
// history[r, steps[r]] = pick while steps[r] < max_steps, steps[r] += 1, pos[r] += 1.
struct Advance {
  int64_t* tokens;
  int64_t* pos;
  int64_t* history;
  int64_t hist_stride;
  int64_t* steps;
  int max_steps;
};

// Workgroup-wide reduction of the threads' (value, index) candidates, then thread 0 writes
// the pick (out, and the step's advance when requested).
__device__ __forceinline__ void finish_pick(Best b, Best* part, int row, int64_t* out, const Advance& adv) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(b.v, off, 64);
    const int oi = __shfl_xor(b.i, off, 64);
    if (better(ov, oi, b)) b = Best{ov, oi};
  }
  if ((tid & 63) == 0) part[tid >> 6] = b;
  __syncthreads();
  if (tid == 0) {
    Best r = part[0];
    for (int k = 1; k < int(blockDim.x) / 64; ++k) {
      if (better(part[k].v, part[k].i, r)) r = part[k];
    }
    if (out != nullptr) out[row] = r.i;
    if (adv.tokens != nullptr && adv.pos[row] >= 0) {  // an idle seat (pos < 0) keeps its state
      adv.tokens[row] = r.i;
      const int64_t st = adv.steps[row];
      if (st >= 0 && st < adv.max_steps) adv.history[row * adv.hist_stride + st] = r.i;
      adv.steps[row] = st + 1;
      adv.pos[row] += 1;
    }
  }
}

// One workgroup per row; each thread walks 8-element (16-byte) pieces of the row 4 at a time
// (all 4 loads in flight), then the workgroup reduces (value, index) pairs.
template <typename T>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_rows_kernel(const T* __restrict__ x, int64_t ld, int cols,
                                                                     int64_t* __restrict__ out, bool vec, Advance adv) {
  __shared__ Best part[kArgmaxThreads / 64];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const T* xr = x + int64_t(row) * ld;
  Best b{-INFINITY, INT_MAX};
  if (vec) {
    constexpr int E = 16 / int(sizeof(T));
    constexpr int kUnroll = 4;
    const int pieces = cols / E;
    for (int p0 = tid; p0 < pieces; p0 += kArgmaxThreads * kUnroll) {
      uint4 raw[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int pc = min(p0 + u * kArgmaxThreads, pieces - 1);
        raw[u] = load16(xr + int64_t(pc) * E);
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int pc = p0 + u * kArgmaxThreads;
        if (pc < pieces) {
          const T* e = reinterpret_cast<const T*>(&raw[u]);
#pragma unroll
          for (int k = 0; k < E; ++k) {
            const float v = to_f32(e[k]);
            if (better(v, pc * E + k, b)) b = Best{v, pc * E + k};
          }
        }
      }
    }
    for (int i = pieces * E + tid; i < cols; i += kArgmaxThreads) {  // tail past the last piece
      const float v = to_f32(xr[i]);
      if (better(v, i, b)) b = Best{v, i};
    }
  } else {
    for (int i = tid; i < cols; i += kArgmaxThreads) {
      const float v = to_f32(xr[i]);
      if (better(v, i, b)) b = Best{v, i};
    }
  }
  finish_pick(b, part, row, out, adv);
}

// Greedy pick from per-tile results (the lm_head launch's best (value, column) of each
// 32-column tile for each row, row-major: tiles[row * n_tiles + t]): the same rule applied to
// the tiles' winners gives the row's first maximum.
__global__ __launch_bounds__(kArgmaxThreads) void pick_tiles_kernel(const Best* __restrict__ tiles, int n_tiles,
                                                                    int rows, int64_t* __restrict__ out, Advance adv) {
  __shared__ Best part[kArgmaxThreads / 64];
  const int row = blockIdx.x;
  Best b{-INFINITY, INT_MAX};
  for (int t = threadIdx.x; t < n_tiles; t += kArgmaxThreads) {
    const Best c = tiles[int64_t(row) * n_tiles + t];
    if (better(c.v, c.i, b)) b = c;
  }
  finish_pick(b, part, row, out, adv);
}

template <typename T>
int launch_argmax(const void* x, int64_t ld, int rows, int cols, int64_t* out, const Advance& adv, hipStream_t s) {
  const bool vec = reinterpret_cast<uintptr_t>(x) % 16 == 0 && (ld * int64_t(sizeof(T))) % 16 == 0;
  hipLaunchKernelGGL((argmax_rows_kernel<T>), dim3(rows), dim3(kArgmaxThreads), 0, s, static_cast<const T*>(x), ld,
                     cols, out, vec, adv);
  return launch_status(adv.tokens != nullptr ? "mi_greedy_advance" : "mi_argmax_rows");
}

template <typename T>
int launch_begin(const int64_t* tokens, const int64_t* pos, const int32_t* table, int64_t bt_stride, int block_size,
                 int max_blocks, const void* embed, int64_t vocab, const void* w, int cols, float eps, int32_t* seqlen,
                 int64_t* slots, void* x, void* h, int B, int32_t* err, hipStream_t s) {
  auto go = [&](auto per) {
    constexpr int PER = decltype(per)::value;
    hipLaunchKernelGGL((step_begin_kernel<T, PER>), dim3(B), dim3(kNormThreads), 0, s, tokens, pos, table, bt_stride,
                       block_size, max_blocks, static_cast<const T*>(embed), vocab, static_cast<const T*>(w), cols,
                       eps, seqlen, slots, static_cast<T*>(x), static_cast<T*>(h), err);
  };
  if (cols <= 4 * kNormThreads) go(std::integral_constant<int, 4>{});
  else if (cols <= 8 * kNormThreads) go(std::integral_constant<int, 8>{});
  else go(std::integral_constant<int, 16>{});
  return launch_status("mi_decode_step_begin");
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

extern "C" int mi_argmax_rows(const void* x, int64_t ld, int rows, int cols, int64_t* out, int dtype, void* stream) {
  using namespace miattn;
  if (rows < 0 || cols < 1 || ld < cols) {
    return fail(MI_ERR_INVALID, "mi_argmax_rows: bad shape rows=%d cols=%d ld=%lld", rows, cols, (long long)ld);
  }
  if (x == nullptr || out == nullptr) return fail(MI_ERR_INVALID, "mi_argmax_rows: NULL pointer");
  if (rows == 0) return MI_OK;
  if (rows > 2147483647) return fail(MI_ERR_UNSUPPORTED, "mi_argmax_rows: too many rows");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case MI_BF16: return launch_argmax<bf16_t>(x, ld, rows, cols, out, Advance{}, s);
    case MI_F16: return launch_argmax<f16_t>(x, ld, rows, cols, out, Advance{}, s);
    case MI_F32: return launch_argmax<float>(x, ld, rows, cols, out, Advance{}, s);
    default: return fail(MI_ERR_INVALID, "mi_argmax_rows: unknown dtype %d", dtype);
  }
}

extern "C" int mi_greedy_advance(const void* logits, int64_t ld, int rows, int cols, int dtype, int64_t* tokens,
                                 int64_t* pos, int64_t* history, int64_t hist_stride, int64_t* steps, int max_steps,
                                 void* stream) {
  using namespace miattn;
  if (rows < 0 || cols < 1 || ld < cols || max_steps < 0 || hist_stride < max_steps) {
    return fail(MI_ERR_INVALID, "mi_greedy_advance: bad shape rows=%d cols=%d ld=%lld max_steps=%d", rows, cols,
                (long long)ld, max_steps);
  }
  if (logits == nullptr || tokens == nullptr || pos == nullptr || steps == nullptr ||
      (max_steps > 0 && history == nullptr)) {
    return fail(MI_ERR_INVALID, "mi_greedy_advance: NULL pointer");
  }
  if (rows == 0) return MI_OK;
  const Advance adv{tokens, pos, history, hist_stride, steps, max_steps};
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case MI_BF16: return launch_argmax<bf16_t>(logits, ld, rows, cols, nullptr, adv, s);
    case MI_F16: return launch_argmax<f16_t>(logits, ld, rows, cols, nullptr, adv, s);
    case MI_F32: return launch_argmax<float>(logits, ld, rows, cols, nullptr, adv, s);
    default: return fail(MI_ERR_INVALID, "mi_greedy_advance: unknown dtype %d", dtype);
  }
}

extern "C" int mi_decode_step_begin(const int64_t* tokens, const int64_t* pos, const int32_t* block_table,
                                    int64_t bt_stride, int block_size, int max_blocks, const void* embed,
                                    int64_t vocab, const void* norm_w, int cols, float eps, int32_t* seqlen,
                                    int64_t* slots, void* x, void* h, int B, int dtype, int32_t* error_word,
                                    void* stream) {
  using namespace miattn;
  if (B < 0 || cols < 1 || block_size < 1 || max_blocks < 1 || vocab < 1 || bt_stride < max_blocks) {
    return fail(MI_ERR_INVALID, "mi_decode_step_begin: bad shape B=%d cols=%d block_size=%d max_blocks=%d", B, cols,
                block_size, max_blocks);
  }
  if (cols > kNormThreads * kNormMaxPerThread) {
    return fail(MI_ERR_UNSUPPORTED, "mi_decode_step_begin: rows of at most %d elements, got %d",
                kNormThreads * kNormMaxPerThread, cols);
  }
  if (tokens == nullptr || pos == nullptr || block_table == nullptr || embed == nullptr || norm_w == nullptr ||
      seqlen == nullptr || slots == nullptr || x == nullptr || h == nullptr) {
    return fail(MI_ERR_INVALID, "mi_decode_step_begin: NULL pointer");
  }
  if (B == 0) return MI_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case MI_BF16: return launch_begin<bf16_t>(tokens, pos, block_table, bt_stride, block_size, max_blocks, embed,
                                              vocab, norm_w, cols, eps, seqlen, slots, x, h, B, error_word, s);
    case MI_F16: return launch_begin<f16_t>(tokens, pos, block_table, bt_stride, block_size, max_blocks, embed,
                                            vocab, norm_w, cols, eps, seqlen, slots, x, h, B, error_word, s);
    case MI_F32: return launch_begin<float>(tokens, pos, block_table, bt_stride, block_size, max_blocks, embed,
                                            vocab, norm_w, cols, eps, seqlen, slots, x, h, B, error_word, s);
    default: return fail(MI_ERR_INVALID, "mi_decode_step_begin: unknown dtype %d", dtype);
  }
}

extern "C" int mi_greedy_advance_tiles(const void* tile_best, int n_tiles, int rows, int64_t* tokens, int64_t* pos,
                                       int64_t* history, int64_t hist_stride, int64_t* steps, int max_steps,
                                       void* stream) {
  using namespace miattn;
  if (rows < 0 || n_tiles < 1 || max_steps < 0 || hist_stride < max_steps) {
    return fail(MI_ERR_INVALID, "mi_greedy_advance_tiles: bad shape rows=%d n_tiles=%d max_steps=%d", rows, n_tiles,
                max_steps);
  }
  if (tile_best == nullptr || tokens == nullptr || pos == nullptr || steps == nullptr ||
      (max_steps > 0 && history == nullptr)) {
    return fail(MI_ERR_INVALID, "mi_greedy_advance_tiles: NULL pointer");
  }
  if (rows == 0) return MI_OK;
  const Advance adv{tokens, pos, history, hist_stride, steps, max_steps};
  hipLaunchKernelGGL(pick_tiles_kernel, dim3(rows), dim3(kArgmaxThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const Best*>(tile_best), n_tiles, rows, nullptr, adv);
  return launch_status("mi_greedy_advance_tiles");
}
