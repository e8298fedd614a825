// out = A W^T for the few activation rows of a decode step (M <= 32): the q/k/v, o, gate/up,
// down and lm_head projections of the reference's decode step (reference
// model/layers.py:176-222 and :325-335, model/minillm.py lm_head), which run as nn.Linear
// at batch = number of running sequences.
//
// At M = 32 a projection is a weight stream: each weight element is used for 32 products,
// so the kernel is HBM bound on W (N x K x 2 bytes) and the point is to have the whole
// weight matrix in flight at once across the chip. Layout:
//   * grid (ceil(N / 32), S): a workgroup owns 32 output columns and 1/S of K; its 4 waves
//     split that K range again, each wave KW = K / (4 S) contiguous k (NIT x 64);
//   * every load a wave makes is issued before its first MFMA. W and A are loaded in whole
//     128-byte lines, 8 lanes per line, and turned into the MFMA operand layout through the
//     wave's own LDS region, one 64-k step at a time. Loading the operand layout directly (each
//     lane 16 bytes of its own row, 32 lines per instruction) measured 1.3-1.5x slower at
//     the Qwen3-0.6B shapes, and 1.6x with the nontemporal hint (each line then fetched
//     from L2 once per 16-byte piece);
//   * v_mfma_f32_32x32x16 with A rows as the M operand and W rows as the N operand; inside
//     a 64-k step, MFMA s takes k = hf * 32 + s * 8 .. + 7 from lane half hf on both operands,
//     a permutation of k that leaves the dot products unchanged;
//   * the 4 waves' 32 x 32 accumulators are summed through LDS in a fixed order, then
//     written as T (S = 1) or as fp32 partials [S][M][N] that the consumer sums in split
//     order and rounds once (the same single rounding nn.Linear's output gets).
// Rows past M and columns past N read a clamped valid row and are never stored.
#include <climits>

#include "common.h"

namespace miattn {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));

constexpr int kTile = 32;        // output columns per workgroup, and the most rows
constexpr int kStepK = 64;       // k per step per wave
constexpr int kGemmWaves = 4;

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

// One wave's 32 rows x NIT 64-k steps of a row-major matrix, loaded in whole lines (load q
// of a step: rows q*8 .. q*8+7, 8 lanes per 128-byte line); rows past row_hi repeat it.
template <typename T, int NIT, bool kStream>
__device__ __forceinline__ void stage_rows(const T* __restrict__ base, int64_t ld, int row_hi, int64_t k0,
                                           uint4 (&frag)[NIT][4]) {
  const int lane = threadIdx.x & 63;
  const int rr = lane >> 3, cc = lane & 7;
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const T* p = base + int64_t(min(q * 8 + rr, row_hi)) * ld + k0 + it * kStepK + cc * 8;
      frag[it][q] = kStream ? load16_nt(p) : load16(p);
    }
  }
}
// Through the wave's LDS region (one 64-k step, 32 rows x 128 B) into the MFMA operand
// layout (lane: row lane & 31, k-half lane >> 5), one step at a time through the same
// region: every load is already in flight, so the region only has to hold the step being
// converted, and the small region lets registers rather than LDS set the occupancy (the
// lm_head launch: 77.5 -> 63.5 us against staging all steps at once). 16-byte slots are
// XOR-swizzled by row: the writes and the operand reads are both conflict-free.
template <int NIT>
__device__ __forceinline__ void to_operands(uint4* __restrict__ lds, uint4 (&frag)[NIT][4]) {
  const int lane = threadIdx.x & 63;
  const int rr = lane >> 3, cc = lane & 7;
  const int j = lane & 31, hf = lane >> 5;
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = q * 8 + rr;
      lds[row * 8 + (cc ^ (row & 7))] = frag[it][q];
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int s = 0; s < 4; ++s) frag[it][s] = lds[j * 8 + ((hf * 4 + s) ^ (j & 7))];
    __builtin_amdgcn_wave_barrier();
  }
}

// Round an fp32 result to T behind an empty asm, so the compiler cannot fold the op and the
// rounding into a native fp16 op of different rounding.
template <typename T>
__device__ __forceinline__ float round_t(float x) {
  asm volatile("" : "+v"(x));
  return to_f32(from_f32<T>(x));
}

// kGLU: W holds gate and up rows interleaved by 16 (column tile t = gate rows 16t..16t+15,
// then up rows 16t..16t+15) and the launch is unsplit; the epilogue writes
// out[i, 16t + c] = silu(g) * u with g, u the tile's columns c and 16 + c, rounded as the
// reference's F.silu(gate(x)) * up(x) is: g and u to T, silu(g) = g / (1 + exp(-g)) in fp32 to
// T, the product to T.
// A tile's best column of each row under torch.argmax's rule on the rounded outputs: the
// largest value, the lowest column on ties, NaN above every number.
struct TileBest {
  float v;
  int i;
};

// best != null (unsplit launches only): each workgroup also writes, per row, its 32 columns'
// best (value as rounded to T, column) to best[row * n_tiles + blockIdx.x], and writes the
// outputs themselves only when out != null.
template <typename T, int NIT, bool kGLU>
__global__ __launch_bounds__(256) void rows_gemm_kernel(const T* __restrict__ a, int64_t lda,
                                                        const T* __restrict__ w, int64_t ldw,
                                                        T* __restrict__ out, int64_t ldo,
                                                        float* __restrict__ part, int M, int N, int K,
                                                        TileBest* __restrict__ best) {
  constexpr int kRegion = 2 * 256;  // 16-byte slots per wave: one step of W, one of A
  __shared__ uint4 lds[kGemmWaves * kRegion];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n0 = blockIdx.x * kTile;
  const int split = blockIdx.y;
  constexpr int kw = NIT * kStepK;
  const int64_t kb = int64_t(split) * (kGemmWaves * kw) + wave * kw;  // this wave's k range
  uint4* wl = lds + wave * kRegion;

  uint4 wr[NIT][4], ar[NIT][4];
  stage_rows<T, NIT, true>(w + int64_t(n0) * ldw, ldw, N - 1 - n0, kb, wr);
  stage_rows<T, NIT, false>(a, lda, M - 1, kb, ar);
  __builtin_amdgcn_sched_barrier(0);  // every load above is issued before the first use
  to_operands<NIT>(wl, wr);
  to_operands<NIT>(wl + 256, ar);

  floatx16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
#pragma unroll
    for (int s = 0; s < 4; ++s) acc = mfma32<T>(ar[it][s], wr[it][s], acc);
  }

  // The 4 waves' accumulators, summed in wave order through each wave's own region (its
  // operands are in registers by now): red[wave][r][lane].
  float* red = reinterpret_cast<float*>(lds);
  constexpr int kRedStride = kRegion * 4;  // floats per wave region (>= 16 x 64)
#pragma unroll
  for (int r = 0; r < 16; ++r) red[wave * kRedStride + r * 64 + lane] = acc[r];
  __syncthreads();
  if constexpr (kGLU) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int h = q * 256 + tid;                         // 512 (row, gate column) pairs
      const int r = h >> 5, ln = (h & 15) | ((h & 16) << 1);  // accumulator (r, lane), lane & 31 < 16
      const int e = r * 64 + ln;
      auto total = [&](int x) {
        return ((red[x] + red[kRedStride + x]) + red[2 * kRedStride + x]) + red[3 * kRedStride + x];
      };
      const float g = round_t<T>(total(e));
      const float u = round_t<T>(total(e + 16));
      const float sg = round_t<T>(g / (1.0f + expf(-g)));
      const int i = 8 * (r >> 2) + 4 * (ln >> 5) + (r & 3);
      const int n = blockIdx.x * 16 + (ln & 15);
      if (i < M) out[int64_t(i) * ldo + n] = from_f32<T>(round_t<T>(sg * u));
    }
    return;
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int e = q * 256 + tid;
    const float v = ((red[e] + red[kRedStride + e]) + red[2 * kRedStride + e]) + red[3 * kRedStride + e];
    const int r = e >> 6, ln = e & 63;
    const int i = 8 * (r >> 2) + 4 * (ln >> 5) + (r & 3);  // accumulator row (activation row)
    const int n = n0 + (ln & 31);                            // accumulator column
    if (best != nullptr) {  // wave-uniform: the 32 lanes of each half hold one row's 32 columns
      // first maximum of the half: the max over its non-NaN columns (DPP), then the lowest
      // lane holding it; a NaN column, if any, wins instead (the lowest NaN lane)
      const bool valid = n < N;
      const float vr = to_f32(from_f32<T>(v));
      const bool is_nan = valid && vr != vr;
      const float vv = valid && !is_nan ? vr : -INFINITY;
      const float mx = group_allreduce<32, MaxOp>(vv);
      const int sh = (ln >> 5) * 32;
      const uint32_t nan_lanes = uint32_t(__ballot(is_nan) >> sh);
      const uint32_t max_lanes = uint32_t(__ballot(valid && !is_nan && vv == mx) >> sh);
      if ((ln & 31) == 0 && i < M) {
        const int jn = __builtin_ffs(int(nan_lanes)) - 1, jm = __builtin_ffs(int(max_lanes)) - 1;
        best[int64_t(i) * gridDim.x + blockIdx.x] =
            nan_lanes != 0 ? TileBest{__builtin_nanf(""), n0 + jn} : TileBest{mx, n0 + jm};
      }
      if (out == nullptr) continue;
    }
    if (i < M && n < N) {
      if (part == nullptr) {
        out[int64_t(i) * ldo + n] = from_f32<T>(v);
      } else {
        part[(int64_t(split) * M + i) * N + n] = v;
      }
    }
  }
}

template <typename T, bool kGLU>
int launch_rows(const void* a, int64_t lda, const void* w, int64_t ldw, void* out, int64_t ldo, float* part,
                int M, int N, int K, int S, int nit, hipStream_t s, TileBest* best = nullptr) {
  const dim3 grid((N + kTile - 1) / kTile, S), block(256);
  const T* at = static_cast<const T*>(a);
  const T* wt = static_cast<const T*>(w);
  T* ot = static_cast<T*>(out);
  switch (nit) {
    case 1: hipLaunchKernelGGL((rows_gemm_kernel<T, 1, kGLU>), grid, block, 0, s, at, lda, wt, ldw, ot, ldo, part, M, N, K, best); break;
    case 2: hipLaunchKernelGGL((rows_gemm_kernel<T, 2, kGLU>), grid, block, 0, s, at, lda, wt, ldw, ot, ldo, part, M, N, K, best); break;
    case 3: hipLaunchKernelGGL((rows_gemm_kernel<T, 3, kGLU>), grid, block, 0, s, at, lda, wt, ldw, ot, ldo, part, M, N, K, best); break;
    default: hipLaunchKernelGGL((rows_gemm_kernel<T, 4, kGLU>), grid, block, 0, s, at, lda, wt, ldw, ot, ldo, part, M, N, K, best); break;
  }
  return launch_status(kGLU ? "mi_rows_gemm_glu" : "mi_rows_gemm");
}

}  // namespace
}  // namespace miattn

// Split count for an M x N x K product: the smallest divisor S of K / 256 with at most 2
// 64-k steps per wave (4 for a launch of 1024+ column tiles) that gives 192+ workgroups.
// Measured at M = 32 (bf16, MI355X, graph replay): N x K = 4096 x 1024 -> S 2, 4.3 us;
// 1024 x 2048 -> 8, 3.4 us; 6144 x 1024 -> 2, 5.5 us; 1024 x 3072 -> 6, 4.0 us;
// 151936 x 1024 -> 1, 77 us (hipBLASLt: 8.1, 8.2, 11.3, 7.5, 77 us).
extern "C" int mi_rows_gemm_split(int M, int N, int K) {
  using namespace miattn;
  if (M < 1 || N < 1 || K < 1 || K % (kGemmWaves * kStepK) != 0) return 0;
  const int64_t tiles = (N + kTile - 1) / kTile;
  const int units = K / (kGemmWaves * kStepK);
  int fallback = 0;
  for (int S = 1; S <= units; ++S) {
    if (units % S != 0 || units / S > 4) continue;
    if (fallback == 0) fallback = S;
    const int nit = units / S;
    if ((nit <= 2 || tiles >= 1024) && tiles * S >= 192) return S;
  }
  return fallback != 0 ? fallback : units;
}

extern "C" int mi_rows_gemm(const void* a, int64_t lda, const void* w, int64_t ldw, void* out, int64_t ldo,
                            float* partials, int M, int N, int K, int n_split, int dtype, void* stream) {
  using namespace miattn;
  if (M < 1 || M > kTile || N < 1 || K < 1) {
    return fail(MI_ERR_INVALID, "mi_rows_gemm: bad shape M=%d N=%d K=%d (1 <= M <= %d)", M, N, K, kTile);
  }
  if (n_split < 1 || K % (n_split * kGemmWaves * kStepK) != 0) {
    return fail(MI_ERR_UNSUPPORTED, "mi_rows_gemm: K=%d is not a multiple of n_split (%d) x %d", K, n_split,
                kGemmWaves * kStepK);
  }
  const int nit = K / (n_split * kGemmWaves * kStepK);
  if (nit > 4) {
    return fail(MI_ERR_UNSUPPORTED, "mi_rows_gemm: K / n_split = %d is more than %d", K / n_split,
                4 * kGemmWaves * kStepK);
  }
  if (n_split > 65535) return fail(MI_ERR_UNSUPPORTED, "mi_rows_gemm: n_split %d > 65535", n_split);
  if (a == nullptr || w == nullptr || (n_split == 1 ? out == nullptr : partials == nullptr)) {
    return fail(MI_ERR_INVALID, "mi_rows_gemm: NULL pointer argument");
  }
  if (lda < K || ldw < K || (n_split == 1 && ldo < N)) {
    return fail(MI_ERR_INVALID, "mi_rows_gemm: row strides (%lld, %lld, %lld) shorter than the rows",
                (long long)lda, (long long)ldw, (long long)ldo);
  }
  if ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(w)) % 16 != 0 || lda % 8 != 0 || ldw % 8 != 0) {
    return fail(MI_ERR_UNSUPPORTED, "mi_rows_gemm: A and W need 16-byte aligned rows");
  }
  float* part = n_split == 1 ? nullptr : partials;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case MI_BF16: return launch_rows<bf16_t, false>(a, lda, w, ldw, out, ldo, part, M, N, K, n_split, nit, s);
    case MI_F16: return launch_rows<f16_t, false>(a, lda, w, ldw, out, ldo, part, M, N, K, n_split, nit, s);
    default: return fail(MI_ERR_UNSUPPORTED, "mi_rows_gemm: dtype %d (bf16 and fp16 only)", dtype);
  }
}

extern "C" int mi_rows_gemm_glu(const void* a, int64_t lda, const void* w_glu, int64_t ldw, void* out, int64_t ldo,
                                int M, int inter, int K, int dtype, void* stream) {
  using namespace miattn;
  if (M < 1 || M > kTile || inter < 1 || inter % 16 != 0 || K < 1) {
    return fail(MI_ERR_INVALID, "mi_rows_gemm_glu: bad shape M=%d inter=%d K=%d (1 <= M <= %d, inter %% 16 == 0)", M,
                inter, K, kTile);
  }
  if (K % (kGemmWaves * kStepK) != 0 || K / (kGemmWaves * kStepK) > 4) {
    return fail(MI_ERR_UNSUPPORTED, "mi_rows_gemm_glu: K=%d must be a multiple of %d and at most %d", K,
                kGemmWaves * kStepK, 4 * kGemmWaves * kStepK);
  }
  if (a == nullptr || w_glu == nullptr || out == nullptr) return fail(MI_ERR_INVALID, "mi_rows_gemm_glu: NULL pointer");
  if (lda < K || ldw < K || ldo < inter) {
    return fail(MI_ERR_INVALID, "mi_rows_gemm_glu: row strides (%lld, %lld, %lld) shorter than the rows",
                (long long)lda, (long long)ldw, (long long)ldo);
  }
  if ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(w_glu)) % 16 != 0 || lda % 8 != 0 ||
      ldw % 8 != 0) {
    return fail(MI_ERR_UNSUPPORTED, "mi_rows_gemm_glu: A and W need 16-byte aligned rows");
  }
  const int nit = K / (kGemmWaves * kStepK);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case MI_BF16: return launch_rows<bf16_t, true>(a, lda, w_glu, ldw, out, ldo, nullptr, M, 2 * inter, K, 1, nit, s);
    case MI_F16: return launch_rows<f16_t, true>(a, lda, w_glu, ldw, out, ldo, nullptr, M, 2 * inter, K, 1, nit, s);
    default: return fail(MI_ERR_UNSUPPORTED, "mi_rows_gemm_glu: dtype %d (bf16 and fp16 only)", dtype);
  }
}

extern "C" int mi_rows_gemm_argmax(const void* a, int64_t lda, const void* w, int64_t ldw, void* out, int64_t ldo,
                                   void* tile_best, int M, int N, int K, int dtype, void* stream) {
  using namespace miattn;
  if (M < 1 || M > kTile || N < 1 || K < 1) {
    return fail(MI_ERR_INVALID, "mi_rows_gemm_argmax: bad shape M=%d N=%d K=%d (1 <= M <= %d)", M, N, K, kTile);
  }
  if (K % (kGemmWaves * kStepK) != 0 || K / (kGemmWaves * kStepK) > 4) {
    return fail(MI_ERR_UNSUPPORTED, "mi_rows_gemm_argmax: K=%d must be a multiple of %d and at most %d", K,
                kGemmWaves * kStepK, 4 * kGemmWaves * kStepK);
  }
  if (a == nullptr || w == nullptr || tile_best == nullptr) {
    return fail(MI_ERR_INVALID, "mi_rows_gemm_argmax: NULL pointer argument");
  }
  if (lda < K || ldw < K || (out != nullptr && ldo < N)) {
    return fail(MI_ERR_INVALID, "mi_rows_gemm_argmax: row strides (%lld, %lld, %lld) shorter than the rows",
                (long long)lda, (long long)ldw, (long long)ldo);
  }
  if ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(w)) % 16 != 0 || lda % 8 != 0 || ldw % 8 != 0) {
    return fail(MI_ERR_UNSUPPORTED, "mi_rows_gemm_argmax: A and W need 16-byte aligned rows");
  }
  const int nit = K / (kGemmWaves * kStepK);
  TileBest* best = static_cast<TileBest*>(tile_best);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case MI_BF16: return launch_rows<bf16_t, false>(a, lda, w, ldw, out, ldo, nullptr, M, N, K, 1, nit, s, best);
    case MI_F16: return launch_rows<f16_t, false>(a, lda, w, ldw, out, ldo, nullptr, M, N, K, 1, nit, s, best);
    default: return fail(MI_ERR_UNSUPPORTED, "mi_rows_gemm_argmax: dtype %d (bf16 and fp16 only)", dtype);
  }
}
