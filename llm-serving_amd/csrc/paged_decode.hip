// Block-table paged-decode GQA attention for gfx950.
//
// Replaces paged_decode / _paged_decode_kernel (reference model/triton_decode.py:250-328,
// :545-643). Same math: one query token per row, fp32 online softmax in the log2 domain
// with scale*log2(e), tail of the last page masked by `token < seqlen`, page walk clamped
// to max_blocks, out = acc / max(l, 1) so an empty row is exact zeros.
//
// Different shape, chosen for MI355X:
//   * one workgroup per (row, KV head, head chunk, split): the GB query heads that share a
//     KV head are served by one workgroup, so each K/V byte is read from HBM once (the
//     reference launches one program per query head and relies on the cache, :33-36);
//   * split-K: a row's tokens are cut into `chunk`-token splits, one workgroup each, so
//     B * H_kv = 256 units become thousands of workgroups and ragged rows balance over
//     256 CUs; a log-sum-exp merge kernel folds the per-split (m, l, acc) partials;
//   * lane layout: a KV row of one head (D elements) is spread over LPR = D*esize/16
//     lanes holding 16 bytes each, so one wave-wide 16-byte load fetches 64/LPR whole
//     token rows (4 rows of 256 B at D=128 bf16) straight into registers; the q.k dot is
//     reduced across the LPR lanes with DPP butterflies, and each lane accumulates
//     p * v for its own 16-byte slice of D;
//   * each row of lanes keeps its own online-softmax state over the tokens it owns; the
//     4 * RPW row states of a workgroup are merged through LDS at the end of the split.
// HBM-bound: per (token, KV head) the kernel reads 2 * D * esize bytes of K+V.
#include "common.h"

namespace miattn {
namespace {

struct DecodeArgs {
  int B, H, H_kv, G, n_hchunks, bs_log2, max_blocks, chunk, n_splits;
  int64_t qs0, qs1, ks0, ks1, ks2, vs0, vs1, vs2, os0, os1, bts0;
  float scale_log2;
};

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
// Tokens per lane-row per batch: 2 * unroll 16-byte loads in flight per lane. Fewer when
// one workgroup serves many query heads, whose scores and accumulators take the VGPRs.
constexpr int unroll_for(int GB) { return GB <= 2 ? 8 : 16 / GB; }

template <typename T, int D, int GB>
struct Layout {
  static constexpr int esize = sizeof(T) == 4 ? 4 : 2;
  static constexpr int EPL = 16 / esize;       // elements per lane
  static constexpr int LPR = D / EPL;          // lanes per KV row
  static constexpr int RPW = 64 / LPR;         // KV rows per wave-wide load
  static constexpr int NR = kWaves * RPW;      // row states per workgroup
  static constexpr int U = unroll_for(GB);     // tokens per row per batch
  static constexpr int BATCH = NR * U;         // tokens per workgroup batch
  static_assert(LPR >= 1 && LPR <= 64 && (64 % LPR) == 0, "unsupported D/dtype");
};

template <typename T, int D, int GB>
__global__ __launch_bounds__(kThreads) void decode_split_kernel(
    const T* __restrict__ q, const T* __restrict__ kc, const T* __restrict__ vc,
    const int32_t* __restrict__ block_table, const int32_t* __restrict__ seqlen,
    T* __restrict__ out, float* __restrict__ ws_acc, float* __restrict__ ws_ml, DecodeArgs a) {
  using L = Layout<T, D, GB>;
  constexpr int EPL = L::EPL, LPR = L::LPR, RPW = L::RPW, NR = L::NR;
  constexpr int kUnroll = L::U;
  extern __shared__ float smem[];  // [NR][GB] m, [NR][GB] l, [NR][GB][D] acc

  const int split = blockIdx.x;
  const int kvh = blockIdx.y / a.n_hchunks;
  const int h0 = kvh * a.G + (blockIdx.y - kvh * a.n_hchunks) * GB;
  const int b = blockIdx.z;

  const int capacity = a.max_blocks << a.bs_log2;
  int len = seqlen[b];
  len = len < capacity ? len : capacity;  // page-walk clamp (reference :593)
  const int t_begin = split * a.chunk;
  if (t_begin >= len) {
    if (split == 0) {  // empty row: exact zeros, like acc / max(0, 1)
      for (int i = threadIdx.x; i < GB * D; i += kThreads) {
        const int g = i / D, d = i - g * D;
        out[b * a.os0 + (h0 + g) * a.os1 + d] = from_f32<T>(0.0f);
      }
    }
    return;
  }
  const int t_end = min(len, t_begin + a.chunk);
  const int n_split_b = (len + a.chunk - 1) / a.chunk;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane / LPR;           // row within the wave
  const int c = lane - r * LPR;       // 16-byte slice within the row
  const int R = wave * RPW + r;       // row state index within the workgroup

  float qv[GB][EPL];
#pragma unroll
  for (int g = 0; g < GB; ++g) {
    const uint4 raw = load16(q + b * a.qs0 + (h0 + g) * a.qs1 + c * EPL);
#pragma unroll
    for (int e = 0; e < EPL; ++e) qv[g][e] = Vec16<T>::get(raw, e);
  }

  float m[GB], l[GB], acc[GB][EPL];
#pragma unroll
  for (int g = 0; g < GB; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[g][e] = 0.0f;
  }

  const int32_t* bt_row = block_table + b * a.bts0;
  const int bs_mask = (1 << a.bs_log2) - 1;
  const T* kbase = kc + kvh * a.ks2 + c * EPL;
  const T* vbase = vc + kvh * a.vs2 + c * EPL;

  for (int t0 = t_begin; t0 < t_end; t0 += L::BATCH) {
    uint4 kr[kUnroll], vr[kUnroll];
    bool valid[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int tok = t0 + u * NR + R;
      valid[u] = tok < t_end;
      const int page = tok >> a.bs_log2;
      const int64_t blk = valid[u] ? int64_t(bt_row[page]) : 0;
      const int off = tok & bs_mask;
      kr[u] = valid[u] ? load16(kbase + blk * a.ks0 + off * a.ks1) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int tok = t0 + u * NR + R;
      const int page = tok >> a.bs_log2;
      const int64_t blk = valid[u] ? int64_t(bt_row[page]) : 0;
      const int off = tok & bs_mask;
      vr[u] = valid[u] ? load16(vbase + blk * a.vs0 + off * a.vs1) : make_uint4(0, 0, 0, 0);
    }

    float s[kUnroll][GB];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
      for (int g = 0; g < GB; ++g) {
        float dot = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) dot = fmaf(qv[g][e], Vec16<T>::get(kr[u], e), dot);
        dot = group_allreduce<LPR, SumOp>(dot);
        s[u][g] = valid[u] ? dot * a.scale_log2 : -INFINITY;
      }
    }

#pragma unroll
    for (int g = 0; g < GB; ++g) {
      float mb = s[0][g];
#pragma unroll
      for (int u = 1; u < kUnroll; ++u) mb = fmaxf(mb, s[u][g]);
      const float m_new = fmaxf(m[g], mb);
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      const float alpha = fast_exp2(m[g] - m_use);
      m[g] = m_new;
      float lsum = l[g] * alpha;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[g][e] *= alpha;
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const float p = fast_exp2(s[u][g] - m_use);
        lsum += p;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] = fmaf(p, Vec16<T>::get(vr[u], e), acc[g][e]);
      }
      l[g] = lsum;
    }
  }

  // Merge the NR row states of this workgroup through LDS.
  float* sm_m = smem;
  float* sm_l = sm_m + NR * GB;
  float* sm_acc = sm_l + NR * GB;
#pragma unroll
  for (int g = 0; g < GB; ++g) {
    if (c == 0) {
      sm_m[R * GB + g] = m[g];
      sm_l[R * GB + g] = l[g];
    }
#pragma unroll
    for (int e = 0; e < EPL; ++e) sm_acc[(R * GB + g) * D + c * EPL + e] = acc[g][e];
  }
  __syncthreads();

  for (int i = threadIdx.x; i < GB * D; i += kThreads) {
    const int g = i / D, d = i - g * D;
    float M = -INFINITY;
    for (int j = 0; j < NR; ++j) M = fmaxf(M, sm_m[j * GB + g]);
    const float M_use = M == -INFINITY ? 0.0f : M;
    float Ls = 0.0f, As = 0.0f;
    for (int j = 0; j < NR; ++j) {
      const float w = fast_exp2(sm_m[j * GB + g] - M_use);
      Ls = fmaf(sm_l[j * GB + g], w, Ls);
      As = fmaf(sm_acc[(j * GB + g) * D + d], w, As);
    }
    const int h = h0 + g;
    if (n_split_b <= 1) {
      out[b * a.os0 + h * a.os1 + d] = from_f32<T>(As / fmaxf(Ls, 1.0f));
    } else {
      const int64_t slot = (int64_t(b) * a.H + h) * a.n_splits + split;
      ws_acc[slot * D + d] = As;
      if (d == 0) {
        ws_ml[slot * 2 + 0] = M;
        ws_ml[slot * 2 + 1] = Ls;
      }
    }
  }
}

// Log-sum-exp merge of the split partials of one (row, query head); rows that fit in one
// split were finished by the split kernel and are skipped here.
template <typename T, int D>
__global__ __launch_bounds__(D) void decode_merge_kernel(const int32_t* __restrict__ seqlen,
                                                         const float* __restrict__ ws_acc,
                                                         const float* __restrict__ ws_ml,
                                                         T* __restrict__ out, DecodeArgs a) {
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int capacity = a.max_blocks << a.bs_log2;
  int len = seqlen[b];
  len = len < capacity ? len : capacity;
  const int n = (len + a.chunk - 1) / a.chunk;
  if (n <= 1) return;
  const int d = threadIdx.x;
  const int64_t base = (int64_t(b) * a.H + h) * a.n_splits;
  float M = -INFINITY;
  for (int s = 0; s < n; ++s) M = fmaxf(M, ws_ml[(base + s) * 2]);
  const float M_use = M == -INFINITY ? 0.0f : M;
  float Ls = 0.0f, As = 0.0f;
  for (int s = 0; s < n; ++s) {
    const float w = fast_exp2(ws_ml[(base + s) * 2] - M_use);
    Ls = fmaf(ws_ml[(base + s) * 2 + 1], w, Ls);
    As = fmaf(ws_acc[(base + s) * D + d], w, As);
  }
  out[b * a.os0 + h * a.os1 + d] = from_f32<T>(As / fmaxf(Ls, 1.0f));
}

int ilog2_exact(int x) {
  int lg = 0;
  while ((1 << lg) < x) ++lg;
  return (1 << lg) == x ? lg : -1;
}

bool supported_d(int D) { return D == 16 || D == 32 || D == 64 || D == 128 || D == 256; }

int esize_of(int dtype) { return dtype == MI_F32 ? 4 : (dtype == MI_F16 || dtype == MI_BF16) ? 2 : 0; }

template <typename T, int D, int GB>
size_t smem_bytes() {
  return size_t(Layout<T, D, GB>::NR) * GB * (D + 2) * sizeof(float);
}

// Heads per workgroup: the largest of 8/4/2/1 that divides the GQA group and keeps the
// LDS merge buffer within 64 KiB.
int pick_gb(int G, int NR, int D) {
  for (int gb = 8; gb >= 1; gb /= 2) {
    if (G % gb == 0 && size_t(NR) * gb * (D + 2) * 4 <= 65536) return gb;
  }
  return 1;
}

int rows_per_batch(int dtype, int D, int GB) {
  const int es = esize_of(dtype);
  const int lpr = D * es / 16;
  return kWaves * (64 / lpr) * unroll_for(GB);
}

// Tokens per split: as large as 256 (fewer partials to merge) but small enough that the
// grid has >= 2048 workgroups to spread over 256 CUs, never below one batch.
int pick_chunk(int B, int H_kv, int n_hchunks, int capacity, int batch) {
  int chunk = batch > 256 ? batch : 256;
  while (chunk > batch && chunk > 64) {
    const long long wgs = (long long)B * H_kv * n_hchunks * ((capacity + chunk - 1) / chunk);
    if (wgs >= 2048) break;
    chunk /= 2;
  }
  return chunk;
}

template <typename T, int D, int GB>
int launch_typed(const void* q, const void* kc, const void* vc, const int32_t* bt,
                 const int32_t* seqlen, void* out, float* ws_acc, float* ws_ml,
                 const DecodeArgs& a, hipStream_t stream) {
  const size_t smem = smem_bytes<T, D, GB>();
  dim3 grid(a.n_splits, a.H_kv * a.n_hchunks, a.B);
  hipLaunchKernelGGL((decode_split_kernel<T, D, GB>), grid, dim3(kThreads), smem, stream,
                     static_cast<const T*>(q), static_cast<const T*>(kc),
                     static_cast<const T*>(vc), bt, seqlen, static_cast<T*>(out), ws_acc, ws_ml,
                     a);
  int rc = launch_status("mi_paged_decode (split kernel)");
  if (rc != MI_OK || a.n_splits <= 1) return rc;
  hipLaunchKernelGGL((decode_merge_kernel<T, D>), dim3(a.H, a.B), dim3(D), 0, stream, seqlen,
                     ws_acc, ws_ml, static_cast<T*>(out), a);
  return launch_status("mi_paged_decode (merge kernel)");
}

template <typename T, int D>
int dispatch_gb(int GB, const void* q, const void* kc, const void* vc, const int32_t* bt,
                const int32_t* seqlen, void* out, float* ws_acc, float* ws_ml,
                const DecodeArgs& a, hipStream_t s) {
  switch (GB) {
    case 1: return launch_typed<T, D, 1>(q, kc, vc, bt, seqlen, out, ws_acc, ws_ml, a, s);
    case 2: return launch_typed<T, D, 2>(q, kc, vc, bt, seqlen, out, ws_acc, ws_ml, a, s);
    case 4: return launch_typed<T, D, 4>(q, kc, vc, bt, seqlen, out, ws_acc, ws_ml, a, s);
    case 8: return launch_typed<T, D, 8>(q, kc, vc, bt, seqlen, out, ws_acc, ws_ml, a, s);
  }
  return fail(MI_ERR_UNSUPPORTED, "mi_paged_decode: no kernel for %d heads per workgroup", GB);
}

template <typename T>
int dispatch_d(int D, int GB, const void* q, const void* kc, const void* vc, const int32_t* bt,
               const int32_t* seqlen, void* out, float* ws_acc, float* ws_ml,
               const DecodeArgs& a, hipStream_t s) {
  switch (D) {
    case 16:
      if constexpr (sizeof(T) == 2) return dispatch_gb<T, 16>(GB, q, kc, vc, bt, seqlen, out, ws_acc, ws_ml, a, s);
      break;
    case 32: return dispatch_gb<T, 32>(GB, q, kc, vc, bt, seqlen, out, ws_acc, ws_ml, a, s);
    case 64: return dispatch_gb<T, 64>(GB, q, kc, vc, bt, seqlen, out, ws_acc, ws_ml, a, s);
    case 128: return dispatch_gb<T, 128>(GB, q, kc, vc, bt, seqlen, out, ws_acc, ws_ml, a, s);
    case 256: return dispatch_gb<T, 256>(GB, q, kc, vc, bt, seqlen, out, ws_acc, ws_ml, a, s);
  }
  return fail(MI_ERR_UNSUPPORTED,
              "mi_paged_decode: head_dim %d is not supported by the HIP decode kernel "
              "(supported: 32, 64, 128, 256; 16 for fp16/bf16)",
              D);
}

size_t workspace_bytes_for(int B, int H, int D, int n_splits) {
  if (n_splits <= 1) return 0;
  return size_t(B) * H * n_splits * (size_t(D) + 2) * sizeof(float);
}

}  // namespace
}  // namespace miattn

extern "C" size_t mi_paged_decode_workspace_size(int B, int H, int H_kv, int D, int block_size,
                                                 int max_blocks) {
  (void)H_kv;
  if (B <= 0 || H <= 0 || D <= 0 || block_size <= 0 || max_blocks <= 0) return 0;
  // Upper bound over every dtype and chunk choice: the smallest chunk the launcher picks
  // is 64 tokens.
  const long long capacity = (long long)max_blocks * block_size;
  const int n_splits = int((capacity + 63) / 64);
  return miattn::workspace_bytes_for(B, H, D, n_splits);
}

extern "C" int mi_paged_decode(const void* q, const void* k_cache, const void* v_cache,
                               const int32_t* block_table, const int32_t* seqlen, void* out, int B,
                               int H, int H_kv, int D, int block_size, int max_blocks,
                               const int64_t* strides, float scale, int dtype, void* workspace,
                               size_t workspace_bytes, void* stream) {
  using namespace miattn;
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
  const int64_t* st = strides;
  // 16-byte vector access needs a contiguous head_dim and 16-byte aligned rows.
  const int es = esize_of(dtype);
  auto al = [&](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  const bool rows_ok = st[2] == 1 && st[6] == 1 && st[10] == 1 && st[13] == 1;
  const bool strides_ok = (st[0] * es) % 16 == 0 && (st[1] * es) % 16 == 0 &&
                          (st[3] * es) % 16 == 0 && (st[4] * es) % 16 == 0 &&
                          (st[5] * es) % 16 == 0 && (st[7] * es) % 16 == 0 &&
                          (st[8] * es) % 16 == 0 && (st[9] * es) % 16 == 0;
  if (!rows_ok || !strides_ok || !al(q) || !al(k_cache) || !al(v_cache)) {
    return fail(MI_ERR_UNSUPPORTED,
                "mi_paged_decode: q/k_cache/v_cache need a contiguous, 16-byte aligned head_dim "
                "(strides q=%lld,%lld,%lld k=%lld,%lld,%lld,%lld)",
                (long long)st[0], (long long)st[1], (long long)st[2], (long long)st[3],
                (long long)st[4], (long long)st[5], (long long)st[6]);
  }
  const int G = H / H_kv;
  const int lpr = D * es / 16;
  const int NR = kWaves * (64 / lpr);
  const int GB = pick_gb(G, NR, D);
  const int n_hchunks = G / GB;
  const int capacity = max_blocks * block_size;
  const int batch = rows_per_batch(dtype, D, GB);
  const int chunk = pick_chunk(B, H_kv, n_hchunks, capacity, batch);
  const int n_splits = (capacity + chunk - 1) / chunk;
  if (n_splits > 65535 || H_kv * n_hchunks > 65535 || B > 65535) {
    return fail(MI_ERR_UNSUPPORTED, "mi_paged_decode: grid too large (B=%d, splits=%d)", B, n_splits);
  }
  const size_t need = workspace_bytes_for(B, H, D, n_splits);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    return fail(MI_ERR_WORKSPACE, "mi_paged_decode: workspace of %zu bytes < %zu needed",
                workspace_bytes, need);
  }
  float* ws_acc = static_cast<float*>(workspace);
  float* ws_ml = need > 0 ? ws_acc + size_t(B) * H * n_splits * D : nullptr;

  DecodeArgs a;
  a.B = B; a.H = H; a.H_kv = H_kv; a.G = G; a.n_hchunks = n_hchunks; a.bs_log2 = bs_log2;
  a.max_blocks = max_blocks; a.chunk = chunk; a.n_splits = n_splits;
  a.qs0 = st[0]; a.qs1 = st[1];
  a.ks0 = st[3]; a.ks1 = st[4]; a.ks2 = st[5];
  a.vs0 = st[7]; a.vs1 = st[8]; a.vs2 = st[9];
  a.os0 = st[11]; a.os1 = st[12];
  a.bts0 = st[14];
  a.scale_log2 = scale * 1.4426950408889634f;

  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case MI_F32: return dispatch_d<float>(D, GB, q, k_cache, v_cache, block_table, seqlen, out, ws_acc, ws_ml, a, s);
    case MI_F16: return dispatch_d<f16_t>(D, GB, q, k_cache, v_cache, block_table, seqlen, out, ws_acc, ws_ml, a, s);
    case MI_BF16: return dispatch_d<bf16_t>(D, GB, q, k_cache, v_cache, block_table, seqlen, out, ws_acc, ws_ml, a, s);
  }
  return fail(MI_ERR_INVALID, "mi_paged_decode: unknown dtype %d", dtype);
}
