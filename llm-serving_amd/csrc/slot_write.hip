// Paged KV slot write: pool_flat[slot_ids[i]] = src[i] for K and V in one launch.
//
// Replaces the two index_copy_ calls of PagedPool.write_slots (reference
// model/paged.py:236-239). A slot is one row of the flat (n_blocks * block_size, H_kv, D)
// pool view, i.e. H_kv * D contiguous elements (2 KiB at the Qwen3-0.6B shape in bf16).
//
// HBM-bound byte copy: each thread moves one 16-byte chunk of K and the matching chunk
// of V, so a wave reads 1 KiB of a source row and writes 1 KiB of a destination row, both
// contiguous whenever the source row is. Algorithmic traffic is 2 * n_tokens * H_kv * D *
// esize read + the same written. Loads and stores carry the nontemporal hint: each byte is
// touched once here; the written slots are next read a decode step later, and the prefill
// that follows reads the source rows, but a packed group's K/V (17.7 MB at 4311 tokens, 35 MB
// read and written) is far more than one XCD's 4 MB L2 (measured on that group: 10.06 -> 9.30 us, the prefill
// after it unchanged; more chunks per thread, 2/4/8 with all loads first, measured slower:
// 10.2/10.6/11.7 us). The row loads do not wait for the slot id (one round trip per chunk,
// not two: 9.4 -> 8.7-9.0 us).
// Sources with a non-unit element stride or 16-byte misalignment take the scalar kernel
// (same bytes, element granularity).
#include <type_traits>

#include "common.h"

namespace miattn {
namespace {

template <typename IdxT>
__device__ __forceinline__ bool slot_in_range(IdxT slot, int64_t n_slots) {
  return slot >= 0 && int64_t(slot) < n_slots;
}

__device__ __forceinline__ void record_bad_token(int32_t* err, int64_t token) {
  if (err != nullptr) atomicCAS(err, 0, int32_t(token + 1));
}

// chunks_per_row = H_kv * D * esize / 16; chunks_per_head = D * esize / 16.
// Source strides are in bytes here (the launcher converts). kPow2: both counts are powers of
// two (row_log2 / head_log2 their logs), so a chunk's token, head and part come from shifts
// and masks; otherwise from a 64-bit and a 32-bit division, ~130 instructions ahead of the
// first load.
template <typename IdxT, bool kPow2>
__global__ __launch_bounds__(256) void slot_write_vec16(
    const uint8_t* __restrict__ k, const uint8_t* __restrict__ v, const IdxT* __restrict__ slots,
    uint8_t* __restrict__ k_pool, uint8_t* __restrict__ v_pool, int64_t n_tokens,
    int chunks_per_row, int chunks_per_head, int row_log2, int head_log2, int64_t ks0, int64_t ks1,
    int64_t vs0, int64_t vs1, int64_t n_slots, int32_t* err) {
  const int64_t total = n_tokens * chunks_per_row;
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
    int64_t token;
    int chunk, head, part;
    if constexpr (kPow2) {
      token = i >> row_log2;
      chunk = int(i & (chunks_per_row - 1));
      head = chunk >> head_log2;
      part = chunk & (chunks_per_head - 1);
    } else {
      token = i / chunks_per_row;
      chunk = int(i - token * chunks_per_row);
      head = chunk / chunks_per_head;
      part = chunk - head * chunks_per_head;
    }
    // the source rows do not depend on the slot: their loads go out with the slot id's, so
    // the chain is one memory round trip, not two
    uint4 kv = load16_nt(k + token * ks0 + head * ks1 + part * 16);
    uint4 vv = load16_nt(v + token * vs0 + head * vs1 + part * 16);
    IdxT slot = slots[token];
    // (pinned here: left alone the compiler sinks the row loads behind the slot check)
    asm volatile("" : "+v"(kv.x), "+v"(kv.y), "+v"(kv.z), "+v"(kv.w), "+v"(vv.x), "+v"(vv.y), "+v"(vv.z),
                      "+v"(vv.w), "+v"(slot));
    if (!slot_in_range(slot, n_slots)) {
      record_bad_token(err, token);
      continue;
    }
    const int64_t dst = (int64_t(slot) * chunks_per_row + chunk) * 16;
    store16_nt(k_pool + dst, kv);
    store16_nt(v_pool + dst, vv);
  }
}

// Element-granular copy for strided or misaligned sources; strides in elements.
template <typename E, typename IdxT>
__global__ __launch_bounds__(256) void slot_write_scalar(
    const E* __restrict__ k, const E* __restrict__ v, const IdxT* __restrict__ slots,
    E* __restrict__ k_pool, E* __restrict__ v_pool, int64_t n_tokens, int H_kv, int D,
    int64_t ks0, int64_t ks1, int64_t ks2, int64_t vs0, int64_t vs1, int64_t vs2,
    int64_t n_slots, int32_t* err) {
  const int64_t row = int64_t(H_kv) * D;
  const int64_t total = n_tokens * row;
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t token = i / row;
    const int64_t within = i - token * row;
    const int head = int(within / D);
    const int d = int(within - int64_t(head) * D);
    const IdxT slot = slots[token];
    if (!slot_in_range(slot, n_slots)) {
      record_bad_token(err, token);
      continue;
    }
    const int64_t dst = int64_t(slot) * row + within;
    k_pool[dst] = k[token * ks0 + head * ks1 + d * ks2];
    v_pool[dst] = v[token * vs0 + head * vs1 + d * vs2];
  }
}

int esize_of(int dtype) {
  switch (dtype) {
    case MI_F32: return 4;
    case MI_F16:
    case MI_BF16: return 2;
    default: return 0;
  }
}

template <typename IdxT>
int launch(const void* k, const void* v, const IdxT* slots, void* k_pool, void* v_pool,
           int64_t n_tokens, int H_kv, int D, int64_t n_slots, const int64_t* st, int esize,
           int32_t* err, hipStream_t stream) {
  const int64_t row_bytes = int64_t(H_kv) * D * esize;
  const bool aligned =
      (reinterpret_cast<uintptr_t>(k) % 16 == 0) && (reinterpret_cast<uintptr_t>(v) % 16 == 0) &&
      (reinterpret_cast<uintptr_t>(k_pool) % 16 == 0) &&
      (reinterpret_cast<uintptr_t>(v_pool) % 16 == 0) && st[2] == 1 && st[5] == 1 &&
      (int64_t(D) * esize) % 16 == 0 && (st[0] * esize) % 16 == 0 && (st[1] * esize) % 16 == 0 &&
      (st[3] * esize) % 16 == 0 && (st[4] * esize) % 16 == 0;
  if (aligned) {
    const int chunks_per_row = int(row_bytes / 16);
    const int chunks_per_head = int(int64_t(D) * esize / 16);
    const int64_t total = n_tokens * chunks_per_row;
    const int64_t blocks = (total + 255) / 256;
    const unsigned grid = unsigned(blocks < (1 << 20) ? blocks : (1 << 20));
    auto log2_of = [](int x) { return (x & (x - 1)) == 0 ? __builtin_ctz(unsigned(x)) : -1; };
    const int row_log2 = log2_of(chunks_per_row), head_log2 = log2_of(chunks_per_head);
    auto go = [&](auto pow2) {
      hipLaunchKernelGGL((slot_write_vec16<IdxT, decltype(pow2)::value>), dim3(grid), dim3(256), 0, stream,
                         static_cast<const uint8_t*>(k), static_cast<const uint8_t*>(v), slots,
                         static_cast<uint8_t*>(k_pool), static_cast<uint8_t*>(v_pool), n_tokens, chunks_per_row,
                         chunks_per_head, row_log2, head_log2, st[0] * esize, st[1] * esize, st[3] * esize,
                         st[4] * esize, n_slots, err);
    };
    if (row_log2 >= 0 && head_log2 >= 0) {
      go(std::true_type{});
    } else {
      go(std::false_type{});
    }
    return launch_status("mi_kv_slot_write");
  }
  const int64_t total = n_tokens * H_kv * D;
  const int64_t blocks = (total + 255) / 256;
  const unsigned grid = unsigned(blocks < (1 << 20) ? blocks : (1 << 20));
#define MI_SCALAR(E)                                                                        \
  hipLaunchKernelGGL((slot_write_scalar<E, IdxT>), dim3(grid), dim3(256), 0, stream,        \
                     static_cast<const E*>(k), static_cast<const E*>(v), slots,             \
                     static_cast<E*>(k_pool), static_cast<E*>(v_pool), n_tokens, H_kv, D,   \
                     st[0], st[1], st[2], st[3], st[4], st[5], n_slots, err)
  if (esize == 4) {
    MI_SCALAR(uint32_t);
  } else {
    MI_SCALAR(uint16_t);
  }
#undef MI_SCALAR
  return launch_status("mi_kv_slot_write");
}

}  // namespace
}  // namespace miattn

extern "C" int mi_kv_slot_write(const void* k, const void* v, const void* slot_ids, int slot_bits,
                                void* k_pool, void* v_pool, int64_t n_tokens, int H_kv, int D,
                                int64_t n_slots, const int64_t* src_strides, int dtype,
                                int32_t* error_word, void* stream) {
  using namespace miattn;
  const int esize = esize_of(dtype);
  if (esize == 0) return fail(MI_ERR_INVALID, "mi_kv_slot_write: unknown dtype code %d", dtype);
  if (n_tokens < 0 || H_kv < 1 || D < 1 || n_slots < 0) {
    return fail(MI_ERR_INVALID,
                "mi_kv_slot_write: bad sizes n_tokens=%lld H_kv=%d D=%d n_slots=%lld",
                (long long)n_tokens, H_kv, D, (long long)n_slots);
  }
  if (slot_bits != 32 && slot_bits != 64) {
    return fail(MI_ERR_INVALID, "mi_kv_slot_write: slot_bits must be 32 or 64, got %d", slot_bits);
  }
  if (src_strides == nullptr) return fail(MI_ERR_INVALID, "mi_kv_slot_write: src_strides is NULL");
  if (n_tokens == 0) return MI_OK;
  if (k == nullptr || v == nullptr || slot_ids == nullptr || k_pool == nullptr || v_pool == nullptr) {
    return fail(MI_ERR_INVALID, "mi_kv_slot_write: NULL tensor pointer");
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (slot_bits == 32) {
    return launch(k, v, static_cast<const int32_t*>(slot_ids), k_pool, v_pool, n_tokens, H_kv, D,
                  n_slots, src_strides, esize, error_word, s);
  }
  return launch(k, v, static_cast<const int64_t*>(slot_ids), k_pool, v_pool, n_tokens, H_kv, D,
                n_slots, src_strides, esize, error_word, s);
}
