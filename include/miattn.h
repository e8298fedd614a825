/*
 * miattn.h -- C ABI of the MI355X (gfx950) attention hot path.
 *
 * Three operations, each a hand-written HIP kernel family in libmiattn.so:
 *
 *   mi_kv_slot_write   paged KV slot scatter   replaces PagedPool.write_slots
 *                                              (reference model/paged.py:188-239, the two
 *                                              index_copy_ calls at :238-239)
 *   mi_paged_decode    block-table GQA decode  replaces paged_decode + _paged_decode_kernel
 *                                              (reference model/triton_decode.py:250-328,
 *                                              kernel :545-643)
 *   mi_varlen_prefill  packed varlen causal    replaces FlashVarlen.prefill_varlen
 *                      prefill attention       (reference model/attention/varlen.py:317-357)
 *   mi_qk_norm_rope_write  decode-step         fuses q_norm/k_norm + apply_rotary_emb +
 *                      attention epilogue      PagedKV.write (reference model/layers.py:193-211,
 *                                              :342-350, :59-89; model/paged.py:503-520)
 *   mi_add_rms_norm,   decode-step small ops   residual add + RMSNorm, SiLU(gate) * up
 *   mi_silu_mul                                (reference model/layers.py:365-367, :342-350,
 *                                              :325-335)
 *   mi_rows_gemm       decode-step projections nn.Linear at a few rows: q/k/v, o, gate/up,
 *   (+ _glu, _argmax)                          down, lm_head (reference model/layers.py:176-222,
 *                                              :325-335; model/minillm.py lm_head)
 *   mi_decode_step_begin, decode-step          slot map + seqlen + embedding + layer-0 norm;
 *   mi_greedy_advance(_tiles), bookkeeping     greedy argmax, tokens, history, positions
 *   mi_argmax_rows                             (reference model/paged.py:474-501, the
 *                                              generate loop's argmax)
 *
 * Conventions shared by every entry point:
 *   - every pointer except the `host_*` arguments is a device pointer;
 *   - strides are in ELEMENTS, not bytes;
 *   - `stream` is a hipStream_t passed as void* (0 = the legacy default stream);
 *   - the return value is MI_OK (0) or a negative MI_ERR_* code; mi_last_error() gives the
 *     message of the last failing call on the calling host thread;
 *   - no entry point allocates device memory: scratch space is a caller-owned workspace
 *     whose size the matching *_workspace_size() query returns (mi_paged_decode_noalloc
 *     uses a library-held device array instead);
 *   - launches are asynchronous on `stream`; nothing here synchronises the device.
 */
#ifndef MIATTN_H_
#define MIATTN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of q/k/v/out and of the KV pools. */
enum mi_dtype { MI_F32 = 0, MI_F16 = 1, MI_BF16 = 2 };

/* Return codes. The Python shim maps INVALID/UNSUPPORTED/WORKSPACE to ValueError and
 * LAUNCH to RuntimeError, the split the reference draws between caller bugs and
 * environment failures (reference model/triton_decode.py:120-132). */
enum mi_status {
  MI_OK = 0,
  MI_ERR_INVALID = -1,     /* argument/shape contract violated                         */
  MI_ERR_UNSUPPORTED = -2, /* legal shape that no kernel instantiation covers           */
  MI_ERR_WORKSPACE = -3,   /* workspace pointer/size does not cover the launch          */
  MI_ERR_LAUNCH = -4       /* the HIP runtime rejected the launch                       */
};

/* Message of the last failing call on this host thread ("" when none). */
const char* mi_last_error(void);

/* ABI version: bumps whenever a signature below or a layout it documents changes. */
int mi_abi_version(void);

/* ------------------------------------------------------------------ KV slot write
 * Replaces PagedPool.write_slots (reference model/paged.py:188-239):
 *     k_pool_flat[slot_ids[i]] = k[i];  v_pool_flat[slot_ids[i]] = v[i]
 * over the flat (n_slots, H_kv, D) view of a (n_blocks, block_size, H_kv, D) pool.
 * The pools are contiguous; k/v are (n_tokens, H_kv, D) with arbitrary element strides
 * src_strides = {k_s0, k_s1, k_s2, v_s0, v_s1, v_s2}. slot_ids are int32
 * (slot_bits == 32) or int64 (slot_bits == 64). A pure copy: bit-exact by construction.
 * A slot outside [0, n_slots) is never written: the kernel skips that token and stores
 * 1 + its index into *error_word (device int32, may be NULL) so the caller can raise
 * without a per-call host synchronisation. Distinct slots are the caller's contract
 * (reference model/paged.py:196-199); with duplicates the winner is unspecified. */
int mi_kv_slot_write(const void* k, const void* v, const void* slot_ids, int slot_bits,
                     void* k_pool, void* v_pool, int64_t n_tokens, int H_kv, int D,
                     int64_t n_slots, const int64_t* src_strides, int dtype,
                     int32_t* error_word, void* stream);

/* ------------------------------------------------------------------ decode-step epilogue
 * One decode step's attention epilogue of one layer, fused (the reference runs it as tensor
 * ops: q_norm / k_norm = RMSNorm, model/layers.py:342-350 at :193-194; apply_rotary_emb,
 * :59-89 at :210-211; then PagedKV.write, model/paged.py:503-520). For each row b of the
 * packed projection output qkv (B rows of row_stride elements, each [q (H x D) | k (H_kv
 * x D) | v (H_kv x D)]):
 *     q_out[b, h]           = rope(rmsnorm(q[b, h], q_norm_w), pos[b])       (B, H, D) contiguous
 *     k_pool_flat[slot[b]]  = rope(rmsnorm(k[b, :], k_norm_w), pos[b])
 *     v_pool_flat[slot[b]]  = v[b, :]
 * norm_mode 0: rmsnorm(x, w) = x / sqrt(mean(x^2) + eps) * w with the reference's per-op
 * rounding to the activation dtype (Qwen3, model/layers.py:342-350); norm_mode 1: Qwen3.5's
 * zero-centred norm x * (1 / sqrt(mean(x^2) + eps)) * (1 + w) in fp32, rounded once
 * (model/qwen35.py:67-89). rope: NeoX rotation of the first rotary_dim elements of each head
 * (64, 128 or 256, <= D; the rest pass through, model/layers.py:91-117) with the
 * (n_pos, rotary_dim/2) cos/sin tables at row pos[b] (int64), each product and sum rounded
 * to the activation dtype (see csrc/decode_epilogue.hip). slot_ids as for mi_kv_slot_write (int32 or
 * int64 per slot_bits; pools (n_slots, H_kv, D) contiguous). A row with slot -1 has nothing to
 * write this step and is skipped silently; any other row whose position is outside
 * [0, n_pos) or whose slot is outside [0, n_slots) is not written to the pools and 1 + its
 * index goes to *error_word (may be NULL). Both kinds of row get zeros in q_out (and in
 * k_out / v_out when given). D = 64, 128 or 256. qkv_parts = 0: qkv holds `dtype` values;
 * qkv_parts = n >= 1: qkv holds fp32 split-K partial sums [n][B][row_stride] (mi_rows_gemm
 * with n_split = n), summed in split order and rounded once to `dtype` before the above.
 * k_out / v_out (may be NULL): the roped k and the v rows also written packed, (B, H_kv, D)
 * contiguous -- a packed prefill group's q/k norm + RoPE + slot write in one launch, its
 * attention then reading q_out, k_out, v_out (reference model/packed.py:187-218). */
int mi_qk_norm_rope_write(const void* qkv, int64_t row_stride, int qkv_parts, const void* q_norm_w,
                          const void* k_norm_w, const void* cos_tab, const void* sin_tab,
                          int64_t n_pos, int rotary_dim, const int64_t* pos, const void* slot_ids,
                          int slot_bits, void* q_out, void* k_pool, void* v_pool, void* k_out, void* v_out,
                          int B, int H, int H_kv, int D, int64_t n_slots, float eps, int norm_mode, int dtype,
                          int32_t* error_word, void* stream);

/* ------------------------------------------------------------------ decode-step small ops
 * The residual stream's add + RMSNorm and the MLP's SiLU(gate) * up, each one launch (the
 * reference runs them as tensor ops: block x = x + attn(norm1(x)); x = x + mlp(norm2(x)),
 * model/layers.py:365-367; RMSNorm :342-350; MLP down(silu(gate(x)) * up(x)), :325-335),
 * rounded op by op to the activation dtype like those ops (see csrc/decode_step.hip).
 * mi_add_rms_norm: rows x cols contiguous; s = x + delta (delta may be NULL: s = x);
 *   x_out = s (may be NULL, may alias x); h_out = s / sqrt(mean(s^2) + eps) * weight.
 *   cols <= 4096.
 * mi_silu_mul: gate_up (rows, 2 * inter) contiguous rows [gate | up];
 *   out (rows, inter) = silu(gate) * up.
 * delta_parts / gate_up_parts = 0: that input holds `dtype` values; n >= 1: it holds fp32
 * split-K partial sums [n][rows][cols] of mi_rows_gemm, summed in split order and rounded
 * once to `dtype` (the projection output's own rounding) before the chain above. */
int mi_add_rms_norm(const void* x, const void* delta, int delta_parts, const void* weight, void* x_out,
                    void* h_out, int rows, int cols, float eps, int dtype, void* stream);
int mi_silu_mul(const void* gate_up, int gate_up_parts, void* out, int rows, int inter, int dtype,
                void* stream);

/* Greedy pick of the decode step (the reference's logits.argmax(-1) in its generate loop):
 * out[r] = torch.argmax(x[r, :cols]) for each of `rows` rows of row stride ld -- the first
 * index of the largest value, NaN above every number. out: int64 (rows,). */
int mi_argmax_rows(const void* x, int64_t ld, int rows, int cols, int64_t* out, int dtype, void* stream);

/* The rest of a captured greedy decode step's bookkeeping, so the step needs no tensor ops
 * (reference: the slot map model/paged.py:474-501, the embedding lookup and layer 0's input
 * norm model/minillm.py:111-136, model/layers.py:342-350, the generate loop's argmax and
 * position advance).
 * mi_decode_step_begin, per row b (block_table (B, >= max_blocks) int32, row stride bt_stride;
 * a row with pos[b] < 0 is an idle seat: made inert as below without a report):
 *   seqlen[b] = pos[b] + 1;  slots[b] = table[b, pos[b] / block_size] * block_size + pos[b] % block_size;
 *   x[b] = embed[tokens[b]] (embed (vocab, cols));  h[b] = x[b] / sqrt(mean(x[b]^2) + eps) * norm_w,
 *   rounded as mi_add_rms_norm. A row whose token is outside [0, vocab), whose position is
 *   outside [0, max_blocks * block_size) or whose table entry at that position is negative
 *   (pad each row's table with -1 past its own blocks) is refused: 1 + its index goes to
 *   *error_word (may be NULL) and the row is made inert for the step (seqlen 0, slot -1,
 *   x = h = 0), so no later launch of the step writes or reads pool memory for it.
 * mi_greedy_advance: pick[r] = argmax of logits row r as mi_argmax_rows; tokens[r] = pick;
 *   history[r * hist_stride + steps[r]] = pick while 0 <= steps[r] < max_steps; steps[r] += 1;
 *   pos[r] += 1 (all int64); a row with pos[r] < 0 (an idle seat) is left unchanged. */
int mi_decode_step_begin(const int64_t* tokens, const int64_t* pos, const int32_t* block_table, int64_t bt_stride,
                         int block_size, int max_blocks, const void* embed, int64_t vocab, const void* norm_w,
                         int cols, float eps, int32_t* seqlen, int64_t* slots, void* x, void* h, int B, int dtype,
                         int32_t* error_word, void* stream);
int mi_greedy_advance(const void* logits, int64_t ld, int rows, int cols, int dtype, int64_t* tokens, int64_t* pos,
                      int64_t* history, int64_t hist_stride, int64_t* steps, int max_steps, void* stream);
/* mi_greedy_advance from mi_rows_gemm_argmax's per-tile picks (rows x n_tiles) instead of the
 * logits: the same pick, token, history, step and position updates. */
int mi_greedy_advance_tiles(const void* tile_best, int n_tiles, int rows, int64_t* tokens, int64_t* pos,
                            int64_t* history, int64_t hist_stride, int64_t* steps, int max_steps, void* stream);

/* ------------------------------------------------------------------ decode-step projections
 * out = a w^T for 1 <= M <= 32 rows (nn.Linear without bias, the reference's projections at
 * decode batch = running sequences). a (M, K), w (N, K), both with unit element stride, row
 * strides lda / ldw (multiples of 8, 16-byte aligned rows); bf16 or fp16.
 * n_split = 1: out (M, N) row stride ldo, in `dtype` (fp32 accumulation, rounded once).
 * n_split = S > 1: K is split S ways; partials (S, M, N) fp32 contiguous receive each
 *   split's sums, for a consumer that sums them (the *_parts arguments above). Needs
 *   K % (S * 256) == 0 and K / S <= 1024. One launch of ceil(N / 32) x S workgroups.
 * mi_rows_gemm_split returns the split the launcher is tuned for at that shape (0 if K is
 * not a multiple of 256). */
int mi_rows_gemm_split(int M, int N, int K);
int mi_rows_gemm(const void* a, int64_t lda, const void* w, int64_t ldw, void* out, int64_t ldo,
                 float* partials, int M, int N, int K, int n_split, int dtype, void* stream);
/* The MLP's first half in one launch: out (M, inter) = silu(a w_gate^T) * (a w_up^T), rounded
 * as the reference's F.silu(gate(x)) * up(x) (model/layers.py:325-335). w_glu (2 * inter, K)
 * holds the gate and up rows interleaved by 16: rows 32t .. 32t+15 are gate rows 16t .. 16t+15
 * and rows 32t+16 .. 32t+31 are up rows 16t .. 16t+15. inter % 16 == 0, K % 256 == 0,
 * K <= 1024 (unsplit), other requirements as mi_rows_gemm. */
int mi_rows_gemm_glu(const void* a, int64_t lda, const void* w_glu, int64_t ldw, void* out, int64_t ldo,
                     int M, int inter, int K, int dtype, void* stream);
/* An unsplit product (K % 256 == 0, K <= 1024) that also picks, for each row and each
 * 32-column tile t, the tile's best column under torch.argmax's rule on the outputs rounded
 * to `dtype` (largest value, lowest column on ties, NaN above every number):
 * tile_best[row * n_tiles + t] = {float value, int32 column}, n_tiles = ceil(N / 32). out may be NULL (the
 * products are then not stored). For a greedy step's lm_head with mi_greedy_advance_tiles. */
int mi_rows_gemm_argmax(const void* a, int64_t lda, const void* w, int64_t ldw, void* out, int64_t ldo,
                        void* tile_best, int M, int N, int K, int dtype, void* stream);

/* ------------------------------------------------------------------ paged decode
 * Replaces paged_decode (reference model/triton_decode.py:250-328) and its kernel
 * (:545-643): one query token per row against a paged KV pool.
 *   q            (B, H, D), strides {q_s0, q_s1, q_s2}, D contiguous (q_s2 == 1)
 *   k/v_cache    (n_blocks, block_size, H_kv, D), D contiguous
 *   block_table  (B, max_blocks) int32, row stride bt_s0, column-contiguous
 *   seqlen       (B,) int32 in [0, max_blocks * block_size]
 *   out          (B, H, D), strides {o_s0, o_s1, o_s2}
 * strides = {q_s0,q_s1,q_s2, k_s0,k_s1,k_s2,k_s3, v_s0,v_s1,v_s2,v_s3, o_s0,o_s1,o_s2,
 *            bt_s0}   (15 entries, elements)
 * GQA: query head h reads KV head h / (H / H_kv). Softmax is fp32 online softmax in the
 * log2 domain with scale*log2(e); out = acc / max(l, 1), so a zero-length row is exact
 * zeros (reference :639). The page walk is clamped to max_blocks (reference :593) and
 * block ids are trusted, as in the reference (:64-66).
 *
 * Split-K workspace: rows longer than one split are cut into splits whose (m, l, acc)
 * partials go to the caller's workspace; a second launch on the same stream merges them
 * (log-sum-exp) and writes `out`. mi_paged_decode_workspace_size() gives the exact size
 * for a shape and dtype (0 when no row can need a split); the workspace must be 16-byte
 * aligned. Calls that share one workspace must be ordered (one stream). */
size_t mi_paged_decode_workspace_size(int B, int H, int H_kv, int D, int block_size,
                                      int max_blocks, int dtype);
int mi_paged_decode(const void* q, const void* k_cache, const void* v_cache,
                    const int32_t* block_table, const int32_t* seqlen, void* out, int B,
                    int H, int H_kv, int D, int block_size, int max_blocks,
                    const int64_t* strides, float scale, int dtype, void* workspace,
                    size_t workspace_bytes, void* stream);

/* mi_paged_decode_fused -- one launch pair for a decode step's attention from the packed
 * q/k/v projection: what mi_qk_norm_rope_write followed by mi_paged_decode computes
 * (reference: q_norm / k_norm, apply_rotary_emb and PagedKV.write, model/layers.py:193-211
 * and model/paged.py:503-520, then paged_decode, model/triton_decode.py:250-328), with the
 * same result bit for bit and the same pool contents afterwards, minus the epilogue launch
 * and q's round trip through memory. Each decode workgroup computes its row's q (per-head
 * RMSNorm x / rms * w and whole-head NeoX RoPE at pos[b], each op rounded to the dtype as
 * in mi_qk_norm_rope_write); the workgroup holding the row's new token computes that
 * token's k and v, writes them to k_cache / v_cache at slot_ids[b] and reads them from
 * registers, not from the pool. Contract: the new token is the row's last one, pos[b] =
 * seqlen[b] - 1 (the decode step's layout). A row with slot -1 is idle (nothing written;
 * it should have seqlen 0). Any other row whose pos is outside [0, n_pos) or not seqlen - 1,
 * or whose slot is outside [0, n_slots), writes nothing, attends with q = 0 and puts 1 + its
 * index into *error_word (may be NULL) -- as the two-launch form treats it. qkv as for
 * mi_qk_norm_rope_write (T values, or fp32 split-K partials when qkv_parts >= 1), 16-byte
 * aligned rows; the other arguments as for mi_paged_decode (strides' q entries are not
 * read). Supported: head_dim 128, rotary_dim == 128, norm_mode 0 (Qwen3), fp16/bf16;
 * anything else is MI_ERR_UNSUPPORTED (use the two entry points). The new tokens' K/V are
 * written while the launch reads the pools, so no row's slot may lie inside another row's
 * first seqlen tokens (a block holding one row's new token mapped into another row's
 * table below that row's length): such a row would read the old or the new value, where
 * the two-launch form reads the new one. Tables of distinct blocks per row, as the
 * reference's BlockManager hands out, never do. */
int mi_paged_decode_fused(const void* qkv, int64_t row_stride, int qkv_parts, const void* q_norm_w,
                          const void* k_norm_w, const void* cos_tab, const void* sin_tab, int64_t n_pos,
                          int rotary_dim, const int64_t* pos, const void* slot_ids, int slot_bits,
                          void* k_cache, void* v_cache, const int32_t* block_table, const int32_t* seqlen,
                          void* out, int B, int H, int H_kv, int D, int block_size, int max_blocks,
                          int64_t n_slots, const int64_t* strides, float scale, float eps, int norm_mode,
                          int dtype, void* workspace, size_t workspace_bytes, int32_t* error_word,
                          void* stream);

/* mi_paged_decode_noalloc -- no counterpart in the reference: for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). mi_paged_decode with the same arguments minus the workspace: the
 * split-K partials go to a device array the library holds per GPU, MI_DECODE_SCRATCH_BYTES
 * (8 MiB; the Qwen3 shape fits up to B = 496 rows), from first use until the process ends.
 * A shape whose mi_paged_decode_workspace_size() exceeds it returns MI_ERR_WORKSPACE.
 * Nothing is allocated: the array's address on the current device is looked up once per
 * device (hipGetSymbolAddress); `stream` must belong to the current device. Every call on
 * one GPU shares that GPU's array, so calls that overlap on one GPU (several streams or host
 * threads in flight at once) race: order them on one stream. */
#define MI_DECODE_SCRATCH_BYTES (8u << 20)
int mi_paged_decode_noalloc(const void* q, const void* k_cache, const void* v_cache,
                            const int32_t* block_table, const int32_t* seqlen, void* out, int B,
                            int H, int H_kv, int D, int block_size, int max_blocks,
                            const int64_t* strides, float scale, int dtype, void* stream);

/* ------------------------------------------------------------------ varlen prefill
 * Replaces FlashVarlen.prefill_varlen (reference model/attention/varlen.py:317-357):
 * attention inside each cu_seqlens segment of a packed token axis, causal within the
 * segment when `causal` is non-zero; q (total, H, D), k/v (total, H_kv, D), out
 * (total, H, D), all contiguous; bf16 or fp16 (fp32 is MI_ERR_UNSUPPORTED, the same
 * dtype contract as FA2, reference :338-343).
 *   cu_seqlens      device int32 (n_seqs + 1)
 *   schedule        device copy of the int32 words mi_varlen_schedule wrote
 * mi_varlen_schedule (host only) cuts the packed batch into query tiles, splits the
 * longest causal tiles' key ranges into pieces when the launch underfills the chip, and
 * orders the pieces heaviest-first so the causal triangle does not leave a tail of long
 * tiles. By default head_dim 64/128 batches whose longest segment reaches 1536 tokens run
 * the tall kernel (below) when its schedule needs no split pieces; otherwise batches whose
 * longest segment reaches 8192 tokens run the LDS-ring kernel (128-row tiles) and shorter
 * ones the persistent duo kernel (64-row tiles, two workgroups per CU, each working through
 * its own item list); head_dim 256 runs the duo kernel at one workgroup per CU; batches of
 * more than 255 heads (beyond the duo kernel's item word) run the ring kernel at head_dim
 * 64/128 and the register-staged kernel at 256. mi_varlen_schedule_for names the kernel
 * instead (MI_PREFILL_*; the ring and tall kernels take head_dim 64 and 128, the duo
 * kernel 64, 128 and 256 with at most 255 heads, the register-staged kernel all three).
 * Layout of
 * the staged and ring schedules:
 * {n_work, n_merge, n_partials, layout}, then n_work work entries and n_merge merge
 * entries of two words each; the duo schedule is {n_workgroups, n_merge, n_partials,
 * layout}, n_workgroups entries of eight words {first item word, item count, the first
 * item's four words, 0, 0}, the merge entries of two words each, then the items of four
 * words each. It returns the word count (host_schedule = NULL sizes it).
 * It depends only on the segment lengths, H and head_dim, so a caller builds it once per
 * packed group and reuses it for every layer, passing the four header words to
 * mi_varlen_prefill.
 * Split pieces write (O, max, sum) partials into the caller's workspace of
 * mi_varlen_workspace_size() bytes (0 when nothing is split; 16-byte aligned); a second
 * launch on the same stream merges them. Calls sharing a workspace must be ordered.
 * MI_PREFILL_TALL (head_dim 64/128, at most 65535 heads) runs 128-row tiles in which each
 * wave owns 32 query rows over every key of a step; the schedule cuts long tiles' key
 * ranges into pieces that run at the same time on different workgroups and merges them in
 * the same launch (no second launch): its workspace starts with one int32 counter per split
 * tile x head (rounded up to 256 bytes), which must be zero before the first call (zero the
 * workspace once when allocating it) and which every call leaves zero, then the partials.
 * Its schedule is {n_workgroups, n_counters, n_partials, layout}, n_workgroups entries of
 * eight words {first item word, item count, the first item's six words}, then the items of
 * six words each.
 * error_word (device int32, may be NULL): a launch whose bounded wait gave up stores a
 * non-zero code there (see mi_prefill_wait_limit) and ends normally; its output is not valid.
 * The caller reads and clears it when it chooses (no per-call host synchronisation). */
enum { MI_PREFILL_AUTO = -1, MI_PREFILL_STAGED = 0, MI_PREFILL_RING = 1, MI_PREFILL_DUO = 3, MI_PREFILL_TALL = 4 };
int mi_varlen_schedule(const int32_t* host_cu_seqlens, int n_seqs, int H, int H_kv,
                       int D, int causal, int32_t* host_schedule, int capacity);
int mi_varlen_schedule_for(const int32_t* host_cu_seqlens, int n_seqs, int H, int H_kv,
                           int D, int causal, int kernel, int32_t* host_schedule, int capacity);
size_t mi_varlen_workspace_size(const int32_t* host_schedule, int H);
int mi_varlen_prefill(const void* q, const void* k, const void* v, void* out,
                      const int32_t* cu_seqlens, int n_seqs, int total_tokens,
                      int max_seqlen, const int32_t* schedule, int n_work, int n_merge,
                      int n_partials, int layout, int H, int H_kv, int D, float scale,
                      int causal, int dtype, void* workspace, size_t workspace_bytes,
                      int32_t* error_word, void* stream);
/* Test hook of the kernels' bounded waits (a tall owner waiting for its producers, a
 * head_dim 256 duo wave waiting for its partner): polls >= 0 sets how many polls a wait makes
 * before it gives up (for launches from then on, process-wide; 0: every wait gives up at
 * once); polls < 0 only queries. Returns the previous limit. A correct launch never comes
 * near the default; a small limit forces the give-up path, whose launch still ends normally
 * with its output not to be trusted and 1 (tall) or 2 (duo) in the error word. */
int mi_prefill_wait_limit(int polls);

#ifdef __cplusplus
}
#endif

#endif /* MIATTN_H_ */
