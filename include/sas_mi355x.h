/*
 * sas_mi355x.h - C ABI of the MI355X (gfx950) sparse shared-KV attention library.
 *
 * Plain pointers and sizes only; no torch or HIP C++ types beyond hipStream_t
 * (passed as void*). Every entry point returns 0 on success or a negative
 * SAS_E* code; sas_last_error() returns a message for the calling thread.
 *
 * Reference interfaces replaced (yangqiang2018/sparse_attn_sharedkv):
 *   sas_metadata_build     <- metadata.sparse_attn_sharedkv_metadata  (metadata.py:1018-1086)
 *                             (port of the AICPU SparseAttnSharedkvMetadata scheduler)
 *   sas_attention_launch   <- the JIT kernel callable built by build_sparse_attn_sharedkv
 *                             func(Q, ori_kv, ori_block_table, cmp_kv, cmp_block_table,
 *                                  cmp_indices, q_prefix, act_q_lens, seqused_kv, sinks,
 *                                  metadata) -> (Output, LSE)          (kernel.py:73-183, :353-382;
 *                             api.py:372-384 is the call site); the metadata-free twin
 *                             build_sparse_flash_mla (sparse_flash_mla_kernel.py:19-107, :189-210)
 *                             maps onto the same entry point with metadata built by the host.
 *   sas_workspace_bytes    <- workspace_idx auto-allocation of the JIT (kernel.py:353-382): the
 *                             caller allocates the split-KV partial buffer instead.
 *   sas_kv_fp8_append      <- no counterpart in the reference (its caches are bf16/fp16 only,
 *                             api.py:51-56): writer of the fp8 cache-row format that
 *                             SAS_KV_FP8_DS_MLA selects for sas_attention_launch.
 */
#ifndef SAS_MI355X_H_
#define SAS_MI355X_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- metadata layout (int32 words) -------------------------------------
 * FA rows ("virtual cores" = workgroups of the attention kernel), 8 words each,
 * same field order as metadata.py:45-52:
 *   [enable, bn2_start, m_start, s2_start, bn2_end, m_end, s2_end, first_partial_slot]
 * An item is (bn2 = batch, m = m-block): m-block m of batch b is query row
 * m / HB of that batch, heads [(m % HB) * m_base, +m_base) with
 * HB = ceil(num_heads / m_base) (the reference's s1g blocks of mBaseSize,
 * metadata.py:388, :676-679). A row covers the items from
 * (bn2_start, m_start) block s2_start up to, excluding, (bn2_end, m_end)
 * block s2_end; s2 counts SAS blocks of s2_base positions over the item's
 * attended list [window rows ++ compressed positions].
 * FD rows (split-KV merge tasks), 8 words each, field order of metadata.py:54-60:
 *   [enable, bn2_idx, m_idx, partial_slot_first, partial_count, head_start, head_count, 0]
 * (head_start / head_count are relative to the item's m-block, as fd_m_start / fd_m_num).
 * Config row (last 8 words): [SAS_META_MAGIC, s2_base, num_fa, num_fd,
 *                             num_partial_slots, num_heads, m_base, total_items]
 * Schedule key (words [SAS_META_KEY_OFFSET, SAS_CFG_OFFSET), both schedulers write it;
 * the kernels never read it): [SAS_KEY_MAGIC, items, batch, num_heads, m_base,
 * ori_win_left, scenario, cmp_ratio, cmp_topk, num_cores, s2_base, min_split_blocks,
 * fd_head_chunk, 0, 0, 0, query rows of each batch..., block count of each item...];
 * word 0 is 0 when the inputs do not fit the key region. The device scheduler
 * leaves a buffer that already holds the key of its inputs (and a valid config
 * row) as it is when called with reuse != 0: the schedule is a function of exactly
 * these words. Pass reuse != 0 only for a buffer that nothing else writes between calls.
 */
#define SAS_AIC_CORE_NUM 512
#define SAS_AIV_CORE_NUM 1024
#define SAS_FA_METADATA_SIZE 8
#define SAS_FD_METADATA_SIZE 8
#define SAS_FD_OFFSET (SAS_AIC_CORE_NUM * SAS_FA_METADATA_SIZE)
#define SAS_META_SIZE 16384
#define SAS_CFG_OFFSET (SAS_META_SIZE - 8)
#define SAS_META_MAGIC 0x5A53A355
#define SAS_META_KEY_OFFSET (SAS_FD_OFFSET + SAS_AIV_CORE_NUM * SAS_FD_METADATA_SIZE)
#define SAS_KEY_MAGIC 0x5A53C0DE

/* ---- error codes ---- */
#define SAS_OK 0
#define SAS_E_INVALID (-1)     /* bad argument (shape, pointer, scenario)      */
#define SAS_E_UNSUPPORTED (-2) /* combination this library has no kernel for   */
#define SAS_E_CAPACITY (-3)    /* schedule does not fit the metadata capacity  */
#define SAS_E_HIP (-4)         /* HIP runtime error (launch or attribute call) */

/* Scenario codes (api.py:196-202): 1 = SWA, 2 = CFA (dense compressed), 3 = SCFA (top-k). */

#define SAS_SCHED_DEVICE (-1) /* SasAttnArgs.num_fd: schedule summary read on the device */

/* Host-side scheduler (no GPU needed). Fills meta_out[SAS_META_SIZE].
 * act_q[b]: query rows of batch b; act_kv[b]: raw KV length of batch b.
 * m_base: heads per item: 32 when num_heads <= 32, 64 up to 64 heads; above 64 heads
 * 64 or 128 (one item per token: the 128-head kernel, native or fp8 rows; the
 * pipelined kernel, SAS_PHASE_PIPELINED, takes 64 only).
 * num_cores: workgroups to balance over (<= SAS_AIC_CORE_NUM).
 * s2_base: positions per schedulable block (multiple of 32).
 * min_split_blocks: an item is split across workgroups only into pieces of at
 * least this many blocks. fd_head_chunk: heads per merge task.
 * Returns the number of FA rows used (>= 1) or a negative error code. */
int sas_metadata_build(int32_t* meta_out, int batch, const int32_t* act_q,
                       const int32_t* act_kv, int num_heads, int m_base, int ori_win_left,
                       int scenario, int cmp_ratio, int cmp_topk, int num_cores,
                       int s2_base, int min_split_blocks, int fd_head_chunk);

/* On-device twin of sas_metadata_build (no reference counterpart: the reference
 * schedules on the host, metadata.py:1018-1086). One workgroup on `stream` writes
 * meta[SAS_META_SIZE] (device memory) from device-resident lengths: batch b has
 * act_q[b] query rows (act_q: [batch] int32, device) or, when act_q is NULL,
 * uniform_q rows; seqused_kv: [batch] int32 (device). Same algorithm and the same words as sas_metadata_build for the same
 * lengths. Limits: batch <= SAS_DEV_SCHED_MAX_BATCH, items (query rows x head blocks)
 * <= SAS_DEV_SCHED_MAX_ITEMS. Errors the host cannot see (a negative length, too many
 * items, a schedule over capacity) leave the config row without SAS_META_MAGIC and
 * its word 1 = -1 / -2 / -3; sas_attention_launch then writes NaN outputs.
 * reuse: 0 always rebuilds meta; nonzero keeps it when it already holds the schedule key
 * of these inputs and a valid config row (about 5 us instead of a full rebuild), which is
 * only sound for a buffer that the caller owns and nothing else writes between calls
 * (a captured graph's static buffer, a per-stream buffer kept for the purpose).
 * Asynchronous; returns SAS_E_INVALID for arguments checkable on the host. */
#define SAS_DEV_SCHED_MAX_BATCH 4096
#define SAS_DEV_SCHED_MAX_ITEMS 16384
int sas_metadata_build_device(int32_t* meta, int batch, const int32_t* act_q,
                              int uniform_q, const int32_t* seqused_kv, int num_heads,
                              int m_base, int ori_win_left, int scenario, int cmp_ratio,
                              int cmp_topk, int num_cores, int s2_base, int min_split_blocks,
                              int fd_head_chunk, int reuse, void* stream);

/* Bytes of split-KV partial workspace for a schedule:
 * num_partial_slots * m_base * (2 * head_dim_v + 8): the partials [slot][head][head_dim_v]
 * as fp16 (acc / l times the power of two that puts the row's largest |value| into
 * [2^14, 2^15); 1 for an all-zero row), then [slot][head] fp32 lse and [slot][head]
 * fp32 inverse scales. */
int64_t sas_workspace_bytes(int num_partial_slots, int m_base, int head_dim_v);

/* dtype codes */
#define SAS_DTYPE_BF16 0
#define SAS_DTYPE_FP16 1

/* KV cache row formats (SasAttnArgs.kv_format)
 * SAS_KV_NATIVE: a row is head_dim elements of `dtype`.
 * SAS_KV_FP8_DS_MLA: a row is SAS_FP8_ROW_BYTES = 656 bytes, for head_dim 576, dtype bf16:
 *   bytes [0, 512)   dims 0..511 as OCP fp8 e4m3 (e4m3fn: no infinities, 0x7F/0xFF NaN)
 *   bytes [512, 528) four fp32 scales; scale t covers dims 128t..128t+127
 *   bytes [528, 656) dims 512..575 (rope) as bf16
 * The attention reads dim d < 512 as bf16_rne(fp32(e4m3[d]) * scale[d / 128]) (one fp32
 * multiply, then round-to-nearest-even to bf16), i.e. exactly the bf16 cache that
 * dequantization gives, and computes on it as on a native bf16 cache. */
#define SAS_KV_NATIVE 0
#define SAS_KV_FP8_DS_MLA 1
#define SAS_FP8_ROW_BYTES 656

typedef struct SasAttnArgs {
  /* inputs (device pointers) */
  const void* q;                 /* [total_tokens, num_heads, head_dim] dtype                 */
  const void* ori_kv;            /* [ori_block_num, ori_block_size, 1, head_dim] dtype         */
  const int32_t* ori_block_table;/* [batch, ori_table_len]                                     */
  const void* cmp_kv;            /* [cmp_block_num, cmp_block_size, 1, head_dim] or NULL        */
  const int32_t* cmp_block_table;/* [batch, cmp_table_len] or NULL                             */
  const int32_t* cmp_indices;    /* [total_tokens, 1, topk] (scenario 3) or NULL               */
  const int32_t* q_prefix;       /* [batch] first flat token of each batch                     */
  const int32_t* act_q_lens;     /* [batch]                                                    */
  const int32_t* seqused_kv;     /* [batch]                                                    */
  const float* sinks;            /* [num_heads] fp32 (may hold -inf)                           */
  const int32_t* metadata;       /* [SAS_META_SIZE] from sas_metadata_build                    */
  /* outputs (device pointers) */
  void* out;                     /* [total_tokens, num_heads, head_dim_v] dtype                */
  float* lse;                    /* [total_tokens, num_heads] fp32                             */
  float* workspace;              /* sas_workspace_bytes(...) bytes, or NULL if num_fd == 0     */
  /* sizes */
  int32_t batch, total_tokens, num_heads, head_dim, head_dim_v;
  int32_t ori_block_num, ori_block_size, ori_table_len;
  int32_t cmp_block_num, cmp_block_size, cmp_table_len, topk;
  int32_t scenario, cmp_ratio, ori_win_left, dtype;
  float softmax_scale;
  /* schedule summary (copies of the metadata config row, known to the host). With
   * num_fd == SAS_SCHED_DEVICE the kernels read the summary from the config row of
   * `metadata` on the device instead (a schedule built by sas_metadata_build_device, or
   * any schedule the host has not read back): num_fa is then the launch capacity (the
   * schedule's core count must not exceed it; its FA rows fill [0, num_fa)),
   * num_partial_slots the workspace capacity in slots, and s2_base is taken from the
   * config row. A config row without SAS_META_MAGIC, or built for another head count,
   * m_base or larger capacities, makes the launch write NaN to out and lse. */
  int32_t num_fa, num_fd, num_partial_slots, s2_base, m_base;
  /* kernels to enqueue: bit 0 attention, bit 1 split-KV merge; neither means both.
   * A caller may enqueue the two phases as separate calls (attention first).
   * SAS_PHASE_PIPELINED (bit 2) runs native rows through the attention kernel
   * that fp8 rows of 64-head items use (two waves per SIMD, software-pipelined); by
   * default native rows take the one-wave-per-SIMD kernel (the 128-head kernel for
   * 128-head items and row pairs), which is faster on them. Results of the kernels
   * agree to within rounding, not bit for bit.
   * SAS_PHASE_FP8_QK (bit 3, fp8 rows only) forms Q·Kᵀ on fp8 MFMA
   * (v_mfma_f32_16x16x128_f8f6f4): each head's 512 latent query dims are quantized
   * to e4m3 with one fp32 scale: inv = 448 / amax (an IEEE fp32 division), codes =
   * RNE_e4m3(clamp(q * inv, -448, 448)) (the product in fp32), scale sq = amax / 448
   * (inv = sq = 1 for an all-zero head);
   * the cache rows' e4m3 dims are used as stored, and each row's 128-dim block scales and
   * the head's scale are applied to the four block dot products in fp32; the rope
   * dims stay bf16. P·V stays on the dequantized bf16 rows. No reference counterpart
   * (kernel.py:2036-2352 forms Q·Kᵀ in bf16): it adds the query's quantization error,
   * which is small against golden for N(0,1)-scaled data but not for the reference
   * tests' U(-10, 10) data, so it is opt-in.
   * SAS_PHASE_ROW_ITEMS (bit 4, native rows) turns off row pairs: by default a launch
   * whose sequences hold several query rows, with items of 64 heads (num_heads <= 64)
   * and scenario 1 or 2, runs two consecutive query rows per workgroup on the 128-head
   * kernel over the union of their attended rows (prefill: the two windows share all
   * but two rows); pieces of split items run alone. No
   * reference counterpart (the reference's prefill task is one query row,
   * kernel.py:262, :293); results agree with the one-row items to within rounding. */
  int32_t phases;
  /* row format of ori_kv and cmp_kv: SAS_KV_NATIVE or SAS_KV_FP8_DS_MLA */
  int32_t kv_format;
  /* Split-KV merge inside the attention kernel (no reference counterpart: the reference
   * merges in a separate stage, metadata.py:925-954). NULL: the merge kernel runs after
   * the attention kernel, as in the reference. Otherwise SAS_MERGE_SYNC_WORDS arrival
   * counters (device memory, 8-byte aligned) that are zero before the call: each piece
   * of a split item adds its block count to its item's counter after storing its
   * partial, and the piece that completes the count merges the item's partials into
   * out and lse at once, so the merge kernel is not launched (the merge phase enqueues
   * nothing). The completing piece returns the counter to zero, so a buffer zeroed once
   * stays usable; calls that may overlap (other streams, graphs replayed concurrently)
   * need distinct buffers. Results are bit-identical to the merge kernel's. Native
   * cache rows only (not with SAS_PHASE_PIPELINED); fp8 rows ignore it and run the
   * merge kernel. */
  uint64_t* merge_sync;
} SasAttnArgs;

/* SasAttnArgs.phases bits beyond the attention / merge selection (see phases) */
#define SAS_PHASE_PIPELINED 4
#define SAS_PHASE_FP8_QK 8
#define SAS_PHASE_ROW_ITEMS 16

#define SAS_MERGE_SYNC_WORDS (2 * SAS_AIC_CORE_NUM) /* uint64 counters: one per partial slot */

/* Launch the attention kernel and, when num_fd > 0 and the merge is not done inside
 * the attention kernel (merge_sync), the split-KV merge kernel on `stream` (a
 * hipStream_t). Asynchronous; no allocation, no host synchronisation. */
int sas_attention_launch(const SasAttnArgs* args, void* stream);

/* Allocation-free variant of sas_attention_launch (no counterpart in the reference:
 * for callers that cannot allocate device memory, such as code under HIP graph
 * capture, tight serving loops and harnesses that forbid allocation). Same arguments
 * and kernels; args->workspace is ignored and the split-KV partials go to a fixed
 * per-device scratch array of SAS_NOALLOC_SCRATCH_BYTES inside the library, so
 * sas_workspace_bytes(num_partial_slots, m_base, head_dim_v) must not exceed it
 * (else SAS_E_CAPACITY, nothing launched). Calls no hipMalloc/hipFree. All calls on
 * one device share its scratch array: calls that may overlap on one device (other
 * streams, concurrent threads) race and must be serialised by the caller. */
#define SAS_NOALLOC_SCRATCH_BYTES (72ull << 20)
int sas_attention_launch_noalloc(const SasAttnArgs* args, void* stream);

/* Quantize-on-append into a SAS_KV_FP8_DS_MLA cache (no reference counterpart: the
 * reference has no fp8 cache; this is the producer of the format above).
 * src: [n, 576] bf16 rows (device); slot_mapping: [n] int32 flat row index into the pool
 * (block * block_size + offset; a negative entry skips that row); cache: [cache_rows, 656]
 * bytes (device). Per row and 128-dim block t: amax = max |x|, scale = amax / 448 in fp32
 * (1 when amax is 0), e4m3[d] = rne_e4m3(clamp(x[d] / scale, -448, 448)) with an IEEE fp32
 * division; the rope dims are copied. Rows with a non-finite value give unspecified bytes.
 * Slots outside [0, cache_rows) are skipped. Asynchronous on `stream`; returns
 * SAS_E_INVALID for a null pointer or n < 0. */
int sas_kv_fp8_append(const void* src, const int32_t* slot_mapping, void* cache, int n,
                      int64_t cache_rows, void* stream);

/* Library version (major * 100 + minor). */
int sas_version(void);

/* sizeof(SasAttnArgs) as compiled into the library (binding layout check). */
int sas_args_struct_size(void);

/* Message for the last failing call on this thread ("" if none). */
const char* sas_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* SAS_MI355X_H_ */
