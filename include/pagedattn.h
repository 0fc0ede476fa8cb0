/*
 * pagedattn.h -- C ABI of the MI355X (gfx950) paged-KV grouped-query decode
 * attention library `libpagedattn_hip.so`.
 *
 * The reference project has no native ABI: its host wrapper launches two
 * Triton kernels directly. Each entry point below replaces one of those
 * launches (citations are into ParamThakkar123/paged-decode-attention):
 *
 *   pa_decode        <- `_paged_decode_kernel[grid](...)` and, when
 *                       num_splits > 1, the `_split_reduce_kernel[grid](...)`
 *                       launch that follows it
 *                       (pagedattn/triton_decode.py:331-376)
 *   pa_split_reduce  <- `_split_reduce_kernel[(b, hq)](...)` on its own
 *                       (pagedattn/triton_decode.py:198-240, 368-376)
 *   pa_cache_write   <- the KV write before the decode,
 *                       `reshape_and_cache_flash` (integration/vllm_backend.py:
 *                       117-122), with the reference's quantisation
 *                       (pagedattn/cache.py:33-48)
 *
 * Everything is plain C: device pointers, sizes, element strides and enums.
 * No function throws; each returns PA_OK (0) or a negative PA_ERR_* code and
 * records a message readable through pa_last_error() on the same thread.
 * Arguments are validated before any HIP call, so validation is testable on
 * a machine without a GPU. Launches are asynchronous on the stream passed in
 * (a hipStream_t, passed as void*; NULL means the legacy default stream).
 * The library allocates no device memory: the caller owns every buffer,
 * including the split-KV workspace (part_out / part_lse), except that
 * pa_decode_noalloc keeps its partials in a static device array that loads
 * with the library's code object.
 *
 * Tensor layouts (element strides; the innermost dimension is contiguous):
 *   q          [batch, num_q_heads, head_dim]                  fp16 | bf16
 *   k_cache    [num_blocks, block_size, num_kv_heads, head_dim] fp16 | fp8_e5m2 | int8 | bf16
 *   v_cache    same shape and strides as k_cache
 *   k_scale    [num_blocks, block_size, num_kv_heads]           fp16 | fp32 (int8 only)
 *   v_scale    same shape and strides as k_scale
 *   out        [batch, num_q_heads, head_dim]                  fp16 | bf16 (= q's)
 *   part_out   [batch, num_q_heads, num_splits, head_dim]      fp32
 *   part_lse   [batch, num_q_heads, num_splits]                fp32, log2 domain
 *   block_table[batch, max_blocks]                             int32
 *   seq_lens   [batch]                                         int32
 *
 * Size limits (PA_ERR_UNSUPPORTED beyond them): block_size a power of two in
 * [16, 256]; max_blocks * block_size < 2^31 tokens; batch * stride_btb < 2^31
 * block-table entries; one page
 * (block_size * stride_kt) under 2 GiB and the page stride (stride_kn) under
 * 4 GiB in bytes, likewise 2 GiB / 4 GiB for the int8 scale pages; the kv-head
 * stride under 2 GiB in bytes; the q, out and workspace strides under 2^31
 * elements; the pool itself (num_blocks pages) may be any size. q, out,
 * k_cache, v_cache and their strides are 16-byte aligned (PA_ERR_INVALID
 * otherwise).
 */
#ifndef PAGEDATTN_H_
#define PAGEDATTN_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PA_ABI_VERSION 8

/* Return codes. */
#define PA_OK 0
#define PA_ERR_INVALID (-1)     /* bad pointer, size, stride or enum */
#define PA_ERR_UNSUPPORTED (-2) /* valid but not built (e.g. head_dim 96) */
#define PA_ERR_HIP (-3)         /* a HIP runtime call failed */

/* KV cache element type: the reference's `_KV_CODE`
 * (pagedattn/triton_decode.py:30) with fp16 = 0, fp8_e5m2 = 1, int8 = 2. */
#define PA_KV_FP16 0
#define PA_KV_FP8_E5M2 1 /* OCP e5m2 (torch.float8_e5m2), not the FNUZ variant */
#define PA_KV_INT8 2
/* bf16 rows, converted in registers to fp16 (round to nearest even) before
 * the fp16 arithmetic: the reference maps bf16 to its fp16 path
 * (`_KV_CODE["bf16"] = 0`, `k.to(tl.float16)`, pagedattn/triton_decode.py:30,
 * 151-153; dequantize_kv, pagedattn/cache.py:55-56). */
#define PA_KV_BF16 3

/* Per-(token, kv_head) dequantization scale type (int8 KV only). */
#define PA_SCALE_NONE 0
#define PA_SCALE_FP16 1 /* the reference's choice (pagedattn/cache.py:45) */
#define PA_SCALE_FP32 2

/* q / out element type. bf16 q is converted to fp16 (exact for normal
 * values), bf16 out is rounded to nearest even from fp32. */
#define PA_IO_FP16 0
#define PA_IO_BF16 1

/* Largest supported split count, flat split count and GQA group handled in
 * one pass. */
#define PA_MAX_SPLITS 4096
#define PA_MAX_FLAT_SPLITS 65536
#define PA_MAX_FLAT_SEQ_COST 64
#define PA_MAX_GROUP 16
/* Entries of the host-built launch tables (see seq_lens_host). */
#define PA_HOST_TABLE_MAX 256

typedef struct pa_decode_args {
  /* device pointers */
  const void *q;
  const void *k_cache;
  const void *v_cache;
  const void *k_scale; /* int8 only; NULL otherwise */
  const void *v_scale; /* int8 only; NULL otherwise */
  void *out;
  float *part_out; /* num_splits > 1 only; NULL otherwise */
  float *part_lse; /* num_splits > 1 only; NULL otherwise */
  const int32_t *block_table;
  const int32_t *seq_lens;
  /* sizes */
  int32_t batch;
  int32_t num_q_heads;
  int32_t num_kv_heads;
  int32_t head_dim;   /* 32, 64, 128 or 256 */
  int32_t block_size; /* page size in tokens: 16, 32, 64, 128 or 256 */
  int32_t num_blocks; /* pool size; block-table entries are clamped into it */
  int32_t max_blocks; /* block_table row length */
  int32_t num_splits; /* >= 1; > 1 selects the split-KV two-pass path */
  /* Split chunking. 0: each sequence's range is cut into num_splits chunks of
   * ceil(ceil(T_b/32)/num_splits)*32 tokens (the reference's per-sequence
   * formula, pagedattn/triton_decode.py:78-85, with a 32-token unit).
   * > 0: every sequence uses the chunk of a sequence of max_seq_len tokens,
   * so a ragged batch's long sequences get all splits and short ones few
   * (balanced work per workgroup); a sequence longer than max_seq_len falls
   * back to its own per-sequence chunk, so no token is ever dropped. */
  int32_t max_seq_len;
  /* element strides */
  int64_t stride_qb, stride_qh;
  int64_t stride_kn, stride_kt, stride_kh; /* shared by k_cache and v_cache */
  int64_t stride_sn, stride_st;            /* shared by k_scale and v_scale */
  int64_t stride_ob, stride_oh;
  int64_t stride_pb, stride_ph, stride_ps; /* part_out */
  int64_t stride_lb, stride_lh;            /* part_lse */
  int64_t stride_btb;
  /* types and scalars */
  int32_t kv_dtype;    /* PA_KV_* */
  int32_t scale_dtype; /* PA_SCALE_* */
  int32_t io_dtype;    /* PA_IO_* */
  float sm_scale;      /* softmax scale applied to q.k (natural-log domain) */
  /* Flat (work-balanced) split, an addition with no counterpart in the
   * reference. 0: off (num_splits decides). F > 0: per (kv head, 16-head
   * tile), the batch's 32-token tiles are concatenated in sequence order and
   * cut into F equal contiguous ranges, one wave each, so every wave streams
   * the same number of tiles however ragged seq_lens is; num_splits and
   * max_seq_len are ignored. Workspace: part_out [batch + F, num_q_heads,
   * head_dim] with stride_pb / stride_ph (slot, head) and part_lse
   * [batch + F, num_q_heads] with stride_lb / stride_lh; stride_ps is unused.
   * Every wave scans seq_lens once (batch / 64 loads per lane). */
  int32_t flat_splits;
  /* Flat split only (also an addition): tiles of weight charged to each
   * non-empty sequence when the ranges are cut, 0 .. PA_MAX_FLAT_SEQ_COST.
   * 0: equal tile counts. c > 0: sequence b weighs c + ceil(T_b / 32) and the
   * ranges take equal weight, so a range that starts several sequences
   * (each start costs a wave about one tile of time) holds fewer tiles;
   * suits ragged batches. pa_flat_merge must be given the same value. */
  int32_t flat_seq_cost;
  /* Flat split only (also an addition): the lengths in host memory, NULL
   * when the caller has none. Given, they must equal seq_lens. The library
   * then computes the ranges and the merge's list of cut and empty
   * sequences on the host and passes them in the kernel arguments, so no
   * wave reads seq_lens before its first K/V loads and the merge covers only
   * the sequences that need it (and is not launched when none do). Launches
   * beyond PA_HOST_TABLE_MAX ranges or merge entries, a batch above 4096 or
   * sequences of 2^25 tokens and more use the GPU scan as without them.
   * Read during the call only. Ignored while the stream is being captured
   * into a HIP graph: tables in a graph's kernel arguments would be replayed
   * with whatever lengths seq_lens then holds, so captured launches scan. */
  const int32_t *seq_lens_host;
} pa_decode_args;

typedef struct pa_reduce_args {
  const float *part_out; /* [batch, num_heads, num_splits, head_dim] */
  const float *part_lse; /* [batch, num_heads, num_splits], log2 domain */
  void *out;             /* [batch, num_heads, head_dim] */
  int32_t batch;
  int32_t num_heads;
  int32_t head_dim;
  int32_t num_splits;
  int64_t stride_pb, stride_ph, stride_ps;
  int64_t stride_lb, stride_lh;
  int64_t stride_ob, stride_oh;
  int32_t io_dtype; /* PA_IO_* */
} pa_reduce_args;

/* Paged GQA decode attention for one query token per sequence.
 * out[b, h, :] = softmax(sm_scale * q[b, h] . K[b, h / group, 0:T_b]) V[...]
 * with T_b = seq_lens[b] and group = num_q_heads / num_kv_heads.
 * num_splits == 1: one kernel writes `out` directly.
 * num_splits  > 1: the decode kernel writes per-split partials (normalised
 * output and log2-sum-exp) into part_out / part_lse, then the reduce kernel
 * merges them into `out`. Only splits that hold tokens do work: a sequence
 * that fits in one split is written to `out` by the decode kernel and skipped
 * by the merge, and the merge reads a sequence's non-empty splits only. (So
 * part_out / part_lse are scratch here; pa_decode_partials fills them all.)
 * flat_splits > 0: the flat decode kernel writes a sequence held by one
 * wave range to `out` and the others as partial slots, then the merge
 * kernel folds each sequence's slots (see pa_decode_args.flat_splits).
 * A sequence with T_b == 0 yields zeros (the reference yields NaN there).
 * Replaces pagedattn/triton_decode.py:331-376. */
int pa_decode(const pa_decode_args *args, void *stream);

/* Decode pass only: writes part_out / part_lse (num_splits >= 1) and skips
 * the merge, so a caller can time or distribute the passes separately.
 * With flat_splits > 0 it is the flat decode pass alone: partial slots, and
 * `out` for the sequences that one range holds whole.
 * Replaces the `_paged_decode_kernel[(b, hkv, num_splits)]` launch
 * (pagedattn/triton_decode.py:351-367). */
int pa_decode_partials(const pa_decode_args *args, void *stream);

/* Merge of split partials: out = sum_s part_s * 2^(lse_s - m) /
 * sum_s 2^(lse_s - m), m = max_s lse_s; all-empty rows yield zeros.
 * Replaces pagedattn/triton_decode.py:198-240 / 368-376. */
int pa_split_reduce(const pa_reduce_args *args, void *stream);

/* Arguments of pa_cache_write: this step's K/V rows into the paged cache. */
typedef struct pa_cache_write_args {
  const void *key;   /* [num_tokens, num_kv_heads, head_dim] fp16 (bf16 for a bf16 cache), head_dim contiguous */
  const void *value; /* same shape */
  void *k_cache;     /* [num_blocks, block_size, num_kv_heads, head_dim] kv_dtype */
  void *v_cache;     /* same shape and strides as k_cache */
  void *k_scale;     /* [num_blocks, block_size, num_kv_heads] (int8 only; NULL otherwise) */
  void *v_scale;     /* same shape and strides as k_scale */
  const int64_t *slot_mapping; /* [num_tokens]: block * block_size + offset; < 0 skips */
  int32_t num_tokens;
  int32_t num_kv_heads;
  int32_t head_dim;   /* 32, 64, 128 or 256 */
  int32_t block_size; /* >= 1 */
  int32_t num_blocks; /* slots at or past num_blocks * block_size are skipped */
  int64_t stride_kt, stride_kh; /* key element strides (token, head) */
  int64_t stride_vt, stride_vh; /* value element strides (token, head) */
  int64_t stride_cn, stride_ct, stride_ch; /* cache element strides, shared by k/v */
  int64_t stride_sn, stride_st;            /* scale element strides, shared by k/v */
  int32_t kv_dtype;    /* PA_KV_* */
  int32_t scale_dtype; /* PA_SCALE_* (int8: FP16 or FP32) */
} pa_cache_write_args;

/* Scatter this step's K and V rows (fp16) into the paged NHD cache at
 * slot_mapping, quantising as the cache dtype requires, with the reference's
 * semantics (pagedattn/cache.py:33-48): fp16 copies; fp8_e5m2 is the
 * round-to-nearest-even cast (overflow to inf, as torch's); int8 takes one
 * scale per (token, head): amax over head_dim clamped to 1e-6, scale =
 * amax / 127 rounded to the scale type, q = round_half_even(x / scale)
 * clamped to +-127, and writes the scale. Bit-identical to
 * pagedattn.cache.quantize_kv. Replaces the call to vLLM's
 * `reshape_and_cache_flash` at integration/vllm_backend.py:117-122 for
 * caches in this library's formats. */
int pa_cache_write(const pa_cache_write_args *args, void *stream);

/* The flat split's merge pass alone (flat_splits > 0): folds the partial
 * slots that pa_decode_partials with the same arguments wrote into `out`
 * (sequences that one range held whole are already there; empty sequences
 * get zeros). pa_decode_partials + pa_flat_merge == pa_decode. The
 * counterpart of the reference's `_split_reduce_kernel` launch
 * (pagedattn/triton_decode.py:368-376) for the flat split. */
int pa_flat_merge(const pa_decode_args *args, void *stream);

/* Waves of the flat decode kernel for (kv_dtype, scale_dtype, head_dim)
 * that one SIMD holds at once (hipOccupancyMaxActiveBlocksPerMultiprocessor
 * on the current device, times the kernel's workgroup width, over the 4
 * SIMDs of a CU), written to *out. A host planner sizes flat_splits from
 * it: one round of waves is CUs * 4 * min(*out, 2) waves over
 * num_kv_heads * ceil(group / 16) units. No counterpart in the reference
 * (its split count comes from the SM count alone,
 * pagedattn/triton_decode.py:248-263). */
int pa_flat_waves_per_simd(int kv_dtype, int scale_dtype, int head_dim, int *out);

/* Bytes of the static device scratch behind pa_decode_noalloc (per GPU). */
#define PA_NOALLOC_SCRATCH_BYTES (32 << 20)

/* pa_decode without a caller workspace, allocating nothing: no hipMalloc,
 * no allocator call, for callers that cannot allocate (code under HIP graph
 * capture, serving loops or harnesses that forbid allocation). The split
 * partials go to a static device array of PA_NOALLOC_SCRATCH_BYTES inside
 * the library, one per GPU, held until the process ends; its address is
 * looked up once per device (hipGetSymbolAddress) on the first call there.
 * part_out, part_lse and their strides in *args are ignored; everything
 * else means what it means for pa_decode, and the results are pa_decode's.
 * A launch whose partials need more than PA_NOALLOC_SCRATCH_BYTES
 * (split: batch * num_splits, flat: batch + flat_splits slots of
 * num_q_heads * (head_dim + 1) floats) returns PA_ERR_UNSUPPORTED. Every
 * call on one GPU shares that GPU's array, so calls that overlap on one GPU
 * (two streams, two threads) race: the caller serialises them. The first
 * call on a device looks up the array's address there (the runtime may load
 * the code object then), so make one call on each device before capturing
 * calls into a HIP graph; later calls, captured or not, make no runtime call
 * besides the launches. No counterpart in the reference; it is for callers
 * that cannot allocate. */
int pa_decode_noalloc(const pa_decode_args *args, void *stream);

/* The launch tables pa_decode builds from seq_lens_host for a flat split
 * (flat_splits > 0, seq_lens_host set; the other fields as for pa_decode),
 * computed on the host without any HIP call, complete whatever their size:
 * ranges[3 j .. 3 j + 2] = range j's first sequence, its first 32-token tile
 * there and its tile count (all zero for a range without tiles);
 * items[3 i .. 3 i + 2] = the i-th sequence the merge writes (cut by a range
 * boundary, or empty), its first partial slot and its slot count (0: empty,
 * zeros; up to flat_splits), *n_items of them. ranges holds 3 * flat_splits
 * and items 3 * batch int32s. *in_kernel_args (if not NULL) gets
 * PA_HOST_PLAN_RANGES when pa_decode passes the ranges to the decode kernel
 * (at most PA_HOST_TABLE_MAX ranges, a batch up to 4096, block-table rows
 * of fewer than 2^25 tokens) and PA_HOST_PLAN_MERGE when it passes the merge list to the
 * merge (at most PA_HOST_TABLE_MAX items); a pass without its table scans
 * seq_lens on the GPU instead. No counterpart in the reference; for planners
 * and tests. */
#define PA_HOST_PLAN_RANGES 1
#define PA_HOST_PLAN_MERGE 2
int pa_flat_host_plan(const pa_decode_args *args, int32_t *ranges, int32_t *items, int32_t *n_items,
                      int32_t *in_kernel_args);

/* Message for the last non-zero return on the calling thread ("" if none). */
const char *pa_last_error(void);

/* PA_ABI_VERSION of the built library. */
int pa_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* PAGEDATTN_H_ */
