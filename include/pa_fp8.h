/*
 * pa_fp8.h -- C ABI of libpa_fp8.so, the gfx950 (MI355X) FP8-KV paged-attention
 * decode library.
 *
 * Every entry point takes plain pointers and sizes, launches on the caller's
 * HIP stream, never allocates, never synchronises and returns a status code
 * (PA_FP8_OK == 0).  Device pointers are HIP device addresses; strides are in
 * ELEMENTS of the tensor they describe.
 *
 * The reference reaches its kernels through MLIR-generated host stubs,
 * `_mlir_ciface_<launcher>(void **packed_args)`, that end in
 * `mgpuLaunchKernel` -> `hipModuleLaunchKernel`
 * (lib/Runtime/ROCm/FlyRocmRuntimeWrappers.cpp:58-62).  Each entry point below
 * replaces one such launcher; the citation on each names it.
 */
#ifndef PA_FP8_H
#define PA_FP8_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PA_FP8_ABI_VERSION 10

enum pa_fp8_status {
    PA_FP8_OK = 0,
    PA_FP8_ERR_NULL_POINTER = 1,     /* a required pointer is NULL            */
    PA_FP8_ERR_HEAD_DIM = 2,         /* head_dim unsupported by the entry     */
    PA_FP8_ERR_BLOCK_SIZE = 3,       /* block_size not a power of two >= 16   */
    PA_FP8_ERR_GROUP = 4,            /* query_length * group_size not in 1..65535 */
    PA_FP8_ERR_SHAPE = 5,            /* a size or stride out of range         */
    PA_FP8_ERR_DTYPE = 6,            /* unsupported query / output dtype      */
    PA_FP8_ERR_PARTITIONS = 7,       /* max_context_partition_num out of range */
    PA_FP8_ERR_WORKLIST = 8,         /* metadata buffer too small             */
    PA_FP8_ERR_LAYOUT = 9,           /* cache layout / format not valid here  */
    PA_FP8_ERR_SCRATCH = 10,         /* partials exceed the static scratch    */
    PA_FP8_ERR_HIP = 1000            /* 1000 + hipError_t of a failed launch  */
};

/* element types of query / output tensors */
enum pa_fp8_dtype { PA_FP8_BF16 = 0, PA_FP8_F16 = 1, PA_FP8_F32 = 2 };

/* value-cache layouts the decode reads (kernels/pa_decode_fp8.py:2841, trans_v = V.ndim == 5) */
enum pa_fp8_value_layout {
    PA_FP8_V_TRANS = 0,  /* [nb, Hkv, bs/16, D, 16]: 16 consecutive tokens of a head dim in 16 bytes */
    PA_FP8_V_4D = 1      /* [nb, Hkv, D, bs]: every token of a head dim contiguous                    */
};

/*
 * Split-context decode: one workgroup per (sequence, kv head, partition slot).
 * Writes the per-slot partials the LSE reduce consumes:
 *   exp_sums / max_logits  f32  [B, Hkv, P, ql*g]   (sum of exp(logit - max), natural-log max)
 *   tmp_out                bf16 [B, Hkv, P, ql*g, D] (output normalised by its own exp sum)
 * Empty slots write (0, -inf, 0).
 * Slot z covers 256-token partitions [z*pps, min((z+1)*pps, T)), T = ceil(ctx/256),
 * pps = ceil(T/P) (kernels/pa_decode_fp8.py:2311-2320).  With sliding_window > 0
 * the partitions start at tile max(ctx-ql-sw, 0)/256 (kernels/pa_decode_swa.py:1359-1368).
 *
 * Inputs:
 *   query          [B*ql, Hq, D] bf16 or f16 (query_dtype), D = head_dim in {64, 128, 192, 256}
 *   key_cache      [nb, Hkv, D/16, bs, 16] fp8 e4m3fn
 *   value_cache    [nb, Hkv, bs/16, D, 16] (value_layout PA_FP8_V_TRANS) or
 *                  [nb, Hkv, D, bs] (PA_FP8_V_4D) fp8 e4m3fn
 *   block_tables   [B, max_blocks] int32; context_lengths [B] int32
 *   key_scale / value_scale: per-tensor [1] f32, or per-token [nb, Hkv, bs, 1] f32
 *   (per_token_kv = 1, element = blk*stride_ks_block + h*stride_ks_head + slot)
 *
 * A workgroup holds up to 64 of the ql*g query rows of a (sequence, kv head); more
 * rows (e.g. GQA 16 x ql 8) run as chunks of 64 in adjacent workgroups.
 *
 * Replaces the launcher of `compile_pa_decode_ps` (kernels/pa_decode_fp8.py:2739-2803,
 * called at :3061-3093) and of `compile_pa_decode_sw` (kernels/pa_decode_swa.py:1195-1724,
 * called at kernels/pa_decode_fp8.py:2937-2974).
 */
typedef struct pa_fp8_decode_args {
    float *exp_sums;
    float *max_logits;
    void *tmp_out;
    const void *query;
    const uint8_t *key_cache;
    const uint8_t *value_cache;
    const int32_t *block_tables;
    const int32_t *context_lengths;
    const float *key_scale;
    const float *value_scale;
    int64_t stride_q_seq, stride_q_head;
    int64_t stride_k_block, stride_k_head;
    int64_t stride_v_block, stride_v_head;
    int64_t stride_es_seq, stride_es_head, stride_es_part;
    int64_t stride_to_seq, stride_to_head, stride_to_part, stride_to_group;
    int64_t stride_bt_seq;
    int64_t stride_ks_block, stride_ks_head;
    int32_t batch_size;
    int32_t num_kv_heads;
    int32_t query_group_size;
    int32_t query_length;
    int32_t head_dim;
    int32_t block_size;
    int32_t num_blocks;          /* physical blocks in the caches (entries are clamped into range) */
    int32_t max_blocks_per_seq;  /* block_tables.shape[1] */
    int32_t max_context_partition_num;
    int32_t sliding_window;      /* 0 = off */
    int32_t per_token_kv;        /* 0 = per-tensor scales, 1 = per-token */
    int32_t query_dtype;         /* PA_FP8_BF16 or PA_FP8_F16 */
    float softmax_scale;
    /* direct_output = 1: the kernel writes the final rows to output[b, qi, h, gi, :]
     * (5-D view [B, ql, Hkv, g, D], dtype out_dtype) as pa_fp8_lse_reduce would.
     * With max_context_partition_num == 1 each workgroup holds the whole sequence
     * and exp_sums / max_logits / tmp_out are not used.  With more slots it needs
     * the chained layout below with waves_per_slot * slots_per_wave >= the slot
     * count (one workgroup per sequence and kv head): the workgroup writes every
     * slot's partial, then merges them into the output with pa_fp8_lse_reduce's
     * arithmetic (the same bits), so no reduce launch follows. */
    int32_t direct_output;
    int32_t out_dtype;
    void *output;
    int64_t stride_o_seq, stride_o_len, stride_o_head, stride_o_group;
    /* waves per workgroup when ql * query_group_size <= 16: 0 = 4, or 1, 2, 4, 8.
     * With slots_per_wave == 0 the waves split one slot's steps (eight suit grids of
     * at most one workgroup per CU; head dims other than 128 always run four);
     * with slots_per_wave > 0 each wave runs its own chain of slots. */
    int32_t waves_per_slot;
    int32_t value_layout;        /* pa_fp8_value_layout */
    /* 0: one slot per workgroup.  slots_per_wave > 0 (only with
     * ql * query_group_size <= 16, head_dim 128 and the trans_v layout): the chained
     * layout -- wave w of workgroup (b, h, zc) runs the slots
     * [(zc * W + w) * slots_per_wave, (zc * W + w + 1) * slots_per_wave) of its
     * (sequence, kv head) in turn (W = waves_per_slot, 0 meaning 1), its K / V loads
     * running on across slot boundaries, and writes each slot's partial as that slot
     * ends; the grid's third dimension is ceil(max_context_partition_num /
     * (W * slots_per_wave)).  A slot's partial is the same whichever layout runs
     * with one wave per slot. */
    int32_t slots_per_wave;
} pa_fp8_decode_args;

int pa_fp8_decode_partitions(const pa_fp8_decode_args *args, void *hip_stream);

/* Bytes of the static device scratch pa_fp8_decode_partitions_noalloc keeps its
 * partials in (32 MiB on every GPU the library runs on, held until the process ends). */
#define PA_FP8_NOALLOC_SCRATCH_BYTES (32 << 20)

/*
 * The split-context decode and its log-sum-exp reduce in one call that allocates
 * nothing: pa_fp8_decode_partitions followed by pa_fp8_lse_reduce into `output`
 * (out_dtype, stride_o_*), with the partials (exp_sums, max_logits, tmp_out) in a
 * static device array of PA_FP8_NOALLOC_SCRATCH_BYTES instead of caller buffers;
 * args->exp_sums / max_logits / tmp_out and their strides are ignored.  With
 * max_context_partition_num == 1 it is the direct-output decode (no scratch).
 * The partials need B * Hkv * P * ql*g * (8 + 2 * head_dim) bytes (each piece
 * rounded up to 256); more returns PA_FP8_ERR_SCRATCH.  Outputs are bit-identical
 * to the two-call path.  The scratch is looked up (hipGetSymbolAddress) on the
 * first call on each device and never allocated or freed; make that first call
 * before capturing the entry point into a HIP graph.  Every call on a GPU
 * shares that GPU's one scratch: calls that overlap on one GPU (several streams,
 * or host threads, at once) race; calls ordered on one stream do not.
 *
 * No counterpart in the reference.  It is for callers that cannot allocate:
 * code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.
 */
int pa_fp8_decode_partitions_noalloc(const pa_fp8_decode_args *args, void *hip_stream);

/*
 * Log-sum-exp reduce of the partials into the final output
 *   out[b, qi, h, gi, d] = sum_z w_z * tmp_out[b, h, z, qi*g+gi, d],
 *   w_z = s_z e^(m_z - M) / sum_z s_z e^(m_z - M),  M = max_z m_z
 * Output dtype bf16 / f16 / f32 (out_dtype); strides describe the 5-D view
 * [B, ql, Hkv, g, D] of the [B*ql, Hq, D] output; head_dim even, at most 256.
 *
 * Replaces the launcher of `compile_pa_decode_sw_reduce`
 * (kernels/pa_decode_swa.py:1132-1183, called at kernels/pa_decode_fp8.py:3094-3120).
 */
typedef struct pa_fp8_reduce_args {
    void *output;
    const float *exp_sums;
    const float *max_logits;
    const void *tmp_out;
    int64_t stride_o_seq, stride_o_len, stride_o_head, stride_o_group;
    int64_t stride_es_seq, stride_es_head, stride_es_part;
    int64_t stride_to_seq, stride_to_head, stride_to_part, stride_to_group;
    int32_t batch_size;
    int32_t num_kv_heads;
    int32_t query_group_size;
    int32_t query_length;
    int32_t head_dim;
    int32_t max_context_partition_num;
    int32_t out_dtype;           /* PA_FP8_BF16, PA_FP8_F16 or PA_FP8_F32 */
    int32_t reserved;
} pa_fp8_reduce_args;

int pa_fp8_lse_reduce(const pa_fp8_reduce_args *args, void *hip_stream);

/*
 * Persistent worklist decode: workgroup c (grid = num_cu) runs the works
 * [work_indptr[c], work_indptr[c+1]) of the get_pa_metadata_v1 schedule.  Work w
 * is work_info[w] = {batch, partial_qo_loc, qo_start, qo_end, kv_start, kv_end, 0,
 * (qh_end << 16) | qh_start}; kv_start / kv_end are cumulative 256-token partition
 * indices (sequence b's partitions start at partition_indptr[b]) and the kv head
 * is qh_start / query_group_size.  A work attends its partitions' keys under the
 * causal bound tok < ctx + 1 - ql + qi, reading sequence b's pages from
 * kv_page_indices[kv_indptr[b] .. kv_indptr[b+1]).
 *   partial_qo_loc <  0: the normalised rows go to output[qo_start + qi, qhead, :]
 *                        (dtype out_dtype);
 *   partial_qo_loc >= 0: f32 normalised rows go to
 *                        partial_output[(partial_qo_loc + ql + qi) * stride_po_row + qhead * D + d]
 *                        and the row's log-sum-exp (natural log; -inf when nothing is
 *                        visible) to partial_lse[(partial_qo_loc + ql + qi) * stride_pl_row + qhead].
 * Works whose batch, head or partial row fall outside the given sizes are skipped.
 * Q rows are batch * ql + qi.  Caches, scales, query, head dims, value layouts
 * and row chunks as for pa_fp8_decode_partitions (any power-of-two block size >= 16);
 * with more than 64 rows the grid is num_cu * chunks.
 *
 * Replaces the launcher of `compile_pa_decode_metadata`
 * (kernels/pa_decode_fp8.py:941-1721, called at :3155-3187).
 */
typedef struct pa_fp8_worklist_args {
    void *output;
    float *partial_output;
    float *partial_lse;
    const void *query;
    const uint8_t *key_cache;
    const uint8_t *value_cache;
    const int32_t *context_lengths;
    const float *key_scale;
    const float *value_scale;
    const int32_t *work_indptr;      /* [num_cu + 1] */
    const int32_t *work_info;        /* [max_work, 8] */
    const int32_t *kv_page_indices;  /* flat pages of every sequence */
    const int32_t *kv_indptr;        /* [B + 1] */
    const int32_t *partition_indptr; /* [B + 1] cumulative ceil(ctx / 256) */
    int64_t stride_q_seq, stride_q_head;
    int64_t stride_k_block, stride_k_head;
    int64_t stride_v_block, stride_v_head;
    int64_t stride_out_seq, stride_out_head;
    int64_t stride_po_row, stride_pl_row;
    int64_t stride_ks_block, stride_ks_head;
    int32_t batch_size;
    int32_t num_kv_heads;
    int32_t query_group_size;
    int32_t query_length;
    int32_t head_dim;
    int32_t block_size;
    int32_t num_blocks;          /* physical blocks in the caches (page entries are clamped into range) */
    int32_t num_pages;           /* entries of kv_page_indices */
    int32_t num_cu;              /* workgroups = work_indptr entries - 1 */
    int32_t max_work;            /* rows of work_info */
    int32_t partial_rows;        /* rows of partial_output / partial_lse */
    int32_t output_rows;         /* rows of output (B * ql) */
    int32_t per_token_kv;
    int32_t query_dtype;
    int32_t out_dtype;
    float softmax_scale;
    /* bin_groups = G > 1 (with num_cu a multiple of G * num_kv_heads): workgroup c
     * runs bin k*nspk + a*(nspk/G) + j instead of bin c, where a = c / (num_cu/G) is
     * the workgroup's dispatch round (the order in which it joined its CU, when the
     * device takes num_cu/G workgroups per round) and c % (num_cu/G) = k*(nspk/G) + j,
     * nspk = num_cu / num_kv_heads.  So bin group a of every head (see
     * pa_fp8_metadata_args.bin_weight) runs on the workgroups of round a.  Any
     * permutation of the bins gives the same outputs.  Not applied with row chunks. */
    int32_t bin_groups;
    int32_t value_layout;        /* pa_fp8_value_layout */
} pa_fp8_worklist_args;

int pa_fp8_decode_worklist(const pa_fp8_worklist_args *args, void *hip_stream);

/*
 * Merge of split works' partials (the role of aiter's pa_reduce_v1, called at
 * kernels/pa_decode_fp8.py:3189-3200).  For every reduce group g with
 * reduce_indptr[g] < reduce_indptr[g+1], qo range reduce_final_map[g] = {qo_start, qo_end},
 * query row qi < min(qo_end - qo_start, max_qlen) and head h < num_heads:
 *   rows s_j = reduce_partial_map[j] + qi, j in [reduce_indptr[g], reduce_indptr[g+1])
 *   LSE = log sum_j exp(partial_lse[s_j, h]),  w_j = exp(partial_lse[s_j, h] - LSE)
 *   output[qo_start + qi, h, :] = sum_j w_j * partial_output[s_j, h, :]
 *   final_lse[qo_start + qi, h] = LSE (when final_lse is not NULL)
 * A row whose partials are all -inf gets 0 (and LSE -inf).  partial_output /
 * partial_lse point at the row the map's 0 refers to (the launcher passes
 * partial_output[query_length:]).  head_dim even, at most 256.
 */
typedef struct pa_fp8_reduce_v1_args {
    void *output;
    float *final_lse;
    const float *partial_output;
    const float *partial_lse;
    const int32_t *reduce_indptr;       /* [num_groups + 1] */
    const int32_t *reduce_final_map;    /* [num_groups, 2] */
    const int32_t *reduce_partial_map;  /* [partial_map_len] */
    int64_t stride_po_row, stride_po_head;
    int64_t stride_pl_row, stride_pl_head;
    int64_t stride_out_row, stride_out_head;
    int64_t stride_lse_row, stride_lse_head;
    int32_t num_groups;
    int32_t num_heads;
    int32_t head_dim;
    int32_t max_qlen;
    int32_t partial_rows;        /* rows reachable from partial_output */
    int32_t output_rows;
    int32_t partial_map_len;
    int32_t out_dtype;
} pa_fp8_reduce_v1_args;

int pa_fp8_reduce_v1(const pa_fp8_reduce_v1_args *args, void *hip_stream);

/*
 * get_pa_metadata_v1 worklist scheduler on the device (the reference runs its
 * state machine serially on one wave; here a parallel closed form covers the
 * common case and the serial machine the rest).  Writes work_indptr
 * [num_cu+1], work_info [max_work, 8], reduce_indptr [B+1],
 * reduce_final_map [B, 2], reduce_partial_map [max_split_tiles]; only the
 * valid prefixes are defined, and a buffer of no entries may be NULL (one bin
 * per kv head gives max_split_tiles 0).  kv_granularity must be a power of two and
 * num_cu a multiple of num_heads_k.  Optional outputs (NULL: not written):
 * partition_indptr [B+1], the exclusive prefix of ceil(context_len /
 * kv_granularity), and uniform_context [1], 1 when every context length is
 * equal (get_pa_metadata's two derived values, so it needs no other launches).
 * bin_groups = G > 1 (get_pa_metadata's option; 0 gives the reference's
 * schedule): the bins of each kv head form G equal groups and the parallel
 * scheduler splits the partitions in proportion to bin_weight[g] (1..1000) of
 * each bin's group instead of evenly, when every bin still gets a partition
 * (sum of partitions S >= 4 * bins per head, S * least weight >= 2 * Wt with Wt
 * the sum of every bin's weight, at most 4096 bins per head) and the context
 * lengths are not all equal (equal sequences fill equal bins whole; weights would
 * split them).  Workgroups that share a CU progress
 * at different rates (issue arbitration favours the one dispatched first), and
 * pa_fp8_decode_worklist with the same bin_groups runs group a on the
 * workgroups of dispatch round a.
 *
 * Replaces the launcher of `compile_pa_metadata_v1` (kernels/pa_metadata.py:422-447,
 * called from get_pa_metadata_v1 at :515-524).
 */
typedef struct pa_fp8_metadata_args {
    const int32_t *seqlens_qo_indptr;  /* [B+1]; NULL: b * query_length (a decode step) */
    const int32_t *context_lens;
    int32_t *work_indptr;
    int32_t *work_info;
    int32_t *reduce_indptr;
    int32_t *reduce_final_map;
    int32_t *reduce_partial_map;
    int32_t num_batches;
    int32_t gqa;
    int32_t num_heads_k;
    int32_t num_cu;
    int32_t kv_granularity;
    int32_t query_length;
    int32_t max_work;
    int32_t max_split_tiles;
    int32_t *partition_indptr;
    int32_t *uniform_context;
    int32_t bin_groups;
    int32_t bin_weight[4];
    int32_t *partial_count;      /* optional [1]: reduce_indptr[num_batches], the split partials */
    /* 1: the packing schedule where it applies (get_pa_metadata's tuned schedule;
     * 0 gives the sequential fill, as get_pa_metadata_v1 must).  With the same
     * quotas, sequences sorted by (partitions descending, batch) and bins by
     * (quota descending, bin): rank k < min(bins, B) places sequence k whole in
     * bin k, the remaining sequences are poured in rank order into the bins'
     * remaining room in bin-rank order (split at its boundaries; an empty one
     * becomes an empty work in the last bin with room), and split sequences form
     * the reduce groups in batch order.  It applies when every rank k < min(bins,
     * B) fits its bin, B <= 2048, bins per head <= 2048, every quota is below
     * 2^19 partitions, the partitions total 1 .. 2^31 - 1 and no context length
     * is negative; otherwise the sequential fill runs.  Fewer split sequences than the sequential fill (c5: 964 split
     * works instead of 1488) and no sequence is cut at a bin boundary when it fits
     * a bin whole. */
    int32_t pack;
} pa_fp8_metadata_args;

int pa_fp8_metadata_v1(const pa_fp8_metadata_args *args, void *hip_stream);

/*
 * `count` (1..4) independent schedules in one launch: schedule i from args[i],
 * each exactly as pa_fp8_metadata_v1 computes it (one workgroup per schedule, so
 * they run side by side).  get_pa_metadata computes the reference's schedule and
 * its own tuned one this way.  No counterpart in the reference, which builds one
 * schedule per call (kernels/pa_metadata.py:450-524).
 */
int pa_fp8_metadata_multi(const pa_fp8_metadata_args *args, int32_t count, void *hip_stream);

/* KV-cache formats written by pa_fp8_rope_cache */
enum pa_fp8_cache_format {
    PA_FP8_CACHE_ELEM = 0,       /* cache of the element dtype (bf16 / f16), written unscaled   */
    PA_FP8_CACHE_FP8_TENSOR = 1, /* fp8 e4m3fn, code = e4m3(x * v_rcp_f32(scale[0])), scale read */
    PA_FP8_CACHE_FP8_TOKEN = 2   /* fp8 e4m3fn, scale = amax/448 per (token, kv head) written,
                                    code = e4m3(x / scale)                                     */
};

/* KV-cache layouts written by pa_fp8_rope_cache */
enum pa_fp8_kv_layout {
    PA_FP8_KV_FLASH = 0,    /* K, V [nb, bs, Hkv, D]                                */
    PA_FP8_KV_X_PACKED = 1, /* K [nb, Hkv, D/16, bs, 16], V [nb, Hkv, D, bs]        */
    PA_FP8_KV_X_TRANS = 2   /* K [nb, Hkv, D/16, bs, 16], V [nb, Hkv, bs/16, D, 16] */
};

/*
 * Fused NeoX rotary embedding + paged KV-cache write, one launch:
 *   query_out = rope(query), key_out = rope(key) for every token;
 *   for tokens whose slot >= 0 (and slot / block_size < num_blocks): the cache
 *   entry (slot / block_size, slot % block_size) of every kv head receives
 *   rope(key) and value in cache_format / kv_layout.
 * rope pairs head dim d with d + D/2 (NeoX, rotary_dim == D):
 *   out[d]       = r(r(x[d] * c) - r(x[d + D/2] * s))
 *   out[d + D/2] = r(r(x[d + D/2] * c') + r(x[d] * s'))
 * with r = rounding to the element dtype, (c, s) = cos/sin[pos, d] and
 * (c', s') = the same (reuse_freqs_front_part, cos/sin [max_pos, D/2]) or
 * cos/sin[pos, d + D/2] (cos/sin [max_pos, D]).
 * Positions and slots are int32, or int64 of which the low word is read;
 * positions outside [0, max_pos) are clamped into it.
 * query / key / value / outputs [T, H, D] with a free token and head stride
 * (inner dim contiguous, 16-byte aligned rows); cos / sin [max_pos, cols]
 * with a free row stride; caches contiguous inside a (block, head) tile with
 * free block and head strides (and token stride for the flash layout).
 * head_dim: a multiple of 16 in [16, 1024]; with PA_FP8_KV_FLASH also any even
 * head_dim in [2, 1024], read and written element by element (2-byte aligned
 * 16-bit tensors, any non-negative strides).
 * Per-token scales [nb, Hkv, bs, 1] f32: element blk*stride_ks_block +
 * h*stride_ks_head + slot % block_size.
 *
 * Replaces the launcher of `build_fused_rope_cache_module`
 * (kernels/fused_rope_cache_kernel.py:439-475, kernel :106-429).
 * PA_FP8_KV_X_TRANS and PA_FP8_CACHE_FP8_TOKEN have no counterpart there:
 * they write the V layout and the per-token scales pa_fp8_decode_* read.
 */
typedef struct pa_fp8_rope_cache_args {
    const void *query;
    const void *key;
    const void *value;
    const void *positions;
    const void *cos_cache;
    const void *sin_cache;
    const void *slot_mapping;
    void *key_cache;
    void *value_cache;
    void *query_out;
    void *key_out;
    float *key_scale;
    float *value_scale;
    int64_t stride_q_token, stride_q_head;
    int64_t stride_k_token, stride_k_head;
    int64_t stride_v_token, stride_v_head;
    int64_t stride_qo_token, stride_qo_head;
    int64_t stride_ko_token, stride_ko_head;
    int64_t stride_cos_pos, stride_sin_pos;
    int64_t stride_kc_block, stride_kc_head, stride_kc_token;
    int64_t stride_vc_block, stride_vc_head, stride_vc_token;
    int64_t stride_ks_block, stride_ks_head;
    int32_t num_tokens;
    int32_t num_q_heads;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t block_size;
    int32_t num_blocks;
    int32_t max_pos;
    int32_t elem_dtype;     /* PA_FP8_BF16 or PA_FP8_F16 (query, key, value, cos, sin, outputs) */
    int32_t cache_format;   /* pa_fp8_cache_format */
    int32_t kv_layout;      /* pa_fp8_kv_layout */
    int32_t reuse_freqs_front_part;
    int32_t positions_i64;
    int32_t slots_i64;
    int32_t reserved;
} pa_fp8_rope_cache_args;

int pa_fp8_rope_cache(const pa_fp8_rope_cache_args *args, void *hip_stream);

/*
 * y[i] = v_rcp_f32(x[i]) for i < n (device pointers, n >= 0): the hardware
 * reciprocal pa_fp8_rope_cache applies to per-tensor scales, as the reference
 * writer does (kernels/fused_rope_cache_kernel.py:282-283, `rocdl.rcp`).  It is
 * within 1 ulp of 1/x but not always the correctly rounded quotient, so the
 * cache codes of a scale depend on it; this entry exposes the value for
 * checkers that restate the writer.  No counterpart of its own in the reference.
 */
int pa_fp8_hw_reciprocal(const float *x, float *y, int64_t n, void *hip_stream);

/* Human-readable text of a status code (static storage). */
const char *pa_fp8_status_string(int status);

/* PA_FP8_ABI_VERSION of the built library. */
int pa_fp8_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* PA_FP8_H */
