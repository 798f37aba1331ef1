// Kernel parameters of the gfx950 paged-attention decode kernels, shared by the
// C ABI (pa_decode.hip) and the per-head-dim kernel objects (pa_decode_hd.hip,
// built once for each supported head_dim).
#pragma once

#include "pa_common.h"

namespace pa {

// Head dims the decode kernels are built for (multiples of 64, as the reference
// requires: kernels/pa_decode_fp8.py:969-970, :2084-2085).
constexpr int kHeadDims[] = {64, 128, 192, 256};
constexpr int kRowChunk = 64;  // query rows per kv head one workgroup holds (ql * g above it: chunks)

struct DecodeParams {
    float *exp_sums;
    float *max_logits;
    uint16_t *tmp_out;
    const uint16_t *query;
    const uint8_t *kc;
    const uint8_t *vc;
    const int32_t *bt;
    const int32_t *ctx;
    const float *ks;
    const float *vs;
    int64_t s_q_seq, s_q_head;
    int64_t s_k_block, s_k_head;
    int64_t s_v_block, s_v_head;
    int64_t s_es_seq, s_es_head, s_es_part;
    int64_t s_to_seq, s_to_head, s_to_part, s_to_group;
    int64_t s_bt_seq;
    int64_t s_ks_block, s_ks_head;
    int32_t g, ql, eqgs, bs_log2;
    int32_t num_blocks, max_blocks, max_parts, sw;
    int32_t q_f16;
    int32_t chunks;  // row chunks of kRowChunk rows per (sequence, kv head): workgroups per slot
    float qk_scale;  // softmax_scale * log2(e)
    // direct output (one partition slot): final rows go to out[b, qi, h, gi, :]
    void *out;
    int64_t s_o_seq, s_o_len, s_o_head, s_o_group;
    int32_t out_dtype;
    int32_t direct;
    int32_t spw;        // chained layout: partition slots one wave runs in turn (0: one slot per workgroup)
    int32_t merge_lds;  // bytes of dynamic LDS holding the partials a merging workgroup reads (0: global)
    int32_t spread;     // several slots per sequence: spread each sequence's items over the XCDs (slot_item)
};

struct WorklistParams {
    DecodeParams kv;  // caches, query, scales, shape; bt / max_blocks / partials unused
    const int32_t *work_indptr;
    const int32_t *work_info;
    const int32_t *kv_page_indices;
    const int32_t *kv_indptr;
    const int32_t *partition_indptr;
    float *po;
    float *pl;
    void *out;
    int64_t s_out_seq, s_out_head;
    int64_t s_po_row, s_pl_row;
    int32_t batch, num_kv_heads, num_pages, max_work, partial_rows, output_rows, out_dtype;
    int32_t head_dim;
    int32_t bin_groups;  // > 1: bin group a runs on the workgroups of dispatch round a
    int32_t num_bins;    // bins of the schedule (workgroups = num_bins * kv.chunks)
};

// Launch of the partition / worklist kernel for head dim D (v4: the 4-D value
// layout; mtp = 16-row query groups of one workgroup, rounded up; waves = waves
// per slot of the one-group layout).  Defined in the pa_decode_hd.hip object
// built for D.
template <int D>
hipError_t dispatch_partition(const DecodeParams &p, bool per_token, bool v4, int mtp, int waves, dim3 grid,
                              hipStream_t s);
template <int D>
hipError_t dispatch_worklist(const WorklistParams &w, bool per_token, bool v4, int mtp, dim3 grid, hipStream_t s);

#define PA_DECLARE_HEAD_DIM(D)                                                                                     \
    template <>                                                                                                    \
    hipError_t dispatch_partition<D>(const DecodeParams &, bool, bool, int, int, dim3, hipStream_t);              \
    template <>                                                                                                    \
    hipError_t dispatch_worklist<D>(const WorklistParams &, bool, bool, int, dim3, hipStream_t);
PA_DECLARE_HEAD_DIM(64)
PA_DECLARE_HEAD_DIM(128)
PA_DECLARE_HEAD_DIM(192)
PA_DECLARE_HEAD_DIM(256)
#undef PA_DECLARE_HEAD_DIM

}  // namespace pa
