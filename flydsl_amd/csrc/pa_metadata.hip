// get_pa_metadata_v1 worklist scheduler on the device (kernels/pa_metadata.py:145-420).
//
// The schedule is a serial state machine over (CU bin, batch) pairs, so one
// thread runs it; it is tiny (O(num_cu + batch) steps per kv head) and keeps
// the caller free of a device->host copy of context_lens.  Buffers are written
// exactly where the reference writes them, including its overwrite-safe
// unconditional stores; only the valid prefixes are defined.  Every store is
// bounds-checked against the buffer sizes the host passes; a schedule that
// would overflow sets work_indptr[0] = -1 so the host can report it.
#include "pa_common.h"
#include "pa_fp8.h"

namespace {

struct MetaParams {
    const int32_t *sq;
    const int32_t *ctx;
    int32_t *work_indptr;
    int32_t *work_info;
    int32_t *reduce_indptr;
    int32_t *reduce_final_map;
    int32_t *reduce_partial_map;
    int32_t nb, gqa, nhk, num_cu, kv_gran, ql, max_work, max_split_tiles;
};

__device__ __forceinline__ int cdiv_u(int a, int b) { return (int)(((unsigned)a + (unsigned)b - 1u) / (unsigned)b); }

__global__ __launch_bounds__(64) void pa_metadata_v1_kernel(const MetaParams p) {
    if (threadIdx.x != 0) return;
    const int nspk = p.num_cu / p.nhk;
    long long sum_blocks = 0;
    for (int b = 0; b < p.nb; ++b) sum_blocks += cdiv_u(p.ctx[b], p.kv_gran);
    const int average = (int)(sum_blocks / nspk);
    const int reminder = (int)(sum_blocks % nspk);
    auto quota = [&](int c) { return average + ((c % nspk) < reminder ? 1 : 0); };
    auto npart = [&](int b) { return cdiv_u(p.ctx[b], p.kv_gran); };
    bool overflow = false;

    p.work_indptr[0] = 0;
    p.reduce_indptr[0] = 0;
    int cid = 0, num_works = 0, lri = 0, grt = 0;
    for (int kh = 0; kh < p.nhk; ++kh) {
        const int32_t qhr =
            (int32_t)((((unsigned)(kh + 1) * (unsigned)p.gqa) << 16) | (((unsigned)kh * (unsigned)p.gqa) & 0xFFFFu));
        int batch = 0, kvblk = 0, nsplit = 0, pidx = 0, kvbeg = 0;
        int kvend = p.nb > 0 ? npart(0) : 0;
        int remain = quota(cid);
        lri = 0;
        grt = 0;
        while (cid < p.num_cu && batch < p.nb) {
            const int remain_kv = (kvend - kvbeg) - kvblk;
            const bool do_finish = remain >= remain_kv;
            const int qo_start = p.sq[batch];
            const int qo_end = p.sq[batch + 1];
            const int kv_start = kvbeg + kvblk;
            const int w_ploc = do_finish ? (nsplit > 0 ? pidx : -1) : pidx;
            const int w_kv_end = do_finish ? kvend : min(kv_start + remain, kvend);
            if (num_works < p.max_work) {
                int32_t *w = p.work_info + (long long)num_works * 8;
                w[0] = batch;
                w[1] = w_ploc;
                w[2] = qo_start;
                w[3] = qo_end;
                w[4] = kv_start;
                w[5] = w_kv_end;
                w[6] = 0;
                w[7] = qhr;
            } else {
                overflow = true;
            }
            const bool do_reduce = do_finish && nsplit > 0;
            const int num_splits = nsplit + 1;
            if (grt + 1 <= p.nb) p.reduce_indptr[grt + 1] = lri + num_splits;
            if (grt < p.nb) {
                p.reduce_final_map[2 * grt] = qo_start;
                p.reduce_final_map[2 * grt + 1] = qo_end;
            }
            if (do_reduce) {
                for (int s = 0; s < num_splits; ++s) {
                    if (lri + s < p.max_split_tiles)
                        p.reduce_partial_map[lri + s] = pidx - (nsplit - s) * p.ql;
                    else
                        overflow = true;
                }
            }
            const int n_lri = lri + (do_reduce ? num_splits : 0);
            const int n_grt = grt + (do_reduce ? 1 : 0);
            int n_nworks;
            if (do_finish) {
                n_nworks = num_works + 1;
                pidx = nsplit > 0 ? pidx + p.ql : pidx;
                remain = remain - remain_kv;
                batch = batch + 1;
                kvblk = 0;
                nsplit = 0;
                kvbeg = kvend;
                kvend = kvend + (batch < p.nb ? npart(batch) : 0);
                p.work_indptr[cid + 1] = n_nworks;
            } else {
                const bool emit = remain > 0;
                n_nworks = emit ? num_works + 1 : num_works;
                pidx = emit ? pidx + p.ql : pidx;
                kvblk = emit ? kvblk + remain : kvblk;
                nsplit = emit ? nsplit + 1 : nsplit;
                p.work_indptr[cid + 1] = n_nworks;
                cid = cid + 1;
                remain = quota(cid);
            }
            num_works = n_nworks;
            lri = n_lri;
            grt = n_grt;
        }
        if (cid < p.num_cu) cid += 1;
    }
    for (int i = cid; i <= p.num_cu; ++i) p.work_indptr[i] = num_works;
    for (int i = grt; i <= p.nb; ++i) p.reduce_indptr[i] = lri;
    if (overflow) p.work_indptr[0] = -1;
}

}  // namespace

extern "C" int pa_fp8_metadata_v1(const pa_fp8_metadata_args *a, void *stream) {
    if (!a) return PA_FP8_ERR_NULL_POINTER;
    if (a->num_batches < 0 || a->gqa <= 0 || a->num_heads_k <= 0 || a->num_cu <= 0 || a->query_length <= 0)
        return PA_FP8_ERR_SHAPE;
    if (a->num_cu % a->num_heads_k != 0) return PA_FP8_ERR_SHAPE;
    if (a->kv_granularity <= 0 || (a->kv_granularity & (a->kv_granularity - 1)) != 0) return PA_FP8_ERR_SHAPE;
    if (!a->seqlens_qo_indptr || !a->context_lens || !a->work_indptr || !a->work_info || !a->reduce_indptr ||
        !a->reduce_final_map || !a->reduce_partial_map)
        return PA_FP8_ERR_NULL_POINTER;
    if (a->max_work < 0 || a->max_split_tiles < 0) return PA_FP8_ERR_SHAPE;
    MetaParams p;
    p.sq = a->seqlens_qo_indptr;
    p.ctx = a->context_lens;
    p.work_indptr = a->work_indptr;
    p.work_info = a->work_info;
    p.reduce_indptr = a->reduce_indptr;
    p.reduce_final_map = a->reduce_final_map;
    p.reduce_partial_map = a->reduce_partial_map;
    p.nb = a->num_batches;
    p.gqa = a->gqa;
    p.nhk = a->num_heads_k;
    p.num_cu = a->num_cu;
    p.kv_gran = a->kv_granularity;
    p.ql = a->query_length;
    p.max_work = a->max_work;
    p.max_split_tiles = a->max_split_tiles;
    hipLaunchKernelGGL(pa_metadata_v1_kernel, dim3(1), dim3(64), 0, reinterpret_cast<hipStream_t>(stream), p);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? PA_FP8_OK : PA_FP8_ERR_HIP + (int)err;
}
