/*
 * CPU restatement, in plain C, of the get_pa_metadata_v1 worklist scheduler
 * (kernels/pa_metadata.py:145-420).  TEST INFRASTRUCTURE ONLY: it is the
 * checker for the device scheduler in flydsl_amd/csrc/pa_metadata.hip and is
 * never linked into the product library.
 *
 * Buffers are written exactly where the reference kernel writes them,
 * including its unconditional overwrite-safe stores (work slot at num_works,
 * reduce_indptr[grt+1], reduce_final_map[grt]); only the valid prefixes are
 * defined.  Returns 0, or -1 when a store would leave a buffer (the reference
 * sizes its buffers from get_pa_metadata_info_v1, kernels/pa_metadata.py:53-79).
 */
#include <stdint.h>

static int cdiv_u(int a, int b) { return (int)(((unsigned)a + (unsigned)b - 1u) / (unsigned)b); }

int pa_metadata_v1_ref(const int32_t *seqlens_qo_indptr, const int32_t *context_lens, int num_batches,
                       int gqa, int num_heads_k, int num_cu, int kv_granularity, int query_length,
                       int32_t *work_indptr, int32_t *work_info, int max_work, int32_t *reduce_indptr,
                       int32_t *reduce_final_map, int32_t *reduce_partial_map, int max_split_tiles,
                       int32_t *num_reduce_groups)
{
    if (num_heads_k <= 0 || num_cu % num_heads_k != 0 || kv_granularity <= 0 ||
        (kv_granularity & (kv_granularity - 1)) != 0)
        return -2;
    const int nspk = num_cu / num_heads_k;
    long long sum_blocks = 0;
    for (int b = 0; b < num_batches; ++b)
        sum_blocks += cdiv_u(context_lens[b], kv_granularity);
    const int average = (int)(sum_blocks / nspk);
    const int reminder = (int)(sum_blocks % nspk);
#define QUOTA(c) (average + (((c) % nspk) < reminder ? 1 : 0))
#define NPART(b) cdiv_u(context_lens[(b)], kv_granularity)

    work_indptr[0] = 0;
    reduce_indptr[0] = 0;
    int cid = 0, num_works = 0, lri = 0, grt = 0;
    for (int kh = 0; kh < num_heads_k; ++kh) {
        const int32_t qhr = (int32_t)((((unsigned)(kh + 1) * (unsigned)gqa) << 16) |
                                      (((unsigned)kh * (unsigned)gqa) & 0xFFFFu));
        int batch = 0, kvblk = 0, nsplit = 0, pidx = 0, kvbeg = 0;
        int kvend = num_batches > 0 ? NPART(0) : 0;
        int remain = QUOTA(cid);
        lri = 0;
        grt = 0;
        while (cid < num_cu && batch < num_batches) {
            const int remain_kv = (kvend - kvbeg) - kvblk;
            const int do_finish = remain >= remain_kv;
            const int qo_start = seqlens_qo_indptr[batch];
            const int qo_end = seqlens_qo_indptr[batch + 1];
            const int kv_start = kvbeg + kvblk;
            int w_ploc, w_kv_end;
            if (do_finish) {
                w_ploc = nsplit > 0 ? pidx : -1;
                w_kv_end = kvend;
            } else {
                w_ploc = pidx;
                w_kv_end = kv_start + remain < kvend ? kv_start + remain : kvend;
            }
            if (num_works >= max_work)
                return -1;
            int32_t *w = work_info + (long long)num_works * 8;
            w[0] = batch;
            w[1] = w_ploc;
            w[2] = qo_start;
            w[3] = qo_end;
            w[4] = kv_start;
            w[5] = w_kv_end;
            w[6] = 0;
            w[7] = qhr;

            const int do_reduce = do_finish && nsplit > 0;
            const int num_splits = nsplit + 1;
            if (grt + 1 > num_batches)
                return -1;
            reduce_indptr[grt + 1] = lri + num_splits;
            if (grt < num_batches) {
                reduce_final_map[2 * grt] = qo_start;
                reduce_final_map[2 * grt + 1] = qo_end;
            }
            if (do_reduce) {
                for (int s = 0; s < num_splits; ++s) {
                    if (lri + s >= max_split_tiles)
                        return -1;
                    reduce_partial_map[lri + s] = pidx - (nsplit - s) * query_length;
                }
            }
            const int n_lri = lri + (do_reduce ? num_splits : 0);
            const int n_grt = grt + (do_reduce ? 1 : 0);
            int n_cid, n_batch, n_kvblk, n_nsplit, n_nworks, n_pidx, n_kvbeg, n_kvend, n_remain;
            if (do_finish) {
                n_cid = cid;
                n_pidx = nsplit > 0 ? pidx + query_length : pidx;
                n_nworks = num_works + 1;
                n_remain = remain - remain_kv;
                n_batch = batch + 1;
                n_kvblk = 0;
                n_nsplit = 0;
                n_kvbeg = kvend;
                n_kvend = kvend + (n_batch < num_batches ? NPART(n_batch) : 0);
            } else {
                const int emit = remain > 0;
                n_cid = cid + 1;
                n_pidx = emit ? pidx + query_length : pidx;
                n_nworks = emit ? num_works + 1 : num_works;
                n_kvblk = emit ? kvblk + remain : kvblk;
                n_nsplit = emit ? nsplit + 1 : nsplit;
                n_remain = QUOTA(n_cid);
                n_batch = batch;
                n_kvbeg = kvbeg;
                n_kvend = kvend;
            }
            work_indptr[cid + 1] = n_nworks;
            cid = n_cid;
            batch = n_batch;
            kvblk = n_kvblk;
            nsplit = n_nsplit;
            num_works = n_nworks;
            pidx = n_pidx;
            kvbeg = n_kvbeg;
            kvend = n_kvend;
            remain = n_remain;
            lri = n_lri;
            grt = n_grt;
        }
        if (cid < num_cu)
            cid += 1;
    }
    for (int i = cid; i <= num_cu; ++i)
        work_indptr[i] = num_works;
    for (int i = grt; i <= num_batches; ++i)
        reduce_indptr[i] = lri;
    if (num_reduce_groups)
        *num_reduce_groups = grt;
    return 0;
#undef QUOTA
#undef NPART
}
