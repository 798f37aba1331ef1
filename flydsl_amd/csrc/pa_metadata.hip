// get_pa_metadata_v1 worklist scheduler on the device (kernels/pa_metadata.py:145-420).
//
// The reference runs the schedule as a serial state machine over (CU bin, batch)
// pairs.  Here a parallel kernel computes the same output in closed form for the
// common case (pa_metadata_par_kernel) and the serial machine runs, on one wave of
// the same workgroup, only where it cannot (serial_schedule); one launch either way,
// and the caller needs no device->host copy of context_lens.  Buffers are written
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
    int32_t *partition_indptr;  // optional outputs
    int32_t *uniform_context;
    int32_t *partial_count;     // reduce_indptr[nb]: split partials of the schedule
    int32_t nb, gqa, nhk, num_cu, kv_gran, ql, max_work, max_split_tiles;
    int32_t bin_groups;      // > 1: weighted quotas over this many equal groups of each head's bins
    int32_t bin_weight[4];   // weight of group g (bins [g*nspk/G, (g+1)*nspk/G) of every head)
    int32_t pack;            // 1: the packing schedule where it applies (pack_schedule)
};

__device__ __forceinline__ int cdiv_u(int a, int b) { return (int)(((unsigned)a + (unsigned)b - 1u) / (unsigned)b); }

// query offset of batch b: the caller's seqlens_qo_indptr, or b * query_length for
// a null pointer (every batch decodes query_length tokens)
__device__ __forceinline__ int sq_at(const MetaParams &p, int b) { return p.sq ? p.sq[b] : b * p.ql; }

constexpr int kStagedBatches = 4096;   // batches whose qo offsets and partition counts are staged in LDS
constexpr int kRingRows = 1024;        // work_info rows buffered in LDS before a coalesced copy-out
constexpr int kStagedIndptr = 4097;    // work_indptr entries kept in LDS (num_cu + 1)
constexpr int kStagedReduce = 2048;    // batches whose reduce maps are kept in LDS
constexpr int kStagedSplits = 4096;    // reduce_partial_map entries kept in LDS

constexpr int kMaxSchedules = 4;       // schedules one launch computes (one workgroup each)
constexpr int kParThreads = 1024;
constexpr int kParBatches = 4 * kParThreads;         // batches the parallel scheduler handles
constexpr int kParBins = 4096;                       // bins per head the weighted quota table holds
constexpr int kPackBatches = 2048;                   // batches the packing schedule handles
constexpr int kPackBins = 2048;                      // bins per head the packing schedule handles
// LDS of the packing schedule (pack_schedule's arrays)
constexpr int kPackInts = 8 * (kPackBatches + 4) + 2 * 12 + 6 * (kPackBins + 4);
// LDS of the sequential fill's per-batch arrays (works, split works, split batches, first bin)
constexpr int kFillInts = 4 * (kParBatches + 4);
constexpr int kUnionInts = kPackInts > kFillInts ? kPackInts : kFillInts;
// The closed-form kernel's LDS: partitions before each batch, bin starts, and the region
// the sequential fill and the packing schedule share (offsets in ints, 16-byte aligned).
constexpr int kParP = 0;
constexpr int kParQ = kParP + kParBatches + 4;
constexpr int kParU = kParQ + kParBins + 4;
constexpr int kParInts = kParU + kUnionInts;
// The serial state machine's LDS, carved from the same array when it runs instead:
// partition counts, query offsets, the work_info ring, work_indptr, the reduce maps.
constexpr int kSerialNp = 0;
constexpr int kSerialSq = kSerialNp + kStagedBatches;
constexpr int kSerialRing = kSerialSq + kStagedBatches + 4;
constexpr int kSerialWi = kSerialRing + kRingRows * 8;
constexpr int kSerialRi = kSerialWi + (kStagedIndptr + 3) / 4 * 4;
constexpr int kSerialRfm = kSerialRi + (kStagedReduce + 1 + 3) / 4 * 4;
constexpr int kSerialRpm = kSerialRfm + 2 * kStagedReduce;
constexpr int kSerialInts = kSerialRpm + kStagedSplits;
constexpr int kSharedInts = kParInts > kSerialInts ? kParInts : kSerialInts;
static_assert(kParU % 4 == 0 && kSerialRing % 4 == 0, "16-byte aligned regions");

// One wave's LDS and global writes ordered before its later reads (the serial state
// machine runs on a single wave of the workgroup, so it synchronises with no barrier).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

__device__ void serial_schedule(const MetaParams &p, int32_t *lds);

// The schedules of one launch: workgroup i of each kernel computes p[i].
struct MetaSchedules {
    MetaParams p[kMaxSchedules];
};

// Exclusive prefix of one value per thread over the 1024 threads; *total gets the sum.
template <class T>
__device__ __forceinline__ T block_scan_excl(T v, T *s_wave, T &total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    T x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const T y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    if (lane == 63) s_wave[wave] = x;
    __syncthreads();
    T before = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < kParThreads / 64; ++w) {
        const T t = s_wave[w];
        before += w < wave ? t : T(0);
        tot += t;
    }
    __syncthreads();  // s_wave is reused by the next scan
    total = tot;
    return before + x - v;
}

// floor(a / b) for 0 <= a < 2^53 and b > 0: the correctly rounded double quotient
// is within 1 of a / b there, and one integer step either way makes it exact (a
// fraction of the cost of the 64-bit integer division routine)
__device__ __forceinline__ long long floor_div_ll(long long a, long long b) {
    long long q = (long long)((double)a / (double)b);
    if (q * b > a) --q;
    else if ((q + 1) * b <= a) ++q;
    return q;
}

// Weighted quotas apply when every bin keeps at least one partition: S >= 4 nspk
// and S * (least weight) >= 2 * Wt (a bin's quota is at least S w / Wt - 1), and a
// head has at most kParBins bins, and the context lengths are not all equal (equal
// sequences fill equal bins whole, which the weights would break into split
// pieces).  wt gets Wt.
__device__ __forceinline__ bool weighted_quotas(const MetaParams &p, long long S64, int nspk, bool equal_ctx,
                                                long long &wt) {
    const int ng = p.bin_groups;
    bool weighted = !equal_ctx && ng > 1 && ng <= 4 && nspk % ng == 0 && S64 >= 4LL * nspk && nspk <= kParBins;
    long long wmin = 1000;
    wt = 0;
    if (weighted) {
        for (int g = 0; g < ng; ++g) {
            wt += p.bin_weight[g] * (long long)(nspk / ng);
            wmin = min(wmin, (long long)p.bin_weight[g]);
        }
        weighted = S64 * wmin >= 2 * wt;
    }
    return weighted;
}

// Qs(c) = floor(S * Wc(c) / Wt) for c in [0, nspk], Wc(c) the weights of the bins
// before c (the threads of the workgroup share the entries).
__device__ __forceinline__ void fill_weighted_starts(const MetaParams &p, long long S64, int nspk, long long wt,
                                                     int32_t *s_Q) {
    const int ng = p.bin_groups, gm = nspk / ng;
    for (int c = threadIdx.x; c <= nspk; c += blockDim.x) {
        long long wc = 0;
        for (int g = 0; g < ng; ++g) wc += p.bin_weight[g] * (long long)min(max(c - g * gm, 0), gm);
        s_Q[c] = (int)floor_div_ll(S64 * wc, wt);  // S < 2^31, wc <= Wt < 2^22
    }
}

// Inclusive prefix sum of x over the 64 lanes of a wave by DPP: row shifts by 1, 2,
// 4 and 8 inside each row of 16 lanes, then the broadcasts of lane 15 into rows 1
// and 3 and of lane 31 into rows 2 and 3 (row_bcast, GFX9 family).  Six VALU adds
// instead of six dependent cross-lane LDS round trips.
__device__ __forceinline__ int wave_scan_incl(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31
    return x;
}

// The largest (MAX) or smallest x of a wave, in every lane: the same DPP steps with
// the operation's identity for lanes without a source, then lane 63 read out.
template <bool MAX>
__device__ __forceinline__ int wave_extreme(int x) {
    const int id = MAX ? INT32_MIN : INT32_MAX;
    auto op = [](int u, int v) { return MAX ? max(u, v) : min(u, v); };
    x = op(x, __builtin_amdgcn_update_dpp(id, x, 0x111, 0xf, 0xf, false));
    x = op(x, __builtin_amdgcn_update_dpp(id, x, 0x112, 0xf, 0xf, false));
    x = op(x, __builtin_amdgcn_update_dpp(id, x, 0x114, 0xf, 0xf, false));
    x = op(x, __builtin_amdgcn_update_dpp(id, x, 0x118, 0xf, 0xf, false));
    x = op(x, __builtin_amdgcn_update_dpp(id, x, 0x142, 0xa, 0xf, false));
    x = op(x, __builtin_amdgcn_update_dpp(id, x, 0x143, 0xc, 0xf, false));
    return __builtin_amdgcn_readlane(x, 63);
}

// Four non-negative ints per thread scanned over the workgroup in one pass: exclusive
// prefixes and totals of a, b, c and d.  Every total here is below 2^31, so each
// pair of wave totals shares one 64-bit LDS word (the low half never carries).
__device__ __forceinline__ void scan_quad(int a, int b, int c, int d, long long *s_w64, int &pa, int &pb, int &pc,
                                          int &pd, int &ta, int &tb, int &tc, int &td) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    long long x = (long long)wave_scan_incl(a) + ((long long)wave_scan_incl(b) << 32);
    long long y = (long long)wave_scan_incl(c) + ((long long)wave_scan_incl(d) << 32);
    const long long x_in = (long long)a + ((long long)b << 32), y_in = (long long)c + ((long long)d << 32);
    if (lane == 63) {
        s_w64[2 * wave] = x;
        s_w64[2 * wave + 1] = y;
    }
    __syncthreads();
    long long bx = 0, by = 0, tx = 0, ty = 0;
#pragma unroll
    for (int w = 0; w < kParThreads / 64; ++w) {
        const long long vx = s_w64[2 * w], vy = s_w64[2 * w + 1];
        bx += w < wave ? vx : 0;
        by += w < wave ? vy : 0;
        tx += vx;
        ty += vy;
    }
    __syncthreads();
    x = bx + x - x_in;
    y = by + y - y_in;
    pa = (int)(x & 0xffffffffLL);
    pb = (int)(x >> 32);
    pc = (int)(y & 0xffffffffLL);
    pd = (int)(y >> 32);
    ta = (int)(tx & 0xffffffffLL);
    tb = (int)(tx >> 32);
    tc = (int)(ty & 0xffffffffLL);
    td = (int)(ty >> 32);
}

// The packing schedule (get_pa_metadata's tuned schedule, when it applies): with
// the same quotas as the sequential fill, sequences in order of (partitions
// descending, batch) and bins in order of (quota descending, bin), rank k < min(n,
// B) places sequence k whole in bin k; the other sequences are poured in rank
// order into the bins' remaining room (in bin-rank order), split at room
// boundaries, and an empty one becomes an empty work in the last bin with room.
// A bin runs its whole sequence, then its poured pieces in rank order.  Split
// sequences form the reduce groups in batch order, their pieces taking
// consecutive partial rows by position.  It applies when every rank k < min(n, B)
// fits its bin (then a head has at most B + bins with room - 1 works and at most
// 2 (bins - 1) split pieces, within the buffers' bounds), B <= kPackBatches,
// n <= kPackBins, no context length is negative and the partitions total 1 ..
// 2^31 - 1.  Returns true when it wrote the schedule (work_indptr[0] = 0), false
// (nothing written, its LDS free again) when the sequential fill is to run.  The
// caller has the partition prefix in s_P and the total S; `u` is LDS for
// kPackInts ints.
// Ranks are counted directly (the lanes of an element compare it with every
// other one, read as LDS broadcasts), which for the batch sizes of a decode step
// is several times quicker than a barrier-per-stage sort.
__device__ bool pack_schedule(const MetaParams &p, const int S, const bool equal_ctx, const int32_t *s_P,
                              int32_t *s_Qs, int32_t *u,
                              long long *s_w64, int32_t *s_red, int32_t *s_flag) {
    int32_t *s_Pv = u;                            // partitions of batch b (padded to 16-value rounds)
    int32_t *s_sq = s_Pv + kPackBatches + 16;     // query rows before batch b
    int32_t *s_ord = s_sq + kPackBatches + 4;     // batch of rank k
    int32_t *s_Qv = s_ord + kPackBatches;         // quota of bin c (padded to 16-value rounds)
    int32_t *s_bo = s_Qv + kPackBins + 16;        // bin of rank j
    int32_t *s_Y = s_bo + kPackBins;              // room of the bin ranks before j (the pour line)
    int32_t *s_G = s_Y + kPackBins + 4;           // bin ranks with room before j
    int32_t *s_X = s_G + kPackBins + 4;           // pour position of rank k (ranks >= m)
    int32_t *s_np = s_X + kPackBatches + 4;       // works of batch b
    int32_t *s_PB = s_np + kPackBatches;          // pieces of split batches before b
    int32_t *s_GB = s_PB + kPackBatches + 4;      // split batches before b
    int32_t *s_cnt = s_GB + kPackBatches + 4;     // works of bin c
    int32_t *s_WI = s_cnt + kPackBins;            // works of the bins before c (one head)
    int32_t *s_J = s_WI + kPackBins + 4;          // first bin rank of pour rank k
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int nb = p.nb, nspk = p.num_cu / p.nhk;
    auto give_up = [&]() {
        __syncthreads();
        return false;
    };
    int pmax = 0;
    for (int b = t; b < nb; b += kParThreads) {
        const int v = s_P[b + 1] - s_P[b];
        s_Pv[b] = v;
        pmax = max(pmax, v);
    }
    pmax = wave_extreme<true>(pmax);
    if (lane == 0) s_red[wv] = pmax;
    if (t == 0) s_flag[0] = 0;
    const long long S64 = S;
    long long wt = 0;
    const bool weighted = weighted_quotas(p, S64, nspk, equal_ctx, wt);
    if (weighted) fill_weighted_starts(p, S64, nspk, wt, s_Qs);
    else
        for (int c = t; c <= nspk; c += kParThreads)
            s_Qs[c] = (int)((long long)c * (S / nspk) + min(c, S % nspk));
    __syncthreads();  // s_Qs, s_Pv, s_sq, the batch maxima
    int qmax = 0;
    for (int c = t; c < nspk; c += kParThreads) {
        s_Qv[c] = s_Qs[c + 1] - s_Qs[c];
        qmax = max(qmax, s_Qv[c]);
    }
    qmax = wave_extreme<true>(qmax);
    if (lane == 0) s_red[kParThreads / 64 + wv] = qmax;
    if (t < 16) {  // padding past the last batch and bin: never counted (real values are >= 0)
        s_Pv[nb + t] = -1;
        s_Qv[nspk + t] = -1;
    }
    __syncthreads();
    int Pmax = 0, Qmax = 0;
#pragma unroll
    for (int w = 0; w < kParThreads / 64; ++w) {
        Pmax = max(Pmax, s_red[w]);
        Qmax = max(Qmax, s_red[kParThreads / 64 + w]);
    }
    // the largest sequence fits no bin (the rule fails at rank 0), or a quota too
    // large for the 31-bit rank keys below
    if (Pmax > Qmax || Qmax >= (1 << 19)) return give_up();
    for (int b = t; b <= nb; b += kParThreads) s_sq[b] = sq_at(p, b);  // read before the writes' barriers
    // ranks: batch b goes before b' when P_b > P_b', or equal and b < b' (bins alike
    // by quota), i.e. when its key v << 12 | (4095 - index) is larger (values <
    // 2^19, indices < 4096).  Batches are ranked by the first half of the threads,
    // bins by the second.  Each element's rank is counted by tpe adjacent lanes
    // (tpe = the power of two <= 512 / n, at most 64); lane `part` reads the
    // 16-byte pieces part, part + tpe, ... (adjacent lanes, adjacent pieces: no bank
    // conflicts), and the counts are summed across the lanes.  The keys replace
    // the values in s_Pv / s_Qv only for the count (the values come back after).
    auto make_keys = [&](int32_t *v, int n, int tid) {
        for (int i = tid; i < n; i += kParThreads / 2) v[i] = (v[i] << 12) | (4095 - i);
        for (int i = tid; i < 16; i += kParThreads / 2) v[n + i] = -1;  // the padding never counts
    };
    auto count = [&](const int32_t *v, int n, int32_t *out, int tid) {
        int tpe = 1;
        while (tpe < 64 && tpe * 2 * n <= kParThreads / 2) tpe <<= 1;
        const int n4 = (n + 3) >> 2;  // 16-byte pieces (the -1 padding covers the tail)
        for (int base = 0; base < n * tpe; base += kParThreads / 2) {
            const int e = (base + tid) / tpe, part = (base + tid) % tpe;
            const int ki = v[e < n ? e : 0];
            int r = 0;
            for (int q = part; q < n4; q += 4 * tpe) {
                int4 w[4];
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    w[u] = q + u * tpe < n4 ? *reinterpret_cast<const int4 *>(v + 4 * (q + u * tpe))
                                            : make_int4(-1, -1, -1, -1);
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    r += (w[u].x > ki) + (w[u].y > ki) + (w[u].z > ki) + (w[u].w > ki);
            }
            for (int o = 1; o < tpe; o <<= 1) r += __shfl_xor(r, o, 64);
            if (part == 0 && e < n) out[r] = e;
        }
    };
    auto rank_all = [&]() {
        if (t < kParThreads / 2) make_keys(s_Pv, nb, t);
        else make_keys(s_Qv, nspk, t - kParThreads / 2);
        __syncthreads();
        if (t < kParThreads / 2) count(s_Pv, nb, s_ord, t);
        else count(s_Qv, nspk, s_bo, t - kParThreads / 2);
        __syncthreads();
        for (int i = t; i < nb; i += kParThreads) s_Pv[i] >>= 12;  // the values again
        for (int i = t; i < nspk; i += kParThreads) s_Qv[i] >>= 12;
        __syncthreads();
    };
    if (equal_ctx) {
        // every sequence has the same partitions and the quotas are even (no weights
        // apply to equal contexts), bins [0, S % bins) one partition above the rest:
        // both orders are the identity, so nothing is ranked
        for (int i = t; i < nb; i += kParThreads) s_ord[i] = i;
        for (int i = t; i < nspk; i += kParThreads) s_bo[i] = i;
        __syncthreads();
    } else {
        rank_all();
    }

    const int m = min(nspk, nb);
    for (int k = t; k < m; k += kParThreads)  // every rank k < m fits its bin
        if (s_Pv[s_ord[k]] > s_Qv[s_bo[k]]) s_flag[0] = 1;
    // room left in each bin (by rank), then the pour lengths of the ranks past m
    int ga[2], la[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int j = 2 * t + i;
        ga[i] = j < nspk ? s_Qv[s_bo[j]] - (j < m ? s_Pv[s_ord[j]] : 0) : 0;
        la[i] = (j >= m && j < nb) ? s_Pv[s_ord[j]] : 0;
    }
    const int za = (2 * t >= m && 2 * t < nb && la[0] == 0) + (2 * t + 1 >= m && 2 * t + 1 < nb && la[1] == 0);
    int y0, g0, Yt, Gt, x0p, z0, Xt, Zc;
    scan_quad(ga[0] + ga[1], (ga[0] > 0) + (ga[1] > 0), la[0] + la[1], za, s_w64, y0, g0, x0p, z0, Yt, Gt, Xt, Zc);
    if (s_flag[0]) return give_up();  // read after the scan's barriers
    if (2 * t < nspk) {
        s_Y[2 * t] = y0;
        s_G[2 * t] = g0;
    }
    if (2 * t + 1 < nspk) {
        s_Y[2 * t + 1] = y0 + ga[0];
        s_G[2 * t + 1] = g0 + (ga[0] > 0);
    }
    if (t == 0) {
        s_Y[nspk] = Yt;
        s_G[nspk] = Gt;
    }
    if (2 * t < nb) s_X[2 * t] = x0p;
    if (2 * t + 1 < nb) s_X[2 * t + 1] = x0p + la[0];
    if (t == 0) s_X[nb] = Xt;
    __syncthreads();
    if (Xt != Yt) return give_up();  // cannot happen: both are S minus the whole sequences
    const int kz = nb - Zc;  // ranks [m, kz) pour, ranks [kz, nb) are empty
    // the last bin rank with room (the empty sequences' bin), the last rank if none:
    // the last j with s_G[j] < Gt
    int zrank = nspk - 1;
    if (Gt > 0) {
        int lo = 0, hi = nspk - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (s_G[mid] < Gt) lo = mid;
            else hi = mid - 1;
        }
        zrank = lo;
    }
    // the bin rank holding pour position x (x < Yt): the last j with s_Y[j] <= x
    auto bin_at = [&](int x) {
        int lo = 0, hi = nspk - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (s_Y[mid] <= x) lo = mid;
            else hi = mid - 1;
        }
        return lo;
    };
    // the pour rank holding position x (x < Yt): the last k in [m, kz) with s_X[k] <= x
    auto rank_at = [&](int x) {
        int lo = m, hi = kz - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (s_X[mid] <= x) lo = mid;
            else hi = mid - 1;
        }
        return lo;
    };
    // works of every batch (and the first bin rank of every pour rank, kept in s_J),
    // and of every bin: its whole sequence, its pour pieces, the empty sequences
    auto pour_span = [&](int j, int &k0, int &k1) {  // pour ranks meeting bin rank j (k1 < k0 if none)
        k0 = 0;
        k1 = -1;
        const int room = s_Y[j + 1] - s_Y[j];
        if (room <= 0) return;
        k0 = rank_at(s_Y[j]);
        k1 = rank_at(s_Y[j] + room - 1);
    };
    for (int k = t; k < nb; k += kParThreads) {
        int w = 1;
        if (k >= m && k < kz) {
            const int x = s_X[k], len = s_Pv[s_ord[k]];
            const int j0 = bin_at(x);
            s_J[k] = j0;
            w = s_G[bin_at(x + len - 1) + 1] - s_G[j0];
        }
        s_np[s_ord[k]] = w;
    }
    for (int j = t; j < nspk; j += kParThreads) {
        int k0, k1;
        pour_span(j, k0, k1);
        s_cnt[s_bo[j]] = (j < m ? 1 : 0) + (k1 >= k0 ? k1 - k0 + 1 : 0) + (j == zrank ? Zc : 0);
    }
    __syncthreads();
    // split batches and their pieces before each batch, works of the bins before each bin
    int sp[2], sg[2], ca[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int b = 2 * t + i;
        const int w = b < nb ? s_np[b] : 0;
        sp[i] = w > 1 ? w : 0;
        sg[i] = w > 1 ? 1 : 0;
        ca[i] = b < nspk ? s_cnt[b] : 0;
    }
    int pb0, gb0, w0, dz, T, G, W, dzt;
    scan_quad(sp[0] + sp[1], sg[0] + sg[1], ca[0] + ca[1], 0, s_w64, pb0, gb0, w0, dz, T, G, W, dzt);
    if (2 * t < nb) {
        s_PB[2 * t] = pb0;
        s_GB[2 * t] = gb0;
    }
    if (2 * t + 1 < nb) {
        s_PB[2 * t + 1] = pb0 + sp[0];
        s_GB[2 * t + 1] = gb0 + sg[0];
    }
    if (2 * t < nspk) s_WI[2 * t] = w0;
    if (2 * t + 1 < nspk) s_WI[2 * t + 1] = w0 + ca[0];
    if (t == 0) s_WI[nspk] = W;
    __syncthreads();
    if ((long long)p.nhk * W > p.max_work || T > p.max_split_tiles) return give_up();  // within bounds by construction
    // work_info rows: one thread per (head, bin rank), so the heads' rows are written in
    // parallel rather than one after another
    for (int i = t; i < p.nhk * nspk; i += kParThreads) {
        const int kh = i / nspk, j = i - kh * nspk;
        const int32_t qhr = (int32_t)((((unsigned)(kh + 1) * (unsigned)p.gqa) << 16) |
                                      (((unsigned)kh * (unsigned)p.gqa) & 0xFFFFu));
        auto put = [&](int row, int b, int ploc, int k0, int k1) {
            int4 *w = reinterpret_cast<int4 *>(p.work_info) + 2 * ((long long)kh * W + row);
            w[0] = make_int4(b, ploc, s_sq[b], s_sq[b + 1]);
            w[1] = make_int4(s_P[b] + k0, s_P[b] + k1, 0, qhr);
        };
        int row = s_WI[s_bo[j]];
        if (j < m) {
            const int b = s_ord[j];
            put(row++, b, -1, 0, s_Pv[b]);
        }
        int k0, k1;
        pour_span(j, k0, k1);
        for (int k = k0; k <= k1; ++k) {
            const int b = s_ord[k];
            const int x = s_X[k], len = s_Pv[b];
            const int a = max(x, s_Y[j]) - x, e = min(x + len, s_Y[j + 1]) - x;
            const int piece = s_G[j] - s_G[s_J[k]];
            put(row++, b, s_np[b] > 1 ? p.ql * (s_PB[b] + piece) : -1, a, e);
        }
        if (j == zrank)
            for (int k = kz; k < nb; ++k) put(row++, s_ord[k], -1, 0, 0);
    }
    // work_indptr, the reduce maps, the split partial count
    for (int i = t; i < p.nhk * nspk; i += kParThreads) {
        const int kh = i / nspk, c = i - kh * nspk;
        p.work_indptr[i + 1] = kh * W + s_WI[c] + s_cnt[c];
    }
    for (int b = t; b < nb; b += kParThreads) {
        const int w = s_np[b];
        if (w < 2) continue;
        const int g = s_GB[b], lb = s_PB[b];
        p.reduce_indptr[g + 1] = lb + w;
        p.reduce_final_map[2 * g] = s_sq[b];
        p.reduce_final_map[2 * g + 1] = s_sq[b + 1];
        for (int i = 0; i < w; ++i) p.reduce_partial_map[lb + i] = p.ql * (lb + i);
    }
    for (int i = G + 1 + t; i <= nb; i += kParThreads) p.reduce_indptr[i] = T;
    if (t == 0) {
        p.reduce_indptr[0] = 0;
        if (p.partial_count) p.partial_count[0] = T;
        p.work_indptr[0] = 0;
    }
    return true;
}

// The state machine's output in closed form, computed in parallel.  With
// S = sum of partitions, avg = S / nspk, rem = S % nspk, bin c of a head takes the
// global partitions [Qs(c), Qs(c+1)), Qs(c) = c*avg + min(c, rem); batch b holds
// [P(b), P(b+1)).  The works of a batch are its non-empty intersections with the
// bins, in bin order (an empty batch makes one empty work in the bin of the
// partition before it, bin 0 if none); a batch with more than one work is split,
// its works take consecutive partial rows and it forms the next reduce group.
// When every bin has a partition (avg >= 1) or a head has one bin, head 0 ends in
// its last bin and every head repeats its schedule nspk bins later, as in the
// serial machine.  Otherwise (or with more than kParBatches batches, or more than
// 2^31 partitions) the workgroup's first wave runs the serial machine itself.
// With bin_groups = G > 1 (get_pa_metadata's option, off for get_pa_metadata_v1)
// the quotas are weighted instead: the bins of each head form G equal groups and
// bin c takes Qs(c) = floor(S * Wc(c) / Wt), Wc(c) the weights of the bins before
// it.  Every head keeps the same schedule, so the reduce maps are unchanged in
// form.  The weights apply when every bin still gets at least one partition
// (S >= 4 * nspk and S * min weight >= 2 * Wt) and a head has at most kParBins
// bins; otherwise the even split is used.
// Workgroup i computes schedule sched.p[i] (one launch can hold several).
__global__ __launch_bounds__(kParThreads) void pa_metadata_par_kernel(const MetaSchedules sched) {
    const MetaParams &p = sched.p[blockIdx.x];
    __shared__ __attribute__((aligned(16))) int32_t s_all[kSharedInts];
    int32_t *s_P = s_all + kParP;  // partitions before batch b
    int32_t *s_Q = s_all + kParQ;  // weighted quotas: first partition of bin c
    // the sequential fill's arrays and the packing schedule's share one region
    int32_t *s_u = s_all + kParU;
    int32_t *s_W = s_u;                        // works of head 0 before batch b
    int32_t *s_L = s_W + kParBatches + 4;      // works of split batches before batch b
    int32_t *s_G = s_L + kParBatches + 4;      // split batches before batch b
    int32_t *s_F = s_G + kParBatches + 4;      // first bin of batch b
    __shared__ long long s_w64[2 * (kParThreads / 64)];
    __shared__ int32_t s_mm[2 * (kParThreads / 64)];
    __shared__ int32_t s_pk[2 * (kParThreads / 64)];
    __shared__ int32_t s_flag[1];
    const int t = threadIdx.x;
    const int nspk = p.num_cu / p.nhk;
    // partitions per batch and their prefix (four consecutive batches per thread,
    // chunks of kParBatches), the optional partition_indptr and uniform_context
    int np4[4];
    long long S64 = 0, run = 0;
    int cmin = INT32_MAX, cmax = INT32_MIN;
    for (int base = 0; base < max(p.nb, 1); base += kParBatches) {
        long long loc = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int b = base + 4 * t + i;
            const int c = b < p.nb ? p.ctx[b] : 0;
            if (b < p.nb) {
                cmin = min(cmin, c);
                cmax = max(cmax, c);
            }
            np4[i] = b < p.nb ? cdiv_u(c, p.kv_gran) : 0;
            loc += np4[i];
        }
        long long total;
        run = S64 + block_scan_excl<long long>(loc, s_w64, total);
        if (p.partition_indptr) {
            long long r = run;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int b = base + 4 * t + i;
                if (b < p.nb) p.partition_indptr[b] = (int)r;
                r += np4[i];
            }
        }
        S64 += total;
    }
    if (p.partition_indptr && t == 0) p.partition_indptr[p.nb] = (int)S64;
    // every context length equal: the uniform_context output, and no weighted quotas
    bool equal_ctx = false;
    if (p.uniform_context || p.bin_groups > 1) {
        cmin = wave_extreme<false>(cmin);
        cmax = wave_extreme<true>(cmax);
        if ((t & 63) == 0) {
            s_mm[2 * (t >> 6)] = cmin;
            s_mm[2 * (t >> 6) + 1] = cmax;
        }
        __syncthreads();
        int a = INT32_MAX, z = INT32_MIN;
        for (int w = 0; w < kParThreads / 64; ++w) {
            a = min(a, s_mm[2 * w]);
            z = max(z, s_mm[2 * w + 1]);
        }
        equal_ctx = p.nb == 0 || a == z;
        if (t == 0 && p.uniform_context) p.uniform_context[0] = equal_ctx ? 1 : 0;
    }
    // the packing schedule, where it applies, instead of the sequential fill
    if (p.pack && p.nb >= 1 && p.nb <= kPackBatches && nspk <= kPackBins && S64 >= 1 && S64 <= 0x7fffffffLL) {
        // no negative context length (the sequential fill keeps those), and the
        // largest sequence within an upper bound on any bin's quota (S / bins rounded
        // up, or S w_max / Wt + 1 with weights), checked before any packing work;
        // s_pk is touched by nothing else, so a rejection needs no further barrier
        int lo = cmin, hi = max(max(np4[0], np4[1]), max(np4[2], np4[3]));
        lo = wave_extreme<false>(lo);
        hi = wave_extreme<true>(hi);
        if ((t & 63) == 0) {
            s_pk[2 * (t >> 6)] = lo;
            s_pk[2 * (t >> 6) + 1] = hi;
        }
        __syncthreads();
        for (int w = 0; w < kParThreads / 64; ++w) {
            lo = min(lo, s_pk[2 * w]);
            hi = max(hi, s_pk[2 * w + 1]);
        }
        long long wt = 0, bound = floor_div_ll(S64 + nspk - 1, nspk);
        if (weighted_quotas(p, S64, nspk, equal_ctx, wt)) {
            long long wmax = 0;
            for (int g = 0; g < p.bin_groups; ++g) wmax = max(wmax, (long long)p.bin_weight[g]);
            bound = floor_div_ll(S64 * wmax, wt) + 1;
        }
        if (lo >= 0 && hi <= bound) {
            long long r = run;
#pragma unroll
            for (int i = 0; i < 4; ++i) {  // one chunk: run and np4 are this thread's prefix and counts
                const int b = 4 * t + i;
                if (b <= p.nb) s_P[b] = (int)r;
                r += np4[i];
            }
            if (t == 0) s_P[p.nb] = (int)S64;
            __syncthreads();
            if (pack_schedule(p, (int)S64, equal_ctx, s_P, s_Q, s_u, s_w64, s_mm, s_flag)) return;
            __syncthreads();  // s_mm, s_Q and the shared region are free again
        }
    }
    const bool ok = p.nb <= kParBatches && S64 <= 0x7fffffffLL && (S64 >= nspk || nspk == 1);
    if (!ok) {  // uniform: the serial machine on the first wave, the other waves end here
        // (every wave has passed a barrier since its last read of s_all, and the serial
        // machine synchronises within its wave only)
        if (t < 64) serial_schedule(p, s_all);
        return;
    }
    // one chunk (nb <= kParBatches): run and np4 are this thread's prefix and counts
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int b = 4 * t + i;
        if (b <= p.nb) s_P[b] = (int)run;
        run += np4[i];
    }
    if (t == 0) s_P[p.nb] = (int)S64;  // batch nb is past every thread's four when nb == kParBatches
    __syncthreads();
    const int S = (int)S64;
    const int avg = S / nspk, rem = S % nspk;
    const int big = rem * (avg + 1);
    long long wt = 0;
    const bool weighted = weighted_quotas(p, S64, nspk, equal_ctx, wt);
    // The first partition of every bin, Qs(c) = floor(S * Wc(c) / Wt), tabulated once
    // in LDS (bins are then found by a binary search over the table).
    if (weighted) {
        fill_weighted_starts(p, S64, nspk, wt, s_Q);
        __syncthreads();
    }
    auto Qs = [&](int c) { return weighted ? s_Q[c] : c * avg + min(c, rem); };
    auto bin_of = [&](int x) {  // the bin holding global partition x
        if (!weighted) return nspk == 1 ? 0 : (x < big ? x / (avg + 1) : rem + (x - big) / avg);
        int lo = 0, hi = nspk - 1;  // last bin whose first partition is <= x
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (s_Q[mid] <= x) lo = mid;
            else hi = mid - 1;
        }
        return lo;
    };
    // first bin and works of each batch, one batch per thread (the bin searches of all
    // batches run side by side; s_W holds the work counts until the scan below
    // replaces them), then the works, split works and split batches before each batch
    // (block scans over four consecutive batches per thread)
    for (int b = t; b < p.nb; b += kParThreads) {
        const int pb = s_P[b], pe = s_P[b + 1];
        const int fb = pe > pb ? bin_of(pb) : (pb == 0 ? 0 : bin_of(pb - 1));
        s_F[b] = fb;
        s_W[b] = pe > pb ? bin_of(pe - 1) - fb + 1 : 1;
    }
    __syncthreads();
    int w4[4], l4[4], g4[4];
    int wl = 0, ll = 0, gl = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int b = 4 * t + i;
        const int nw = b < p.nb ? s_W[b] : 0;  // read by every thread before scan_quad's first barrier
        w4[i] = nw;
        l4[i] = nw > 1 ? nw : 0;
        g4[i] = nw > 1 ? 1 : 0;
        wl += w4[i];
        ll += l4[i];
        gl += g4[i];
    }
    int W, Lt, G, zr, zt;
    int wr, lr, gr;
    scan_quad(wl, ll, gl, 0, s_w64, wr, lr, gr, zr, W, Lt, G, zt);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int b = 4 * t + i;
        if (b <= p.nb) {
            s_W[b] = wr;
            s_L[b] = lr;
            s_G[b] = gr;
        }
        wr += w4[i];
        lr += l4[i];
        gr += g4[i];
    }
    if (t == 0) {  // batch nb is past every thread's four when nb == kParBatches
        s_W[p.nb] = W;
        s_L[p.nb] = Lt;
        s_G[p.nb] = G;
    }
    __syncthreads();
    // a batch's works lie in consecutive bins of one head, so at most nspk of them
    auto works_of = [&](int b) { return min(max(s_W[b + 1] - s_W[b], 0), nspk); };
    const bool overflow = (long long)p.nhk * W > p.max_work || Lt > p.max_split_tiles;

    // work_info rows: one thread per (head, batch), so the heads' rows are written in
    // parallel rather than one after another
    for (int i = t; i < p.nhk * p.nb; i += kParThreads) {
        const int k = i / p.nb, b = i - k * p.nb;
        const int pb = s_P[b], pe = s_P[b + 1];
        const int c0 = s_F[b], nw = works_of(b);
        const int wb = s_W[b], lb = s_L[b];
        const int qs = sq_at(p, b), qe = sq_at(p, b + 1);
        const int32_t qhr = (int32_t)((((unsigned)(k + 1) * (unsigned)p.gqa) << 16) |
                                      (((unsigned)k * (unsigned)p.gqa) & 0xFFFFu));
        for (int j = 0; j < nw; ++j) {
            const long long row = (long long)k * W + wb + j;
            if (row >= p.max_work) continue;
            const int c = c0 + j;
            const int ks = pe > pb ? max(pb, Qs(c)) : pb;
            const int ke = pe > pb ? min(pe, Qs(c + 1)) : pb;
            const int ploc = nw > 1 ? p.ql * (lb + j) : -1;
            int4 *w = reinterpret_cast<int4 *>(p.work_info) + 2 * row;
            w[0] = make_int4(b, ploc, qs, qe);
            w[1] = make_int4(ks, ke, 0, qhr);
        }
    }
    // work_indptr: entry k*nspk + c + 1 = k*W + works of head 0 in bins <= c
    for (int c = t; c < nspk; c += kParThreads) {
        int v = 0;
        if (p.nb > 0) {
            int lo = 0, hi = p.nb - 1;  // last batch whose first bin is <= c (batch 0's is 0)
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (s_F[mid] <= c) lo = mid;
                else hi = mid - 1;
            }
            v = s_W[lo] + min(c - s_F[lo] + 1, works_of(lo));
        }
        for (int k = 0; k < p.nhk; ++k) p.work_indptr[k * nspk + c + 1] = k * W + v;
    }
    // reduce maps (the same for every head)
    for (int b = t; b < p.nb; b += kParThreads) {
        const int nw = works_of(b);
        if (nw < 2) continue;
        const int g = s_G[b], lb = s_L[b];
        p.reduce_indptr[g + 1] = lb + nw;
        p.reduce_final_map[2 * g] = sq_at(p, b);
        p.reduce_final_map[2 * g + 1] = sq_at(p, b + 1);
        for (int j = 0; j < nw; ++j)
            if (lb + j < p.max_split_tiles) p.reduce_partial_map[lb + j] = p.ql * (lb + j);
    }
    for (int i = G + t; i <= p.nb; i += kParThreads) p.reduce_indptr[i] = Lt;
    if (t == 0) {
        if (G > 0) p.reduce_indptr[0] = 0;
        if (p.partial_count) p.partial_count[0] = Lt;
        p.work_indptr[0] = overflow ? -1 : 0;
    }
}

// The serial state machine, run by the first wave of the closed-form kernel's
// workgroup where the closed form does not hold.  Every lane runs it on the same
// (uniform) values.  Its outputs go to LDS -- a ring of work_info rows, work_indptr and the reduce
// maps -- and the 64 lanes copy them to global memory with coalesced stores, so
// the loop is not throttled by single-lane global stores.  Per-batch partition
// counts and qo offsets are staged in LDS first (and the counts summed by all
// lanes).  Buffers larger than the LDS copies are written to global memory
// directly by lane 0.
__device__ void serial_schedule(const MetaParams &p, int32_t *lds) {
    int32_t *s_np = lds + kSerialNp;
    int32_t *s_sq = lds + kSerialSq;
    int32_t *s_ring = lds + kSerialRing;  // 16-byte aligned (lds is)
    int32_t *s_wi = lds + kSerialWi;
    int32_t *s_ri = lds + kSerialRi;
    int32_t *s_rfm = lds + kSerialRfm;
    int32_t *s_rpm = lds + kSerialRpm;
    const int lane = threadIdx.x;  // 0..63: the workgroup's first wave
    const bool lead = lane == 0;
    const int staged = min(p.nb, kStagedBatches);
    const bool wi_lds = p.num_cu + 1 <= kStagedIndptr;
    const bool red_lds = p.nb <= kStagedReduce;
    const bool rpm_lds = p.max_split_tiles <= kStagedSplits;
    long long part = 0;
    for (int b = lane; b < p.nb; b += 64) {
        const int n = cdiv_u(p.ctx[b], p.kv_gran);
        part += n;
        if (b < staged) s_np[b] = n;
    }
    for (int b = lane; b <= staged; b += 64) s_sq[b] = sq_at(p, b);
#pragma unroll
    for (int sh = 32; sh >= 1; sh >>= 1) part += __shfl_xor(part, sh, 64);
    wave_sync();
    const int nspk = p.num_cu / p.nhk;
    const long long sum_blocks = part;
    const int average = (int)(sum_blocks / nspk);
    const int reminder = (int)(sum_blocks % nspk);
    auto quota = [&](int c) { return average + ((c % nspk) < reminder ? 1 : 0); };
    auto npart = [&](int b) { return b < staged ? s_np[b] : cdiv_u(p.ctx[b], p.kv_gran); };
    auto sq = [&](int b) { return b <= staged ? s_sq[b] : sq_at(p, b); };
    auto put_wi = [&](int i, int v) {
        if (wi_lds) { if (lead) s_wi[i] = v; }
        else if (lead) p.work_indptr[i] = v;
    };
    auto put_ri = [&](int i, int v) {
        if (red_lds) { if (lead) s_ri[i] = v; }
        else if (lead) p.reduce_indptr[i] = v;
    };
    // entries [0, rfm_top) / [0, rpm_top) of the LDS reduce maps hold written values (the
    // copy-out leaves the caller's buffer alone past them, as the direct writes do)
    int rfm_top = 0, rpm_top = 0;
    auto put_rfm = [&](int g, int a, int b) {
        rfm_top = max(rfm_top, g + 1);
        if (red_lds) { if (lead) { s_rfm[2 * g] = a; s_rfm[2 * g + 1] = b; } }
        else if (lead) { p.reduce_final_map[2 * g] = a; p.reduce_final_map[2 * g + 1] = b; }
    };
    auto put_rpm = [&](int i, int v) {
        rpm_top = max(rpm_top, i + 1);
        if (rpm_lds) { if (lead) s_rpm[i] = v; }
        else if (lead) p.reduce_partial_map[i] = v;
    };
    // rows [flushed, upto) of the ring go to work_info (rows past max_work are dropped)
    int flushed = 0;
    auto flush = [&](int upto) {
        wave_sync();
        for (int i = flushed * 2 + lane; i < upto * 2; i += 64) {  // half rows of 16 bytes
            const int row = i >> 1;
            if (row < p.max_work)
                reinterpret_cast<int4 *>(p.work_info)[i] =
                    reinterpret_cast<const int4 *>(s_ring)[((row % kRingRows) << 1) | (i & 1)];
        }
        wave_sync();
        flushed = upto;
    };
    bool overflow = false;

    put_wi(0, 0);
    put_ri(0, 0);
    int cid = 0, num_works = 0, lri = 0, grt = 0;
    int last_slot = -1;  // the ring slot written last (the current work's, emitted or not)
    // one kv head of the state machine (kernels/pa_metadata.py:212-387), from the current cid
    auto run_head = [&](int kh) {
        const int32_t qhr =
            (int32_t)((((unsigned)(kh + 1) * (unsigned)p.gqa) << 16) | (((unsigned)kh * (unsigned)p.gqa) & 0xFFFFu));
        int batch = 0, kvblk = 0, nsplit = 0, pidx = 0, kvbeg = 0;
        int kvend = p.nb > 0 ? npart(0) : 0;
        int cpos = cid % nspk;  // cid % nspk, kept incrementally
        int remain = average + (cpos < reminder ? 1 : 0);
        lri = 0;
        grt = 0;
        while (cid < p.num_cu && batch < p.nb) {
            const int remain_kv = (kvend - kvbeg) - kvblk;
            const bool do_finish = remain >= remain_kv;
            const int qo_start = sq(batch);
            const int qo_end = sq(batch + 1);
            const int kv_start = kvbeg + kvblk;
            const int w_ploc = do_finish ? (nsplit > 0 ? pidx : -1) : pidx;
            const int w_kv_end = do_finish ? kvend : min(kv_start + remain, kvend);
            // the work slot at num_works is written every iteration (overwritten when not emitted)
            if (num_works >= flushed + kRingRows) flush(num_works);
            if (num_works < p.max_work) {
                if (lead) {
                    int4 *w = reinterpret_cast<int4 *>(s_ring) + ((num_works % kRingRows) << 1);
                    w[0] = make_int4(batch, w_ploc, qo_start, qo_end);
                    w[1] = make_int4(kv_start, w_kv_end, 0, qhr);
                }
                last_slot = num_works;
            } else {
                overflow = true;
            }
            const bool do_reduce = do_finish && nsplit > 0;
            const int num_splits = nsplit + 1;
            if (grt + 1 <= p.nb) put_ri(grt + 1, lri + num_splits);
            if (grt < p.nb) put_rfm(grt, qo_start, qo_end);
            if (do_reduce) {
                for (int s2 = 0; s2 < num_splits; ++s2) {
                    if (lri + s2 < p.max_split_tiles)
                        put_rpm(lri + s2, pidx - (nsplit - s2) * p.ql);
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
                put_wi(cid + 1, n_nworks);
            } else {
                const bool emit = remain > 0;
                n_nworks = emit ? num_works + 1 : num_works;
                pidx = emit ? pidx + p.ql : pidx;
                kvblk = emit ? kvblk + remain : kvblk;
                nsplit = emit ? nsplit + 1 : nsplit;
                put_wi(cid + 1, n_nworks);
                cid = cid + 1;
                cpos = cpos + 1 == nspk ? 0 : cpos + 1;
                remain = average + (cpos < reminder ? 1 : 0);
            }
            num_works = n_nworks;
            lri = n_lri;
            grt = n_grt;
        }
        if (cid < p.num_cu) cid += 1;
    };

    run_head(0);
    // Head 0 filled exactly bins [0, nspk): every later head then repeats its
    // schedule on bins [k*nspk, (k+1)*nspk) (quotas depend on cid % nspk only and
    // the per-head state restarts), shifted by k*W works and with its own head
    // range, and leaves the same reduce maps.  Replicate it in parallel; otherwise
    // run the remaining heads through the state machine.
    const int W = num_works;
    const bool replicated = p.nhk > 1 && cid == nspk && W <= kRingRows && flushed == 0;
    if (replicated) {
        wave_sync();
        for (int i = lane; i < (p.nhk - 1) * W; i += 64) {
            const int k = 1 + i / W, j = i - (k - 1) * W;
            const int row = k * W + j;
            if (row >= p.max_work) continue;
            const int32_t qhr = (int32_t)((((unsigned)(k + 1) * (unsigned)p.gqa) << 16) |
                                          (((unsigned)k * (unsigned)p.gqa) & 0xFFFFu));
            const int4 *src = reinterpret_cast<const int4 *>(s_ring) + (j << 1);
            int4 hi = src[1];
            hi.w = qhr;
            reinterpret_cast<int4 *>(p.work_info)[row * 2] = src[0];
            reinterpret_cast<int4 *>(p.work_info)[row * 2 + 1] = hi;
        }
        if (p.nhk * W > p.max_work) overflow = true;
        for (int i = lane; i < (p.nhk - 1) * nspk; i += 64) {  // work_indptr[k*nspk + j] for j in 1..nspk
            const int k = 1 + i / nspk, j = 1 + (i - (k - 1) * nspk);
            const int v = (wi_lds ? s_wi[j] : p.work_indptr[j]) + k * W;
            if (wi_lds) s_wi[k * nspk + j] = v;
            else p.work_indptr[k * nspk + j] = v;
        }
        wave_sync();
        cid = p.nhk * nspk;
        num_works = p.nhk * W;
    } else {
        for (int kh = 1; kh < p.nhk; ++kh) run_head(kh);
    }
    for (int i = cid; i <= p.num_cu; ++i) put_wi(i, num_works);
    for (int i = grt; i <= p.nb; ++i) put_ri(i, lri);
    // The ring still holds rows [flushed, num_works); slot num_works is copied too when
    // the last iteration wrote it without emitting it, as the reference leaves that row in
    // the buffer (a slot no iteration wrote holds stale LDS and stays out).  After a
    // replication the ring holds head 0's W rows only (its slot W would overwrite head
    // 1's first row).
    const int tail = last_slot == num_works ? num_works + 1 : num_works;
    flush(replicated ? W : min(tail, flushed + kRingRows));
    if (wi_lds)
        for (int i = lane; i <= p.num_cu; i += 64) p.work_indptr[i] = s_wi[i];
    if (red_lds) {
        for (int i = lane; i <= p.nb; i += 64) p.reduce_indptr[i] = s_ri[i];
        for (int i = lane; i < 2 * rfm_top; i += 64) p.reduce_final_map[i] = s_rfm[i];
    }
    if (rpm_lds)
        for (int i = lane; i < rpm_top; i += 64) p.reduce_partial_map[i] = s_rpm[i];
    wave_sync();
    if (lead && p.partial_count) p.partial_count[0] = lri;
    if (lead && overflow) p.work_indptr[0] = -1;
}

// Checks one schedule's arguments and fills its kernel parameters.
int meta_params(const pa_fp8_metadata_args *a, MetaParams &p) {
    if (!a) return PA_FP8_ERR_NULL_POINTER;
    if (a->num_batches < 0 || a->gqa <= 0 || a->num_heads_k <= 0 || a->num_cu <= 0 || a->query_length <= 0)
        return PA_FP8_ERR_SHAPE;
    if (a->num_cu % a->num_heads_k != 0) return PA_FP8_ERR_SHAPE;
    if (a->kv_granularity <= 0 || (a->kv_granularity & (a->kv_granularity - 1)) != 0) return PA_FP8_ERR_SHAPE;
    if (a->max_work < 0 || a->max_split_tiles < 0) return PA_FP8_ERR_SHAPE;
    // a buffer of no entries may be NULL (torch gives an empty tensor a NULL data
    // pointer): one bin per kv head leaves reduce_partial_map empty, and every
    // write to work_info, reduce_final_map and reduce_partial_map is bounded by
    // max_work, num_batches and max_split_tiles
    // a NULL seqlens_qo_indptr stands for b * query_length
    if (!a->seqlens_qo_indptr && (int64_t)a->num_batches * a->query_length > 0x7fffffffLL) return PA_FP8_ERR_SHAPE;
    if (!a->context_lens || !a->work_indptr || !a->reduce_indptr ||
        (!a->work_info && a->max_work > 0) || (!a->reduce_final_map && a->num_batches > 0) ||
        (!a->reduce_partial_map && a->max_split_tiles > 0))
        return PA_FP8_ERR_NULL_POINTER;
    if (a->bin_groups > 1) {
        if (a->bin_groups > 4) return PA_FP8_ERR_SHAPE;
        for (int g = 0; g < a->bin_groups; ++g)
            if (a->bin_weight[g] < 1 || a->bin_weight[g] > 1000) return PA_FP8_ERR_SHAPE;
    }
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
    p.partition_indptr = a->partition_indptr;
    p.uniform_context = a->uniform_context;
    p.partial_count = a->partial_count;
    p.bin_groups = a->bin_groups;
    for (int g = 0; g < 4; ++g) p.bin_weight[g] = a->bin_weight[g];
    p.pack = a->pack ? 1 : 0;
    return PA_FP8_OK;
}

}  // namespace

extern "C" int pa_fp8_metadata_multi(const pa_fp8_metadata_args *args, int32_t count, void *stream) {
    if (!args) return PA_FP8_ERR_NULL_POINTER;
    if (count < 1 || count > kMaxSchedules) return PA_FP8_ERR_SHAPE;
    MetaSchedules sched = {};
    for (int i = 0; i < count; ++i) {
        const int st = meta_params(&args[i], sched.p[i]);
        if (st != PA_FP8_OK) return st;
    }
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(pa_metadata_par_kernel, dim3(count), dim3(kParThreads), 0, s, sched);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? PA_FP8_OK : PA_FP8_ERR_HIP + (int)err;
}

extern "C" int pa_fp8_metadata_v1(const pa_fp8_metadata_args *a, void *stream) {
    return pa_fp8_metadata_multi(a, 1, stream);
}
