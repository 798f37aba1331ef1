// C ABI of the gfx950 FP8-KV paged-attention decode (include/pa_fp8.h) and the
// two merges of split work: the log-sum-exp reduce of the split-context partials
// (pa_lse_reduce_kernel) and the merge of split worklist partials
// (pa_reduce_v1_*_kernel, the role of aiter's pa_reduce_v1).  The decode kernels
// themselves are in pa_decode_kernels.h, built per head dim in pa_decode_hd.hip.
#include <mutex>

#include "pa_decode_params.h"
#include "pa_fp8.h"

using namespace pa;

namespace {

// ---------------------------------------------------------------- static scratch
// The partials of pa_fp8_decode_partitions_noalloc: a file-scope device array of
// PA_FP8_NOALLOC_SCRATCH_BYTES, which every GPU the library runs on holds until
// the process ends.  Host code must not pass `scratch` itself to a kernel (in host
// code the name is a host-side stand-in, not a device address): its device
// address on each device is looked up once, with that device current, and kept.
__device__ __align__(256) uint8_t scratch[PA_FP8_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t *g_scratch_ptr[kMaxDevices];  // device address of `scratch` on each device, nullptr until looked up

// The device address of `scratch` on device dev (looked up on the first call for dev).
int scratch_on(int dev, uint8_t **out) {
    if (dev < 0 || dev >= kMaxDevices) return PA_FP8_ERR_SHAPE;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        int cur = -1;
        hipError_t e = hipGetDevice(&cur);
        if (e != hipSuccess) return PA_FP8_ERR_HIP + (int)e;
        if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return PA_FP8_ERR_HIP + (int)e;
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (cur != dev) {
            const hipError_t e2 = hipSetDevice(cur);
            if (e == hipSuccess) e = e2;
        }
        if (e != hipSuccess) return PA_FP8_ERR_HIP + (int)e;
        if (!ptr) return PA_FP8_ERR_NULL_POINTER;
        g_scratch_ptr[dev] = static_cast<uint8_t *>(ptr);
    }
    *out = g_scratch_ptr[dev];
    return PA_FP8_OK;
}

constexpr int64_t align256(int64_t n) { return (n + 255) / 256 * 256; }

constexpr int kMaxHeadDim = 256;

struct ReduceParams {
    void *out;
    const float *es;
    const float *ml;
    const uint16_t *to;
    int64_t s_o_seq, s_o_len, s_o_head, s_o_group;
    int64_t s_es_seq, s_es_head, s_es_part;
    int64_t s_to_seq, s_to_head, s_to_part, s_to_group;
    int32_t g, max_parts, head_dim;
    int32_t eqgs;        // query rows per (sequence, kv head): ql * g
    int32_t rpw;         // rows per wave
    int32_t row_groups;  // workgroups per (sequence, kv head): ceil(eqgs / (waves per workgroup * rpw))
};

struct ReduceV1Params {
    void *out;
    float *final_lse;
    const float *po;
    const float *pl;
    const int32_t *reduce_indptr;
    const int32_t *final_map;
    const int32_t *partial_map;
    int64_t s_po_row, s_po_head, s_pl_row, s_pl_head, s_out_row, s_out_head, s_lse_row, s_lse_head;
    int32_t num_groups, num_heads, max_qlen, partial_rows, output_rows, partial_map_len, out_dtype, head_dim;
};

__device__ __forceinline__ void store2(void *out, int out_dtype, int64_t off, float a0, float a1) {
    if (out_dtype == PA_FP8_F32) {
        *reinterpret_cast<float2 *>(reinterpret_cast<float *>(out) + off) = make_float2(a0, a1);
    } else {
        const uint32_t pk = out_dtype == PA_FP8_F16
                                ? uint32_t(f32_to_f16_bits(a0)) | (uint32_t(f32_to_f16_bits(a1)) << 16)
                                : uint32_t(f32_to_bf16_bits(a0)) | (uint32_t(f32_to_bf16_bits(a1)) << 16);
        *reinterpret_cast<uint32_t *>(reinterpret_cast<uint16_t *>(out) + off) = pk;
    }
}

// Merge of the partials of one (reduce group, query row, head) per wave, four
// waves per workgroup; lane owns head dims 2*lane, 2*lane+1 (+128 for the second
// block of a head dim above 128).  Lane j first loads the log-sum-exp of partial j
// (all partials in parallel), the wave forms LSE = log sum_j exp(lse_j) and the
// weights exp(lse_j - LSE), and the partial rows are then summed four at a time
// with the weights and row indices broadcast from the lanes that hold them.
__global__ __launch_bounds__(256) void pa_reduce_v1_kernel(const ReduceV1Params p) {
    const int lane = threadIdx.x & 63;
    const int grp = blockIdx.x;
    const int row = blockIdx.y * 4 + (threadIdx.x >> 6);  // (qi, head) = (row / heads, row % heads)
    const int qi = row / p.num_heads, hd = row - qi * p.num_heads;
    const int j0 = max(p.reduce_indptr[grp], 0);
    const int j1 = min(p.reduce_indptr[grp + 1], p.partial_map_len);
    if (j0 >= j1 || qi >= p.max_qlen) return;
    const int qo_start = p.final_map[2 * grp];
    const int qo_end = p.final_map[2 * grp + 1];
    if (qi >= qo_end - qo_start || qo_start < 0 || qo_start + qi >= p.output_rows) return;
    const int np = j1 - j0;

    // pass 1: max and exp-sum of the partials' log-sum-exps (64 per lane round)
    float mloc = -INFINITY;
    for (int j = lane; j < np; j += 64) {
        const int r = p.partial_map[j0 + j] + qi;
        if (r >= 0 && r < p.partial_rows) mloc = fmaxf(mloc, p.pl[r * p.s_pl_row + hd * p.s_pl_head]);
    }
#pragma unroll
    for (int sh = 32; sh >= 1; sh >>= 1) mloc = fmaxf(mloc, shfl_xor_f(mloc, sh));
    const float Ms = mloc == -INFINITY ? 0.0f : mloc;
    float wl = 0.f;
    for (int j = lane; j < np; j += 64) {
        const int r = p.partial_map[j0 + j] + qi;
        if (r >= 0 && r < p.partial_rows) wl += fast_exp2((p.pl[r * p.s_pl_row + hd * p.s_pl_head] - Ms) * kLog2e);
    }
#pragma unroll
    for (int sh = 32; sh >= 1; sh >>= 1) wl += shfl_xor_f(wl, sh);
    const float inv = wl > 0.f ? 1.0f / wl : 0.0f;

    // pass 2: weighted sum of the partial rows, 64 partials per round, per block of
    // 128 head dims
    const int64_t orow = qo_start + qi;
    for (int db = 0; db < p.head_dim; db += 128) {
        const int d = db + 2 * lane;
        const bool live_d = d < p.head_dim;
        float a0 = 0.f, a1 = 0.f;
        for (int c0 = 0; c0 < np; c0 += 64) {
            const int j = c0 + lane;
            int r = -1;
            float w = 0.f;
            if (j < np) {
                r = p.partial_map[j0 + j] + qi;
                if (r >= 0 && r < p.partial_rows)
                    w = fast_exp2((p.pl[r * p.s_pl_row + hd * p.s_pl_head] - Ms) * kLog2e) * inv;
                else
                    r = -1;
            }
            const int n = min(64, np - c0);
            for (int k = 0; k < n; k += 4) {
                float2 v[4];
                float wk[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int src = min(k + u, n - 1);
                    wk[u] = k + u < n ? __shfl(w, src, 64) : 0.f;
                    const int rk = __shfl(r, src, 64);
                    v[u] = (wk[u] != 0.f && rk >= 0 && live_d)
                               ? *reinterpret_cast<const float2 *>(p.po + rk * p.s_po_row + hd * p.s_po_head + d)
                               : make_float2(0.f, 0.f);
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    a0 += wk[u] * v[u].x;
                    a1 += wk[u] * v[u].y;
                }
            }
        }
        if (live_d) store2(p.out, p.out_dtype, orow * p.s_out_row + hd * p.s_out_head + d, a0, a1);
    }
    if (p.final_lse != nullptr && lane == 0)
        p.final_lse[orow * p.s_lse_row + hd * p.s_lse_head] = wl > 0.f ? Ms + __logf(wl) : -INFINITY;
}

// The same merge with 16-byte accesses: one workgroup per (reduce group, query
// row, 8 heads), thread t owning dims 4*(t%32) .. +3 (and 128 above them for the
// second of NB 128-dim blocks) of head 8*blockIdx.z + t/32.  The partial rows of a
// group are a uniform list (scalar loads); each thread then issues its
// log-sum-exp loads and row loads together, so a group costs two dependent memory
// round trips.  Partials are merged kRedBatch at a time when a group has more.
constexpr int kRedBatch = 8;

template <int NB>
__global__ __launch_bounds__(256) void pa_reduce_v1_rows_kernel(const ReduceV1Params p) {
    const int grp = blockIdx.x, qi = blockIdx.y;
    const int hd = blockIdx.z * 8 + (threadIdx.x >> 5);
    const int d0 = (threadIdx.x & 31) * 4;
    const int j0 = max(p.reduce_indptr[grp], 0);
    const int j1 = min(p.reduce_indptr[grp + 1], p.partial_map_len);
    if (j0 >= j1 || qi >= p.max_qlen || hd >= p.num_heads) return;
    const int qo_start = p.final_map[2 * grp];
    const int qo_end = p.final_map[2 * grp + 1];
    if (qi >= qo_end - qo_start || qo_start < 0 || qo_start + qi >= p.output_rows) return;
    const int np = j1 - j0;
    bool live[NB];
#pragma unroll
    for (int k = 0; k < NB; ++k) live[k] = d0 + 128 * k < p.head_dim;
    auto row_at = [&](int r, int k) {
        return live[k] ? *reinterpret_cast<const float4 *>(p.po + r * p.s_po_row + hd * p.s_po_head + d0 + 128 * k)
                       : make_float4(0.f, 0.f, 0.f, 0.f);
    };

    // first batch of rows and every log-sum-exp, issued before any is used
    float lse[kRedBatch];
    float4 v[kRedBatch][NB];
    int rr[kRedBatch];
#pragma unroll
    for (int j = 0; j < kRedBatch; ++j) {
        const int r = j < np ? p.partial_map[j0 + j] + qi : -1;
        rr[j] = (r >= 0 && r < p.partial_rows) ? r : -1;
        lse[j] = rr[j] >= 0 ? p.pl[rr[j] * p.s_pl_row + hd * p.s_pl_head] : -INFINITY;
#pragma unroll
        for (int k = 0; k < NB; ++k) v[j][k] = rr[j] >= 0 ? row_at(rr[j], k) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float mloc = -INFINITY;
#pragma unroll
    for (int j = 0; j < kRedBatch; ++j) mloc = fmaxf(mloc, lse[j]);
    for (int j = kRedBatch; j < np; ++j) {
        const int r = p.partial_map[j0 + j] + qi;
        if (r >= 0 && r < p.partial_rows) mloc = fmaxf(mloc, p.pl[r * p.s_pl_row + hd * p.s_pl_head]);
    }
    const float Ms = mloc == -INFINITY ? 0.0f : mloc;
    float wl = 0.f;
#pragma unroll
    for (int j = 0; j < kRedBatch; ++j) {
        lse[j] = rr[j] >= 0 ? fast_exp2((lse[j] - Ms) * kLog2e) : 0.f;  // now the weight
        wl += lse[j];
    }
    for (int j = kRedBatch; j < np; ++j) {
        const int r = p.partial_map[j0 + j] + qi;
        if (r >= 0 && r < p.partial_rows) wl += fast_exp2((p.pl[r * p.s_pl_row + hd * p.s_pl_head] - Ms) * kLog2e);
    }
    const float inv = wl > 0.f ? 1.0f / wl : 0.0f;
    float4 a[NB];
#pragma unroll
    for (int k = 0; k < NB; ++k) a[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    auto accumulate = [&](float w, const float4 (&vj)[NB]) {
#pragma unroll
        for (int k = 0; k < NB; ++k) {
            a[k].x += w * vj[k].x;
            a[k].y += w * vj[k].y;
            a[k].z += w * vj[k].z;
            a[k].w += w * vj[k].w;
        }
    };
#pragma unroll
    for (int j = 0; j < kRedBatch; ++j) accumulate(lse[j] * inv, v[j]);
    for (int jb = kRedBatch; jb < np; jb += kRedBatch) {
#pragma unroll
        for (int j = 0; j < kRedBatch; ++j) {
            const int r = jb + j < np ? p.partial_map[j0 + jb + j] + qi : -1;
            rr[j] = (r >= 0 && r < p.partial_rows) ? r : -1;
            lse[j] = rr[j] >= 0 ? p.pl[rr[j] * p.s_pl_row + hd * p.s_pl_head] : -INFINITY;
#pragma unroll
            for (int k = 0; k < NB; ++k) v[j][k] = rr[j] >= 0 ? row_at(rr[j], k) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int j = 0; j < kRedBatch; ++j) accumulate(rr[j] >= 0 ? fast_exp2((lse[j] - Ms) * kLog2e) * inv : 0.f, v[j]);
    }
    const int64_t orow = qo_start + qi;
#pragma unroll
    for (int k = 0; k < NB; ++k) {
        if (!live[k]) continue;
        const int64_t off = orow * p.s_out_row + hd * p.s_out_head + d0 + 128 * k;
        if (p.out_dtype == PA_FP8_F32) {
            *reinterpret_cast<float4 *>(reinterpret_cast<float *>(p.out) + off) = a[k];
        } else {
            const bool f16 = p.out_dtype == PA_FP8_F16;
            const uint32_t lo = f16 ? uint32_t(f32_to_f16_bits(a[k].x)) | (uint32_t(f32_to_f16_bits(a[k].y)) << 16)
                                    : uint32_t(f32_to_bf16_bits(a[k].x)) | (uint32_t(f32_to_bf16_bits(a[k].y)) << 16);
            const uint32_t hi = f16 ? uint32_t(f32_to_f16_bits(a[k].z)) | (uint32_t(f32_to_f16_bits(a[k].w)) << 16)
                                    : uint32_t(f32_to_bf16_bits(a[k].z)) | (uint32_t(f32_to_bf16_bits(a[k].w)) << 16);
            *reinterpret_cast<uint2 *>(reinterpret_cast<uint16_t *>(p.out) + off) = make_uint2(lo, hi);
        }
    }
    if (p.final_lse != nullptr && d0 == 0)
        p.final_lse[orow * p.s_lse_row + hd * p.s_lse_head] = wl > 0.f ? Ms + __logf(wl) : -INFINITY;
}

// Log-sum-exp merge of the P partials of each (sequence, kv head, query row)
// (kernels/pa_decode_swa.py:954-1130): one wave merges p.rpw consecutive rows
// (lse_merge_rows, their loads in flight together; R = p.rpw, 1 or kReduceMaxRows),
// lane owning head dims 2*lane and 2*lane+1 of each of the NB 128-dim blocks.  A workgroup holds kReduceWaves such waves of one
// (sequence, kv head), and consecutive workgroups hold consecutive rows (grid x =
// sequence * row groups + row group), so the workgroups resident together read
// neighbouring pieces of each slot's partial block.  rpw > 1 when the rows outnumber
// what the GPU holds at once: fewer waves, each with several rows' loads in flight.
constexpr int kReduceWaves = 4;
constexpr int kReduceMaxRows = 2;  // rows per wave, at most
// waves the GPU keeps resident at once for this kernel, about (256 CUs x 32)
constexpr int64_t kReduceResidentWaves = 8192;
template <int OUT, int NB, int R>
__global__ __launch_bounds__(kReduceWaves * 64) void pa_lse_reduce_kernel(const ReduceParams p) {
    const int lane = threadIdx.x & 63;
    const int b = blockIdx.x / p.row_groups, h = blockIdx.y;
    const int r0 = ((blockIdx.x - b * p.row_groups) * kReduceWaves + (threadIdx.x >> 6)) * p.rpw;
    if (r0 >= p.eqgs) return;  // the last group's spare waves (no barrier follows)
    const int nrows = min(R, p.eqgs - r0);
    const float *es = p.es + b * p.s_es_seq + h * p.s_es_head + r0;
    const float *ml = p.ml + b * p.s_es_seq + h * p.s_es_head + r0;
    const uint16_t *to = p.to + b * p.s_to_seq + h * p.s_to_head + r0 * p.s_to_group;
    bool live[NB];
#pragma unroll
    for (int k = 0; k < NB; ++k) live[k] = 2 * lane + 128 * k < p.head_dim;
    float a0[R][NB], a1[R][NB];
    lse_merge_rows<NB, R>(es, ml, to, 1, p.s_to_group, p.s_es_part, p.s_to_part, p.max_parts, p.head_dim, lane,
                          nrows, a0, a1);
#pragma unroll
    for (int q = 0; q < R; ++q) {
        if (q >= nrows) break;
        const int r = r0 + q;
        const int qi = r / p.g, gi = r - (r / p.g) * p.g;
        const int64_t off = b * p.s_o_seq + qi * p.s_o_len + h * p.s_o_head + gi * p.s_o_group + 2 * lane;
#pragma unroll
        for (int k = 0; k < NB; ++k) {
            if (!live[k]) continue;
            if constexpr (OUT == PA_FP8_F32) {
                float *o = reinterpret_cast<float *>(p.out) + off + 128 * k;
                *reinterpret_cast<float2 *>(o) = make_float2(a0[q][k], a1[q][k]);
            } else if constexpr (OUT == PA_FP8_F16) {
                uint16_t *o = reinterpret_cast<uint16_t *>(p.out) + off + 128 * k;
                *reinterpret_cast<uint32_t *>(o) =
                    uint32_t(f32_to_f16_bits(a0[q][k])) | (uint32_t(f32_to_f16_bits(a1[q][k])) << 16);
            } else {
                uint16_t *o = reinterpret_cast<uint16_t *>(p.out) + off + 128 * k;
                *reinterpret_cast<uint32_t *>(o) =
                    uint32_t(f32_to_bf16_bits(a0[q][k])) | (uint32_t(f32_to_bf16_bits(a1[q][k])) << 16);
            }
        }
    }
}

// The instance for the head dim's 128-dim blocks (two: above 128) and the rows per wave.
template <int OUT>
void launch_lse_reduce(bool two, bool many, dim3 grid, dim3 block, hipStream_t s, const ReduceParams &p) {
    if (two && many) hipLaunchKernelGGL((pa_lse_reduce_kernel<OUT, 2, kReduceMaxRows>), grid, block, 0, s, p);
    else if (two) hipLaunchKernelGGL((pa_lse_reduce_kernel<OUT, 2, 1>), grid, block, 0, s, p);
    else if (many) hipLaunchKernelGGL((pa_lse_reduce_kernel<OUT, 1, kReduceMaxRows>), grid, block, 0, s, p);
    else hipLaunchKernelGGL((pa_lse_reduce_kernel<OUT, 1, 1>), grid, block, 0, s, p);
}

bool aligned16(const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

int log2_pow2(int v) {
    if (v <= 0 || (v & (v - 1)) != 0) return -1;
    int l = 0;
    while ((1 << l) < v) ++l;
    return l;
}

bool decode_head_dim(int d) { return d == 64 || d == 128 || d == 192 || d == 256; }

hipError_t run_partition(int d, const DecodeParams &p, bool pt, bool v4, int mtp, int waves, dim3 grid,
                         hipStream_t s) {
    switch (d) {
    case 64: return dispatch_partition<64>(p, pt, v4, mtp, waves, grid, s);
    case 192: return dispatch_partition<192>(p, pt, v4, mtp, waves, grid, s);
    case 256: return dispatch_partition<256>(p, pt, v4, mtp, waves, grid, s);
    default: return dispatch_partition<128>(p, pt, v4, mtp, waves, grid, s);
    }
}

hipError_t run_worklist(int d, const WorklistParams &w, bool pt, bool v4, int mtp, dim3 grid, hipStream_t s) {
    switch (d) {
    case 64: return dispatch_worklist<64>(w, pt, v4, mtp, grid, s);
    case 192: return dispatch_worklist<192>(w, pt, v4, mtp, grid, s);
    case 256: return dispatch_worklist<256>(w, pt, v4, mtp, grid, s);
    default: return dispatch_worklist<128>(w, pt, v4, mtp, grid, s);
    }
}

}  // namespace

extern "C" {

int pa_fp8_abi_version(void) { return PA_FP8_ABI_VERSION; }

const char *pa_fp8_status_string(int status) {
    switch (status) {
    case PA_FP8_OK: return "ok";
    case PA_FP8_ERR_NULL_POINTER: return "a required pointer is NULL";
    case PA_FP8_ERR_HEAD_DIM:
        return "unsupported head_dim (decode: 64, 128, 192 or 256; KV-cache writer: a multiple of 16 up to 1024)";
    case PA_FP8_ERR_BLOCK_SIZE: return "block_size must be a power of two >= 16";
    case PA_FP8_ERR_GROUP: return "query_length * query_group_size must be in 1..65535";
    case PA_FP8_ERR_SHAPE: return "a size, stride or alignment is out of range";
    case PA_FP8_ERR_DTYPE: return "unsupported dtype";
    case PA_FP8_ERR_PARTITIONS: return "max_context_partition_num must be in 1..65535";
    case PA_FP8_ERR_WORKLIST: return "worklist buffers too small for the schedule";
    case PA_FP8_ERR_LAYOUT: return "KV-cache layout or format not valid for these sizes";
    case PA_FP8_ERR_SCRATCH:
        return "partials exceed the static scratch of pa_fp8_decode_partitions_noalloc (32 MiB); "
               "use pa_fp8_decode_partitions with caller-allocated partials";
    default: break;
    }
    if (status >= PA_FP8_ERR_HIP) return hipGetErrorString((hipError_t)(status - PA_FP8_ERR_HIP));
    return "unknown status";
}

int pa_fp8_decode_partitions(const pa_fp8_decode_args *a, void *stream) {
    if (!a) return PA_FP8_ERR_NULL_POINTER;
    if (a->batch_size < 0 || a->num_kv_heads <= 0 || a->query_group_size <= 0 || a->query_length <= 0)
        return PA_FP8_ERR_SHAPE;
    if (!decode_head_dim(a->head_dim)) return PA_FP8_ERR_HEAD_DIM;
    const int bs_log2 = log2_pow2(a->block_size);
    if (bs_log2 < 4) return PA_FP8_ERR_BLOCK_SIZE;
    const int64_t eqgs64 = (int64_t)a->query_length * a->query_group_size;
    if (eqgs64 < 1 || eqgs64 > 65535) return PA_FP8_ERR_GROUP;
    const int eqgs = (int)eqgs64;
    if (a->max_context_partition_num < 1 || a->max_context_partition_num > 65535) return PA_FP8_ERR_PARTITIONS;
    if (a->query_dtype != PA_FP8_BF16 && a->query_dtype != PA_FP8_F16) return PA_FP8_ERR_DTYPE;
    if (a->num_kv_heads > 65535 || a->sliding_window < 0) return PA_FP8_ERR_SHAPE;
    if (a->value_layout != PA_FP8_V_TRANS && a->value_layout != PA_FP8_V_4D) return PA_FP8_ERR_LAYOUT;
    if (a->waves_per_slot != 0 && a->waves_per_slot != 1 && a->waves_per_slot != 2 && a->waves_per_slot != 4 &&
        a->waves_per_slot != 8)
        return PA_FP8_ERR_SHAPE;
    // chained slots: one 16-row group, head_dim 128, the trans_v layout
    const int spw = a->slots_per_wave;
    const int wg_waves = a->waves_per_slot > 0 ? a->waves_per_slot : (spw > 0 ? 1 : 4);
    if (spw < 0 || spw > 65535) return PA_FP8_ERR_SHAPE;
    if (spw > 0 && (eqgs > 16 || a->head_dim != 128 || a->value_layout != PA_FP8_V_TRANS)) return PA_FP8_ERR_SHAPE;
    const int P = a->max_context_partition_num;
    const int64_t slots_per_wg = spw > 0 ? (int64_t)wg_waves * spw : 1;
    if (a->direct_output) {
        // several slots per sequence: only when one chained workgroup holds them all
        // (it merges its own partials, which the caller provides)
        if (P != 1 && (spw == 0 || slots_per_wg < P)) return PA_FP8_ERR_PARTITIONS;
        if (a->out_dtype != PA_FP8_BF16 && a->out_dtype != PA_FP8_F16 && a->out_dtype != PA_FP8_F32)
            return PA_FP8_ERR_DTYPE;
    }
    const bool partials = !a->direct_output || P > 1;
    const int chunks = (eqgs + kRowChunk - 1) / kRowChunk;
    if ((int64_t)a->batch_size * chunks > 0x7fffffff) return PA_FP8_ERR_SHAPE;
    if (a->batch_size == 0) return PA_FP8_OK;
    if (!a->query || !a->key_cache || !a->value_cache || !a->block_tables || !a->context_lengths || !a->key_scale ||
        !a->value_scale)
        return PA_FP8_ERR_NULL_POINTER;
    if (a->direct_output) {
        if (!a->output) return PA_FP8_ERR_NULL_POINTER;
        const int esz = a->out_dtype == PA_FP8_F32 ? 4 : 2;
        if ((reinterpret_cast<uintptr_t>(a->output) & 15) ||
            ((a->stride_o_seq | a->stride_o_len | a->stride_o_head | a->stride_o_group) * esz) & 15)
            return PA_FP8_ERR_SHAPE;
    }
    if (partials && (!a->exp_sums || !a->max_logits || !a->tmp_out)) return PA_FP8_ERR_NULL_POINTER;
    if (a->num_blocks <= 0 || a->max_blocks_per_seq <= 0) return PA_FP8_ERR_SHAPE;
    // 16-byte vector accesses: caches, query rows and partial rows must be 16-byte aligned
    if (!aligned16(a->key_cache) || !aligned16(a->value_cache) || !aligned16(a->query) ||
        (partials && !aligned16(a->tmp_out)))
        return PA_FP8_ERR_SHAPE;
    if ((a->stride_k_block | a->stride_k_head | a->stride_v_block | a->stride_v_head) & 15) return PA_FP8_ERR_SHAPE;
    if ((a->stride_q_seq | a->stride_q_head) & 7) return PA_FP8_ERR_SHAPE;
    if ((a->stride_to_seq | a->stride_to_head | a->stride_to_part | a->stride_to_group) & 7) return PA_FP8_ERR_SHAPE;
    if (a->per_token_kv) {
        if (!aligned16(a->key_scale) || !aligned16(a->value_scale)) return PA_FP8_ERR_SHAPE;
        if ((a->stride_ks_block | a->stride_ks_head) & 3) return PA_FP8_ERR_SHAPE;
    }

    DecodeParams p;
    p.exp_sums = a->exp_sums;
    p.max_logits = a->max_logits;
    p.tmp_out = reinterpret_cast<uint16_t *>(a->tmp_out);
    p.query = reinterpret_cast<const uint16_t *>(a->query);
    p.kc = a->key_cache;
    p.vc = a->value_cache;
    p.bt = a->block_tables;
    p.ctx = a->context_lengths;
    p.ks = a->key_scale;
    p.vs = a->value_scale;
    p.s_q_seq = a->stride_q_seq;
    p.s_q_head = a->stride_q_head;
    p.s_k_block = a->stride_k_block;
    p.s_k_head = a->stride_k_head;
    p.s_v_block = a->stride_v_block;
    p.s_v_head = a->stride_v_head;
    p.s_es_seq = a->stride_es_seq;
    p.s_es_head = a->stride_es_head;
    p.s_es_part = a->stride_es_part;
    p.s_to_seq = a->stride_to_seq;
    p.s_to_head = a->stride_to_head;
    p.s_to_part = a->stride_to_part;
    p.s_to_group = a->stride_to_group;
    p.s_bt_seq = a->stride_bt_seq;
    p.s_ks_block = a->per_token_kv ? a->stride_ks_block : 0;
    p.s_ks_head = a->per_token_kv ? a->stride_ks_head : 0;
    p.g = a->query_group_size;
    p.ql = a->query_length;
    p.eqgs = eqgs;
    p.bs_log2 = bs_log2;
    p.num_blocks = a->num_blocks;
    p.max_blocks = a->max_blocks_per_seq;
    p.max_parts = a->max_context_partition_num;
    p.sw = a->sliding_window;
    p.q_f16 = a->query_dtype == PA_FP8_F16;
    p.chunks = chunks;
    p.qk_scale = a->softmax_scale * kLog2e;
    p.direct = a->direct_output ? 1 : 0;
    p.out = a->output;
    p.s_o_seq = a->stride_o_seq;
    p.s_o_len = a->stride_o_len;
    p.s_o_head = a->stride_o_head;
    p.s_o_group = a->stride_o_group;
    p.out_dtype = a->out_dtype;
    p.spw = spw;
    // several workgroups per (sequence, kv head) of the partition kernel: spread each
    // sequence over the XCDs (slot_item)
    const unsigned zg = (unsigned)((P + slots_per_wg - 1) / slots_per_wg);
    p.spread = zg > 1 && spw == 0 ? 1 : 0;
    // a merging workgroup keeps a copy of its partials in LDS when they fit in 48 KiB
    // (then it reads LDS, not the rows it just stored): P rows of eqgs x (D bf16 + 2 f32)
    p.merge_lds = 0;
    if (a->direct_output && P > 1) {
        const int64_t bytes = (int64_t)P * eqgs * (2 * a->head_dim + 8);
        if (bytes <= 48 * 1024) p.merge_lds = (int32_t)bytes;
    }

    const dim3 grid(a->batch_size * chunks, a->num_kv_heads, zg);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int mtp = (min(eqgs, kRowChunk) + 15) / 16;
    const hipError_t err = run_partition(a->head_dim, p, a->per_token_kv != 0, a->value_layout == PA_FP8_V_4D, mtp,
                                         a->waves_per_slot, grid, s);
    return err == hipSuccess ? PA_FP8_OK : PA_FP8_ERR_HIP + (int)err;
}

int pa_fp8_decode_partitions_noalloc(const pa_fp8_decode_args *a, void *stream) {
    if (!a) return PA_FP8_ERR_NULL_POINTER;
    if (a->out_dtype != PA_FP8_BF16 && a->out_dtype != PA_FP8_F16 && a->out_dtype != PA_FP8_F32)
        return PA_FP8_ERR_DTYPE;
    pa_fp8_decode_args d = *a;
    if (a->max_context_partition_num == 1) {  // one slot per sequence: the kernel writes the output itself
        d.direct_output = 1;
        d.exp_sums = d.max_logits = nullptr;
        d.tmp_out = nullptr;
        return pa_fp8_decode_partitions(&d, stream);
    }
    if (a->batch_size < 0 || a->num_kv_heads <= 0 || a->query_group_size <= 0 || a->query_length <= 0 ||
        a->max_context_partition_num < 1 || !decode_head_dim(a->head_dim))
        return pa_fp8_decode_partitions(&d, stream);  // its own status for these
    const int64_t eqgs = (int64_t)a->query_length * a->query_group_size;
    const int64_t n = (int64_t)a->batch_size * a->num_kv_heads * a->max_context_partition_num * eqgs;
    const int64_t es_bytes = align256(n * 4);
    const int64_t to_bytes = align256(n * a->head_dim * 2);
    if (2 * es_bytes + to_bytes > PA_FP8_NOALLOC_SCRATCH_BYTES) return PA_FP8_ERR_SCRATCH;
    if (a->batch_size == 0) return PA_FP8_OK;
    if (!a->output) return PA_FP8_ERR_NULL_POINTER;
    int dev = -1;
    hipError_t e = stream ? hipStreamGetDevice(reinterpret_cast<hipStream_t>(stream), &dev) : hipGetDevice(&dev);
    if (e != hipSuccess) return PA_FP8_ERR_HIP + (int)e;
    uint8_t *base = nullptr;
    const int st = scratch_on(dev, &base);
    if (st != PA_FP8_OK) return st;
    // partials in the scratch: exp_sums, max_logits [B, Hkv, P, eqgs] f32, tmp_out [B, Hkv, P, eqgs, D] bf16
    const int64_t P = a->max_context_partition_num, D = a->head_dim;
    // a chained layout whose workgroups hold every slot of a sequence merges its own
    // partials (direct_output); otherwise the reduce below does
    const bool merged = a->direct_output != 0;
    d.direct_output = merged ? 1 : 0;
    d.exp_sums = reinterpret_cast<float *>(base);
    d.max_logits = reinterpret_cast<float *>(base + es_bytes);
    d.tmp_out = base + 2 * es_bytes;
    d.stride_es_seq = a->num_kv_heads * P * eqgs;
    d.stride_es_head = P * eqgs;
    d.stride_es_part = eqgs;
    d.stride_to_seq = a->num_kv_heads * P * eqgs * D;
    d.stride_to_head = P * eqgs * D;
    d.stride_to_part = eqgs * D;
    d.stride_to_group = D;
    int status = pa_fp8_decode_partitions(&d, stream);
    if (status != PA_FP8_OK || merged) return status;
    pa_fp8_reduce_args r = {};
    r.output = a->output;
    r.exp_sums = d.exp_sums;
    r.max_logits = d.max_logits;
    r.tmp_out = d.tmp_out;
    r.stride_o_seq = a->stride_o_seq;
    r.stride_o_len = a->stride_o_len;
    r.stride_o_head = a->stride_o_head;
    r.stride_o_group = a->stride_o_group;
    r.stride_es_seq = d.stride_es_seq;
    r.stride_es_head = d.stride_es_head;
    r.stride_es_part = d.stride_es_part;
    r.stride_to_seq = d.stride_to_seq;
    r.stride_to_head = d.stride_to_head;
    r.stride_to_part = d.stride_to_part;
    r.stride_to_group = d.stride_to_group;
    r.batch_size = a->batch_size;
    r.num_kv_heads = a->num_kv_heads;
    r.query_group_size = a->query_group_size;
    r.query_length = a->query_length;
    r.head_dim = a->head_dim;
    r.max_context_partition_num = a->max_context_partition_num;
    r.out_dtype = a->out_dtype;
    return pa_fp8_lse_reduce(&r, stream);
}

int pa_fp8_lse_reduce(const pa_fp8_reduce_args *a, void *stream) {
    if (!a) return PA_FP8_ERR_NULL_POINTER;
    if (a->batch_size < 0 || a->num_kv_heads <= 0 || a->query_group_size <= 0 || a->query_length <= 0)
        return PA_FP8_ERR_SHAPE;
    if (a->head_dim <= 0 || a->head_dim > kMaxHeadDim || (a->head_dim & 1)) return PA_FP8_ERR_HEAD_DIM;
    if (a->max_context_partition_num < 1) return PA_FP8_ERR_PARTITIONS;
    const int64_t eqgs = (int64_t)a->query_length * a->query_group_size;
    if (eqgs > 65535 || a->num_kv_heads > 65535) return PA_FP8_ERR_SHAPE;
    if (a->out_dtype != PA_FP8_BF16 && a->out_dtype != PA_FP8_F16 && a->out_dtype != PA_FP8_F32)
        return PA_FP8_ERR_DTYPE;
    if (a->batch_size == 0) return PA_FP8_OK;
    if (!a->output || !a->exp_sums || !a->max_logits || !a->tmp_out) return PA_FP8_ERR_NULL_POINTER;
    const int esz = a->out_dtype == PA_FP8_F32 ? 4 : 2;
    if ((reinterpret_cast<uintptr_t>(a->output) & (2 * esz - 1)) || (reinterpret_cast<uintptr_t>(a->tmp_out) & 3))
        return PA_FP8_ERR_SHAPE;
    if ((a->stride_o_seq | a->stride_o_len | a->stride_o_head | a->stride_o_group) & 1) return PA_FP8_ERR_SHAPE;
    if ((a->stride_to_seq | a->stride_to_head | a->stride_to_part | a->stride_to_group) & 1) return PA_FP8_ERR_SHAPE;

    ReduceParams p;
    p.out = a->output;
    p.es = a->exp_sums;
    p.ml = a->max_logits;
    p.to = reinterpret_cast<const uint16_t *>(a->tmp_out);
    p.s_o_seq = a->stride_o_seq;
    p.s_o_len = a->stride_o_len;
    p.s_o_head = a->stride_o_head;
    p.s_o_group = a->stride_o_group;
    p.s_es_seq = a->stride_es_seq;
    p.s_es_head = a->stride_es_head;
    p.s_es_part = a->stride_es_part;
    p.s_to_seq = a->stride_to_seq;
    p.s_to_head = a->stride_to_head;
    p.s_to_part = a->stride_to_part;
    p.s_to_group = a->stride_to_group;
    p.g = a->query_group_size;
    p.max_parts = a->max_context_partition_num;
    p.head_dim = a->head_dim;
    p.eqgs = (int)eqgs;
    // one row per wave while the rows fit in about two rounds of resident waves
    // (kReduceResidentWaves), else kReduceMaxRows rows per wave
    const int64_t rows = (int64_t)a->batch_size * a->num_kv_heads * eqgs;
    p.rpw = rows > 2 * kReduceResidentWaves ? kReduceMaxRows : 1;
    const int per_group = kReduceWaves * p.rpw;
    p.row_groups = (int)((eqgs + per_group - 1) / per_group);
    if ((int64_t)a->batch_size * p.row_groups > 0x7fffffffLL) return PA_FP8_ERR_SHAPE;
    const dim3 grid((unsigned)(a->batch_size * p.row_groups), a->num_kv_heads);
    const dim3 block(kReduceWaves * 64);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const bool two = a->head_dim > 128, many = p.rpw > 1;
    switch (a->out_dtype) {
    case PA_FP8_F32: launch_lse_reduce<PA_FP8_F32>(two, many, grid, block, s, p); break;
    case PA_FP8_F16: launch_lse_reduce<PA_FP8_F16>(two, many, grid, block, s, p); break;
    default: launch_lse_reduce<PA_FP8_BF16>(two, many, grid, block, s, p); break;
    }
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? PA_FP8_OK : PA_FP8_ERR_HIP + (int)err;
}

int pa_fp8_decode_worklist(const pa_fp8_worklist_args *a, void *stream) {
    if (!a) return PA_FP8_ERR_NULL_POINTER;
    if (a->batch_size < 0 || a->num_kv_heads <= 0 || a->query_group_size <= 0 || a->query_length <= 0)
        return PA_FP8_ERR_SHAPE;
    if (!decode_head_dim(a->head_dim)) return PA_FP8_ERR_HEAD_DIM;
    const int bs_log2 = log2_pow2(a->block_size);
    if (bs_log2 < 4) return PA_FP8_ERR_BLOCK_SIZE;
    const int64_t eqgs64 = (int64_t)a->query_length * a->query_group_size;
    if (eqgs64 < 1 || eqgs64 > 65535) return PA_FP8_ERR_GROUP;
    const int eqgs = (int)eqgs64;
    if (a->query_dtype != PA_FP8_BF16 && a->query_dtype != PA_FP8_F16) return PA_FP8_ERR_DTYPE;
    if (a->out_dtype != PA_FP8_BF16 && a->out_dtype != PA_FP8_F16 && a->out_dtype != PA_FP8_F32) return PA_FP8_ERR_DTYPE;
    if (a->value_layout != PA_FP8_V_TRANS && a->value_layout != PA_FP8_V_4D) return PA_FP8_ERR_LAYOUT;
    if (a->num_cu < 0 || a->max_work < 0 || a->partial_rows < 0 || a->output_rows < 0 || a->num_pages < 0)
        return PA_FP8_ERR_SHAPE;
    const int chunks = (eqgs + kRowChunk - 1) / kRowChunk;
    if ((int64_t)a->num_cu * chunks > 0x7fffffff) return PA_FP8_ERR_SHAPE;
    if (a->batch_size == 0 || a->num_cu == 0) return PA_FP8_OK;
    if (!a->output || !a->query || !a->key_cache || !a->value_cache || !a->context_lengths || !a->key_scale ||
        !a->value_scale || !a->work_indptr || !a->work_info || !a->kv_indptr || !a->partition_indptr)
        return PA_FP8_ERR_NULL_POINTER;
    if (a->num_pages > 0 && !a->kv_page_indices) return PA_FP8_ERR_NULL_POINTER;
    if (a->partial_rows > 0 && (!a->partial_output || !a->partial_lse)) return PA_FP8_ERR_NULL_POINTER;
    if (a->num_blocks <= 0) return PA_FP8_ERR_SHAPE;
    if (!aligned16(a->key_cache) || !aligned16(a->value_cache) || !aligned16(a->query) || !aligned16(a->output))
        return PA_FP8_ERR_SHAPE;
    if (a->partial_rows > 0 && (!aligned16(a->partial_output) || (a->stride_po_row & 3))) return PA_FP8_ERR_SHAPE;
    if ((a->stride_k_block | a->stride_k_head | a->stride_v_block | a->stride_v_head) & 15) return PA_FP8_ERR_SHAPE;
    if ((a->stride_q_seq | a->stride_q_head) & 7) return PA_FP8_ERR_SHAPE;
    const int esz = a->out_dtype == PA_FP8_F32 ? 4 : 2;
    if (((a->stride_out_seq | a->stride_out_head) * esz) & 15) return PA_FP8_ERR_SHAPE;
    if (a->per_token_kv) {
        if (!aligned16(a->key_scale) || !aligned16(a->value_scale)) return PA_FP8_ERR_SHAPE;
        if ((a->stride_ks_block | a->stride_ks_head) & 3) return PA_FP8_ERR_SHAPE;
    }

    WorklistParams w = {};
    DecodeParams &p = w.kv;
    p.query = reinterpret_cast<const uint16_t *>(a->query);
    p.kc = a->key_cache;
    p.vc = a->value_cache;
    p.ctx = a->context_lengths;
    p.ks = a->key_scale;
    p.vs = a->value_scale;
    p.s_q_seq = a->stride_q_seq;
    p.s_q_head = a->stride_q_head;
    p.s_k_block = a->stride_k_block;
    p.s_k_head = a->stride_k_head;
    p.s_v_block = a->stride_v_block;
    p.s_v_head = a->stride_v_head;
    p.s_ks_block = a->per_token_kv ? a->stride_ks_block : 0;
    p.s_ks_head = a->per_token_kv ? a->stride_ks_head : 0;
    p.g = a->query_group_size;
    p.ql = a->query_length;
    p.eqgs = eqgs;
    p.bs_log2 = bs_log2;
    p.num_blocks = a->num_blocks;
    p.max_parts = 1;
    p.sw = 0;
    p.q_f16 = a->query_dtype == PA_FP8_F16;
    p.chunks = chunks;
    p.qk_scale = a->softmax_scale * kLog2e;
    w.work_indptr = a->work_indptr;
    w.work_info = a->work_info;
    w.kv_page_indices = a->kv_page_indices;
    w.kv_indptr = a->kv_indptr;
    w.partition_indptr = a->partition_indptr;
    w.po = a->partial_output;
    w.pl = a->partial_lse;
    w.out = a->output;
    w.s_out_seq = a->stride_out_seq;
    w.s_out_head = a->stride_out_head;
    w.s_po_row = a->stride_po_row;
    w.s_pl_row = a->stride_pl_row;
    w.batch = a->batch_size;
    w.num_kv_heads = a->num_kv_heads;
    w.num_pages = a->num_pages;
    w.max_work = a->max_work;
    w.partial_rows = a->partial_rows;
    w.output_rows = a->output_rows;
    w.out_dtype = a->out_dtype;
    w.head_dim = a->head_dim;
    w.num_bins = a->num_cu;
    w.bin_groups = chunks == 1 && a->bin_groups > 1 && a->bin_groups <= 4 &&
                           a->num_cu % (a->bin_groups * a->num_kv_heads) == 0
                       ? a->bin_groups
                       : 1;

    const dim3 grid(a->num_cu * chunks);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int mtp = (min(eqgs, kRowChunk) + 15) / 16;
    const hipError_t err = run_worklist(a->head_dim, w, a->per_token_kv != 0, a->value_layout == PA_FP8_V_4D, mtp,
                                        grid, s);
    return err == hipSuccess ? PA_FP8_OK : PA_FP8_ERR_HIP + (int)err;
}

int pa_fp8_reduce_v1(const pa_fp8_reduce_v1_args *a, void *stream) {
    if (!a) return PA_FP8_ERR_NULL_POINTER;
    if (a->head_dim <= 0 || a->head_dim > kMaxHeadDim || (a->head_dim & 1)) return PA_FP8_ERR_HEAD_DIM;
    if (a->num_groups < 0 || a->num_heads <= 0 || a->num_heads > 65535 || a->max_qlen <= 0 || a->max_qlen > 65535 ||
        a->partial_rows < 0 || a->output_rows < 0 || a->partial_map_len < 0)
        return PA_FP8_ERR_SHAPE;
    if (a->out_dtype != PA_FP8_BF16 && a->out_dtype != PA_FP8_F16 && a->out_dtype != PA_FP8_F32) return PA_FP8_ERR_DTYPE;
    // nothing to merge (an empty partial tensor also reports a NULL data pointer)
    if (a->num_groups == 0 || a->partial_map_len == 0 || a->partial_rows == 0) return PA_FP8_OK;
    if (!a->output || !a->partial_output || !a->partial_lse || !a->reduce_indptr || !a->reduce_final_map ||
        !a->reduce_partial_map)
        return PA_FP8_ERR_NULL_POINTER;
    const int esz = a->out_dtype == PA_FP8_F32 ? 4 : 2;
    if ((reinterpret_cast<uintptr_t>(a->output) & (2 * esz - 1)) || (reinterpret_cast<uintptr_t>(a->partial_output) & 7))
        return PA_FP8_ERR_SHAPE;
    if (((a->stride_out_row | a->stride_out_head) & 1) || ((a->stride_po_row | a->stride_po_head) & 1))
        return PA_FP8_ERR_SHAPE;

    ReduceV1Params p;
    p.out = a->output;
    p.final_lse = a->final_lse;
    p.po = a->partial_output;
    p.pl = a->partial_lse;
    p.reduce_indptr = a->reduce_indptr;
    p.final_map = a->reduce_final_map;
    p.partial_map = a->reduce_partial_map;
    p.s_po_row = a->stride_po_row;
    p.s_po_head = a->stride_po_head;
    p.s_pl_row = a->stride_pl_row;
    p.s_pl_head = a->stride_pl_head;
    p.s_out_row = a->stride_out_row;
    p.s_out_head = a->stride_out_head;
    p.s_lse_row = a->stride_lse_row;
    p.s_lse_head = a->stride_lse_head;
    p.num_groups = a->num_groups;
    p.num_heads = a->num_heads;
    p.max_qlen = a->max_qlen;
    p.partial_rows = a->partial_rows;
    p.output_rows = a->output_rows;
    p.partial_map_len = a->partial_map_len;
    p.out_dtype = a->out_dtype;
    p.head_dim = a->head_dim;
    // 16-byte path: 16-byte aligned partial rows and heads, 4-element aligned output
    // heads, whole 4-dim pieces
    const bool vec = (reinterpret_cast<uintptr_t>(a->partial_output) & 15) == 0 &&
                     ((a->stride_po_row | a->stride_po_head) & 3) == 0 &&
                     (reinterpret_cast<uintptr_t>(a->output) & (4 * esz - 1)) == 0 &&
                     ((a->stride_out_row | a->stride_out_head) & 3) == 0 && (a->head_dim & 3) == 0;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (vec) {
        const dim3 grid(a->num_groups, a->max_qlen, (a->num_heads + 7) / 8);
        if (a->head_dim > 128)
            hipLaunchKernelGGL(pa_reduce_v1_rows_kernel<2>, grid, dim3(256), 0, s, p);
        else
            hipLaunchKernelGGL(pa_reduce_v1_rows_kernel<1>, grid, dim3(256), 0, s, p);
    } else {
        const int64_t rows = (int64_t)a->num_heads * a->max_qlen;  // (qi, head) rows of a group, four per workgroup
        if ((rows + 3) / 4 > 65535) return PA_FP8_ERR_SHAPE;
        hipLaunchKernelGGL(pa_reduce_v1_kernel, dim3(a->num_groups, (rows + 3) / 4), dim3(256), 0, s, p);
    }
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? PA_FP8_OK : PA_FP8_ERR_HIP + (int)err;
}

}  // extern "C"
