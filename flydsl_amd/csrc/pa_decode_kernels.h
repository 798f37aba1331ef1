// gfx950 split-context and persistent FP8-KV paged-attention decode kernels,
// templated on the head dim D (a multiple of 64).  pa_decode_hd.hip builds them
// for one D per object.
//
// Work decomposition of the split-context kernel (grid = (batch * row chunks,
// kv_heads, partition slots), one workgroup per slot and chunk of up to 64 query
// rows, NW waves per workgroup):
//   * slot z of sequence b covers the 256-token partitions [z*pps, min((z+1)*pps, T))
//     with T = ceil(ctx/256), pps = ceil(T/P) (kernels/pa_decode_fp8.py:2311-2320);
//     with a sliding window the partitions start at tile max(ctx-ql-sw,0)/256
//     (kernels/pa_decode_swa.py:1359-1368) and the first window tile is trimmed
//     to the 16-token group holding the window start.
//   * the slot's tokens are cut into 64-token steps (4 groups of 16 tokens); wave w
//     takes steps w, w+NW, ... and runs its own online softmax; the waves merge
//     through LDS at the end and write one partial (exp_sum, max_logit, bf16 out).
//
// Per step a lane issues D/16 16-byte K loads and D/16 16-byte V loads (the
// 64 D bytes of each a wave consumes per step); the next step is prefetched while
// the current one is computed.  fp8 e4m3fn is converted exactly to bf16 in
// registers (v_cvt_scalef32_pk_bf16_fp8) and both products run on
// v_mfma_f32_16x16x32_bf16:
//   QK : C[token][qrow] = sum_d K[token][d] Q[qrow][d]   (4 tiles x D/32 k-steps)
//   PV : C[dim][qrow]   = sum_t V[t][dim] P[qrow][t]     (D/16 dim tiles x 2 k-steps)
// Lane (l16, kg) holds head dims [D/4 kg, D/4 (kg+1)) of its K token and query
// row.  QK tile jt, row 4*kg+i holds token 16*kg + 4*jt + i of the step, so the QK
// output lane (qrow, kg) owns exactly the 16 tokens of group kg -- the tokens its
// PV operand needs (one 16-byte V row of group kg) -- and P goes from the QK
// accumulators to the PV MFMA without any cross-lane movement.
//
// V rows: 16 consecutive tokens of one head dim are 16 contiguous bytes in both
// value-cache layouts the reference defines (trans_v [nb, Hkv, bs/16, D, 16] and
// 4-D [nb, Hkv, D, bs]); they differ only in the byte strides between head dims
// (16 / bs) and between 16-token groups (16 D / 16) of a (block, kv head) tile.
// The kernels take the layout as a template flag (V4), so the trans_v code keeps
// immediate load offsets.
#pragma once

#include "pa_decode_params.h"
#include "pa_fp8.h"

namespace pa {
namespace {

// N consecutive values to the output tensor at element offset off, converted to
// out_dtype (bf16 / f16 round to nearest even, f32 stored as is).
template <int N>
__device__ __forceinline__ void store_out(void *out, int out_dtype, int64_t off, const float (&v)[N]) {
    if (out_dtype == PA_FP8_F32) {
        float *dst = reinterpret_cast<float *>(out) + off;
#pragma unroll
        for (int j = 0; j < N; j += 4) *reinterpret_cast<float4 *>(dst + j) = make_float4(v[j], v[j + 1], v[j + 2], v[j + 3]);
        return;
    }
    uint32_t pk[N / 2];
#pragma unroll
    for (int j = 0; j < N; j += 2) {
        if (out_dtype == PA_FP8_F16)
            pk[j / 2] = uint32_t(f32_to_f16_bits(v[j])) | (uint32_t(f32_to_f16_bits(v[j + 1])) << 16);
        else
            pk[j / 2] = uint32_t(f32_to_bf16_bits(v[j])) | (uint32_t(f32_to_bf16_bits(v[j + 1])) << 16);
    }
    uint16_t *dst = reinterpret_cast<uint16_t *>(out) + off;
    if constexpr (N == 8) *reinterpret_cast<uint4 *>(dst) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    else *reinterpret_cast<uint2 *>(dst) = make_uint2(pk[0], pk[1]);
}

// Where the partition kernel puts the result of one slot: the bf16 partial row
// plus (exp_sum, max_logit), or (final: one slot per sequence) the final row
// out[b, qi, h, gi, :].
struct SlotSink {
    const DecodeParams &p;
    uint16_t *to;
    float *es;
    float *ml;
    int b, h;
    bool final_row;
    // LDS copy of the slot's partial for a merge inside the workgroup (rows of kHeadDim
    // bf16, then exp_sum / max_logit per row); null when unused
    uint16_t *lto = nullptr;
    float *les = nullptr, *lml = nullptr;

    template <int N>
    __device__ __forceinline__ void row(int r, int d0, const float (&v)[N]) const {
        if (!final_row) {
            uint32_t pk[N / 2];
#pragma unroll
            for (int j = 0; j < N; j += 2)
                pk[j / 2] = uint32_t(f32_to_bf16_bits(v[j])) | (uint32_t(f32_to_bf16_bits(v[j + 1])) << 16);
            uint16_t *dst = to + r * p.s_to_group + d0;
            if constexpr (N == 8) *reinterpret_cast<uint4 *>(dst) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
            else *reinterpret_cast<uint2 *>(dst) = make_uint2(pk[0], pk[1]);
            if (lto) {
                uint16_t *ldst = lto + r * kHeadDim + d0;
                if constexpr (N == 8) *reinterpret_cast<uint4 *>(ldst) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
                else *reinterpret_cast<uint2 *>(ldst) = make_uint2(pk[0], pk[1]);
            }
            return;
        }
        const int qi = r / p.g, gi = r - (r / p.g) * p.g;
        store_out<N>(p.out, p.out_dtype, b * p.s_o_seq + qi * p.s_o_len + h * p.s_o_head + gi * p.s_o_group + d0, v);
    }
    // L = sum of exp2(logit2 - m2) over the slot, m2 = running max in log2 units
    __device__ __forceinline__ void stats(int r, float L, float m2) const {
        if (!final_row) {
            const float m = L > 0.f ? m2 * kLn2 : -INFINITY;
            es[r] = L;
            ml[r] = m;
            if (les) {
                les[r] = L;
                lml[r] = m;
            }
        }
    }
};

__device__ __forceinline__ bf16x8 load_q8(const uint16_t *p, bool f16) {
    uint4 raw = *reinterpret_cast<const uint4 *>(p);
    if (!f16) return __builtin_bit_cast(bf16x8, raw);
    f16x8 hv = __builtin_bit_cast(f16x8, raw);
    bf16x8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (__bf16)(float)hv[i];
    return r;
}

__device__ __forceinline__ bf16x8 pack_bf16x8(f32x4 a, f32x4 b) {
    bf16x4 x = __builtin_convertvector(a, bf16x4);
    bf16x4 y = __builtin_convertvector(b, bf16x4);
    return __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Waves per SIMD the decode kernels are compiled for: one 16-row group per wave
// fits two waves (<= 256 registers each) up to D = 128; more row groups per wave,
// or D = 192 / 256, hold their accumulators in AGPRs and run one wave per SIMD.
template <int MTPW, int D>
constexpr int kWavesPerSimd = (MTPW == 1 && D <= 128) ? 2 : 1;

#ifndef PA_FP8_STAGED_WAVES
#define PA_FP8_STAGED_WAVES 3  // waves per SIMD the LDS-staged layout is compiled for (D <= 128)
#endif
// LDS-staged layout: three waves per SIMD up to D = 128; its ring of three
// 128 D + 768 byte stages allows two workgroups per CU at D = 192 and one at 256.
template <int MTPW, int NS, int D>
constexpr int kWavesFor = NS == 0 ? (D <= 128 ? PA_FP8_STAGED_WAVES : (D <= 192 ? 2 : 1)) : kWavesPerSimd<MTPW, D>;

// Query rows of one wave: MTPW groups of 16 rows (r = qi*g + gi), the QK B
// operands and the keys each row may see.  Lane (qrow l16, kg) holds dims
// [D/4 kg, D/4 (kg+1)) of its row; keys visible to a row are [lo_n, hi_n) (causal
// bound ctx+1-ql+qi, window start ctx-ql-sw+qi); lo_max / hi_min bound them over
// the wave's live rows (wave-uniform).
template <int MTPW, int D>
struct RowSet {
    static constexpr bool kFp8 = false;
    static constexpr int kMtpw = MTPW, kD = D;
    bf16x8 qop[MTPW][D / 32];
    int lo_n[MTPW], hi_n[MTPW];
    int lo_max, hi_min;
};

// Query rows as a two-term fp8 split for the fp8 QK products: x = q * 2^k (2^k the
// largest power of two with amax(x) <= 448), hi = e4m3(x), lo = e4m3(x - hi).  A
// bf16 value has 8 significant bits and hi keeps the top 4 (rounded), so the
// residual is a multiple of the bf16 ulp below 2^-4 |x| and lo holds it exactly
// (while it stays above e4m3's subnormal step 2^-9): hi + lo = x.  2^-k is the E8M0
// block scale qsb = 127 - k of the row's B operand, so the products are q . k exactly
// (f32 accumulation), as on the bf16 path.  A lane's D/4 values fill NF 32-byte
// operands (the last one zero-padded when D/4 is not a multiple of 32).
template <int MTPW, int D>
struct RowSetF8 {
    static constexpr bool kFp8 = true;
    static constexpr int kMtpw = MTPW, kD = D;
    static constexpr int NF = (D / 4 + 31) / 32;
    i32x8 qh[MTPW][NF], ql[MTPW][NF];
    int qsb[MTPW];
    int lo_n[MTPW], hi_n[MTPW];
    int lo_max, hi_min;
};

// fp8 two-term split of one lane's D/4 query values (dims D/4 kg .. D/4 kg + D/4 - 1
// of its row); the row's amax is reduced over its 4 lanes (kg = lane / 16).
template <int MTPW, int D>
__device__ __forceinline__ void split_q_fp8(RowSetF8<MTPW, D> &rw, int mg, const bf16x8 (&q)[D / 32], bool live) {
    constexpr int DL = D / 4;
    constexpr int NF = RowSetF8<MTPW, D>::NF;
    float x[DL];
    float amax = 0.0f;
#pragma unroll
    for (int s = 0; s < D / 32; ++s)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            x[8 * s + i] = (float)q[s][i];
            amax = fmaxf(amax, fabsf(x[8 * s + i]));
        }
    amax = fmaxf(amax, shfl_xor_f(amax, 16));
    amax = fmaxf(amax, shfl_xor_f(amax, 32));
    // 448 / amax in [2^(e-1), 2^e): k = e - 1, clamped to the E8M0 range
    int k = 0;
    if (live && amax > 0.0f) k = min(max(__builtin_amdgcn_frexp_expf(448.0f / amax) - 1, -126), 126);
    rw.qsb[mg] = 127 - k;
    const float inv = __builtin_amdgcn_ldexpf(1.0f, k);
#pragma unroll
    for (int u = 0; u < NF; ++u)
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            float v[4], r[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int k = 32 * u + 4 * w + i;
                v[i] = k < DL ? x[k < DL ? k : 0] * inv : 0.0f;
            }
            int hi = __builtin_amdgcn_cvt_pk_fp8_f32(v[0], v[1], 0, false);
            hi = __builtin_amdgcn_cvt_pk_fp8_f32(v[2], v[3], hi, true);
            const f32x2 h01 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false);
            const f32x2 h23 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
            r[0] = v[0] - h01[0];
            r[1] = v[1] - h01[1];
            r[2] = v[2] - h23[0];
            r[3] = v[3] - h23[1];
            int lo = __builtin_amdgcn_cvt_pk_fp8_f32(r[0], r[1], 0, false);
            lo = __builtin_amdgcn_cvt_pk_fp8_f32(r[2], r[3], lo, true);
            rw.qh[mg][u][w] = hi;
            rw.ql[mg][u][w] = lo;
        }
}

// bf16 negation (sign bits) of eight values.
__device__ __forceinline__ bf16x8 neg_bf16x8(bf16x8 v) {
    u32x4 u = __builtin_bit_cast(u32x4, v);
    u ^= u32x4{0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u};
    return __builtin_bit_cast(bf16x8, u);
}

// |k_fac| kept positive (a zero scale, as from an all-zero K, becomes the smallest
// normal float: every visible logit then scales to about 0, masked ones stay -inf).
__device__ __forceinline__ float logit_scale(float k_fac) { return fmaxf(fabsf(k_fac), 1.17549435e-38f); }

// Query rows (row_group0 + mg) * 16 + l16 of (sequence b, kv head h), negated when
// the logit scale is negative (the softmax then takes |scale|).
template <class RW>
__device__ __forceinline__ void setup_rows(RW &rw, const DecodeParams &p, int b, int h, int ctx, int tok_lo,
                                           int tok_hi, int row_group0, int l16, int kg, bool negate) {
    constexpr int MTPW = RW::kMtpw;
    constexpr int D = RW::kD;
    rw.lo_max = tok_lo;
    rw.hi_min = tok_hi;
#pragma unroll
    for (int mg = 0; mg < MTPW; ++mg) {
        const int n = (row_group0 + mg) * 16 + l16;
        if (n < p.eqgs) {
            const int qi = n / p.g;
            const int gi = n - qi * p.g;
            const uint16_t *qrow =
                p.query + (int64_t)(b * p.ql + qi) * p.s_q_seq + (int64_t)(h * p.g + gi) * p.s_q_head + (D / 4) * kg;
            bf16x8 q[D / 32];
#pragma unroll
            for (int s = 0; s < D / 32; ++s) q[s] = load_q8(qrow + 8 * s, p.q_f16 != 0);
            if (negate) {
#pragma unroll
                for (int s = 0; s < D / 32; ++s) q[s] = neg_bf16x8(q[s]);
            }
            if constexpr (RW::kFp8) {
                split_q_fp8<MTPW, D>(rw, mg, q, true);
            } else {
#pragma unroll
                for (int s = 0; s < D / 32; ++s) rw.qop[mg][s] = q[s];
            }
            rw.hi_n[mg] = min(tok_hi, ctx + 1 - p.ql + qi);
            rw.lo_n[mg] = p.sw > 0 ? max(tok_lo, ctx - p.ql - p.sw + qi) : tok_lo;
        } else {
            bf16x8 q[D / 32];
#pragma unroll
            for (int s = 0; s < D / 32; ++s) q[s] = bf16x8{};
            if constexpr (RW::kFp8) {
                split_q_fp8<MTPW, D>(rw, mg, q, false);
            } else {
#pragma unroll
                for (int s = 0; s < D / 32; ++s) rw.qop[mg][s] = q[s];
            }
            rw.hi_n[mg] = tok_hi;  // padded rows: any finite value, never stored
            rw.lo_n[mg] = tok_lo;
        }
        rw.lo_max = max(rw.lo_max, rw.lo_n[mg]);
        rw.hi_min = min(rw.hi_min, rw.hi_n[mg]);
    }
    // the min / max over the 16 rows of a group: rows differ only through qi
    for (int sh = 1; sh < 16; sh <<= 1) {
        rw.lo_max = max(rw.lo_max, __shfl_xor(rw.lo_max, sh, 64));
        rw.hi_min = min(rw.hi_min, __shfl_xor(rw.hi_min, sh, 64));
    }
    rw.lo_max = __builtin_amdgcn_readfirstlane(rw.lo_max);
    rw.hi_min = __builtin_amdgcn_readfirstlane(rw.hi_min);
}

// Per-lane online-softmax state.  m_run is the reference max (log2 units) the
// exponentials, l_run and o are taken against; it is raised only when a step's
// max exceeds it by more than kSlack, so exp2(logit - m_run) <= 2^kSlack and o is
// rescaled on few steps.  m_top is the true running max, used for the stats.
template <int MTPW, int D>
struct SmState {
    float m_run[MTPW], l_run[MTPW], m_top[MTPW];
    // derived from m_run, updated only when it is raised: the exponent offset
    // (-m_run, 0 while the row has seen no key) and the raise threshold m_run + kSlack
    float m_neg[MTPW], m_raise[MTPW];
    f32x4 o[MTPW][D / 16];

    __device__ __forceinline__ void init() {
#pragma unroll
        for (int mg = 0; mg < MTPW; ++mg) {
            m_run[mg] = -INFINITY;
            m_top[mg] = -INFINITY;
            m_neg[mg] = 0.0f;
            m_raise[mg] = -INFINITY;
            l_run[mg] = 0.0f;
#pragma unroll
            for (int m = 0; m < D / 16; ++m) o[mg][m] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
};

// QK and softmax of one 64-token step: kr holds the step's K ([tile][chunk], 16 fp8
// each: lane (l16, kg) of tile jt holds token 16*(l16>>2) + 4*jt + (l16&3), dims of
// chunks D/64 kg .. D/64 kg + D/64 - 1).  QK tile jt, row 4*kg+i of the MFMA output
// is token trow + 4*jt + i with trow = t0 + 16*kg, so lane (qrow, kg) ends up
// owning the 16 tokens of group kg -- exactly the tokens of its PV operand row.
// Writes the bf16 probabilities of every row group to pop.  After the QK products,
// after_qk() runs (the K registers are free again).
//
// With the fp8 row set (RW::kFp8), QK runs on fp8 MFMAs straight from the K bytes
// (two consecutive 16-byte chunks of tile jt are one 32-byte A operand, matching
// the query's operand u), two products per operand (hi and lo terms of the query),
// and the row's block scale makes them the exact q . k; no K conversion.
//
// Either way the products are q . k before any scale.  The per-token K scale
// multiplies them; the logit scale k_eff (> 0: softmax scale x log2 e x per-tensor K
// scale, its sign moved into the query) joins the max once per row and each
// exponent through an FMA, exp2(s k_eff - m).
// 16-byte K chunks a lane holds per tile: D/64, rounded up to even (the padding
// chunk, zero, completes the last 32-byte fp8 operand when D/64 is odd).
template <int D>
constexpr int kKChunks = (D / 64 + 1) / 2 * 2;

// The 4x4 block transpose of a tile set across the lane rows: afterwards row g of
// register j holds what row j of register g held (two v_permlane32_swap, then two
// v_permlane16_swap rounds; each lane keeps its l16).
__device__ __forceinline__ void rows_transpose4(f32x4 (&t)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(t[0][i]), __float_as_uint(t[2][i]), false, false);
        const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(t[1][i]), __float_as_uint(t[3][i]), false, false);
        const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
        const auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
        t[0][i] = __uint_as_float(c[0]);
        t[1][i] = __uint_as_float(c[1]);
        t[2][i] = __uint_as_float(d[0]);
        t[3][i] = __uint_as_float(d[1]);
    }
}

// KT: kr holds K by page instead: tile jt is the step's 16-token group jt, lane
// (l16, kg) its token l16 (dims as above), so each load instruction reads four
// 256-byte runs.  The products then hold token t0 + 16 jt + 4 kg + i at (tile jt,
// row kg, i), and one transpose of the tiles across the lane rows brings them to
// the layout above before the scales, the mask and the softmax.  Against the
// 64-byte runs of the layout above (four tokens of four groups per instruction)
// the register paths ran 5% faster (c2 88.4 -> 83.9 us, c3 152.2 -> 143.5 us):
// the wider runs stream better, and the K pages come from the V lanes' page-table
// entries, one load per step fewer.
template <int MTPW, int D, bool PER_TOKEN, bool KT, class RW, class KScale, class VScale, class AfterQk>
__device__ __forceinline__ void step_qk_softmax(SmState<MTPW, D> &st, const RW &rw, const uint4 (&kr)[4][kKChunks<D>],
                                                const KScale &ksr, const VScale &vsr, float k_eff, int t0,
                                                int kg, bf16x8 (&pop)[MTPW][2], AfterQk &&after_qk) {
    constexpr int CPL = D / 64;  // 16-byte K chunks per lane that hold keys
    const int trow = t0 + 16 * kg;  // token of (tile jt, i) = trow + 4jt + i
    const bool interior = t0 >= rw.lo_max && t0 + kStep <= rw.hi_min;

    // QK: S[token][qrow] for 4 tiles of 16 tokens.  The wave runs its products and
    // softmax here at raised issue priority (1), and its PV products in step_pv
    // higher still (2); its loads, LDS reads and barrier waits stay at the base
    // level.  The SIMD then keeps feeding the matrix pipe of a wave that reached
    // its products while the other waves' VALU work fills the pipe's busy cycles.
    f32x4 sc[MTPW][4];
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
        if constexpr (RW::kFp8) {
            constexpr int NF = RW::NF;
            static_assert(2 * NF == kKChunks<D>, "one fp8 operand per pair of chunks");
            i32x8 a[NF];
#pragma unroll
            for (int u = 0; u < NF; ++u) {
                const uint4 c0 = kr[jt][2 * u];
                const uint4 c1 = kr[jt][2 * u + 1];
                a[u] = i32x8{(int)c0.x, (int)c0.y, (int)c0.z, (int)c0.w, (int)c1.x, (int)c1.y, (int)c1.z, (int)c1.w};
            }
#pragma unroll
            for (int mg = 0; mg < MTPW; ++mg) {
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int u = 0; u < NF; ++u) {
                    acc = mfma_fp8_k128(a[u], rw.qh[mg][u], acc, rw.qsb[mg]);
                    acc = mfma_fp8_k128(a[u], rw.ql[mg][u], acc, rw.qsb[mg]);
                }
                sc[mg][jt] = acc;
            }
        } else {
            bf16x8 a[D / 32];
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                a[2 * c] = fp8x8_to_bf16x8(kr[jt][c].x, kr[jt][c].y);
                a[2 * c + 1] = fp8x8_to_bf16x8(kr[jt][c].z, kr[jt][c].w);
            }
#pragma unroll
            for (int mg = 0; mg < MTPW; ++mg) {
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < D / 32; ++s) acc = mfma_bf16(a[s], rw.qop[mg][s], acc);
                sc[mg][jt] = acc;
            }
        }
    }
    after_qk();
    if constexpr (KT) {
#pragma unroll
        for (int mg = 0; mg < MTPW; ++mg) rows_transpose4(sc[mg]);
    }

    f32x4 kf[4];  // per-token K scales of the 16 tokens
    if constexpr (PER_TOKEN) {
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) kf[jt] = ksr(jt);
    }

#pragma unroll
    for (int mg = 0; mg < MTPW; ++mg) {
        if constexpr (PER_TOKEN) {
#pragma unroll
            for (int jt = 0; jt < 4; ++jt) sc[mg][jt] *= kf[jt];
        }
        if (!interior) {  // one wave-uniform branch for the whole step
#pragma unroll
            for (int jt = 0; jt < 4; ++jt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int t = trow + 4 * jt + i;
                    sc[mg][jt][i] = (t >= rw.lo_n[mg] && t < rw.hi_n[mg]) ? sc[mg][jt][i] : -INFINITY;
                }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sc[mg][jt][i]);
        }
        mx = rows4_max(mx) * k_eff;  // k_eff > 0: the max of the scaled logits (-inf stays -inf)
        st.m_top[mg] = max_raw(st.m_top[mg], mx);
        const bool raise = mx > st.m_raise[mg];  // m_run + kSlack; false while the row has seen no key
        if (__any(raise)) {                      // wave-uniform
            const float alpha = raise ? fast_exp2(st.m_run[mg] - mx) : 1.0f;  // 0 on a row's first keys
            st.m_run[mg] = raise ? mx : st.m_run[mg];
            st.m_neg[mg] = st.m_run[mg] == -INFINITY ? 0.0f : -st.m_run[mg];
            st.m_raise[mg] = st.m_run[mg] + kSlack;
            st.l_run[mg] *= alpha;
#pragma unroll
            for (int m = 0; m < D / 16; ++m) st.o[mg][m] *= alpha;
        }
        const float m_neg = st.m_neg[mg];
        float psum;
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float pv = fast_exp2(fmaf(sc[mg][jt][i], k_eff, m_neg));
                psum = (jt | i) ? psum + pv : pv;
                sc[mg][jt][i] = pv;
            }
            if constexpr (PER_TOKEN) sc[mg][jt] *= vsr(jt);
        }
        st.l_run[mg] += psum;
        pop[mg][0] = pack_bf16x8(sc[mg][0], sc[mg][1]);
        pop[mg][1] = pack_bf16x8(sc[mg][2], sc[mg][3]);
    }
    __builtin_amdgcn_s_setprio(0);
}

// PV of one step: O[dim][qrow] += V^T P^T over its 64 tokens; vr[m] holds the 16
// tokens of group kg of head dim 16m + l16.
template <int MTPW, int D>
__device__ __forceinline__ void step_pv(SmState<MTPW, D> &st, const uint4 (&vr)[D / 16],
                                        const bf16x8 (&pop)[MTPW][2]) {
    __builtin_amdgcn_s_setprio(2);
#pragma unroll
    for (int m = 0; m < D / 16; ++m) {
        const bf16x8 v0 = fp8x8_to_bf16x8(vr[m].x, vr[m].y);
        const bf16x8 v1 = fp8x8_to_bf16x8(vr[m].z, vr[m].w);
#pragma unroll
        for (int mg = 0; mg < MTPW; ++mg) {
            st.o[mg][m] = mfma_bf16(v0, pop[mg][0], st.o[mg][m]);
            st.o[mg][m] = mfma_bf16(v1, pop[mg][1], st.o[mg][m]);
        }
    }
    __builtin_amdgcn_s_setprio(0);
}

// Rows of a wave that ran every step of the range itself: sum the four kg-lane
// partial exp sums of each row, normalise and emit.
template <int MTPW, int D, class Sink>
__device__ __forceinline__ void finish_rows(SmState<MTPW, D> &st, const DecodeParams &p, int row_group0, int l16,
                                            int kg, float v_fac, const Sink &sink) {
#pragma unroll
    for (int mg = 0; mg < MTPW; ++mg) {
        float lt = st.l_run[mg];
        lt += shfl_xor_f(lt, 16);
        lt += shfl_xor_f(lt, 32);
        const int r = (row_group0 + mg) * 16 + l16;
        if (r < p.eqgs) {
            const float inv = lt > 0.f ? v_fac / lt : 0.f;
#pragma unroll
            for (int m = 0; m < D / 16; ++m) {
                const f32x4 v = st.o[mg][m] * inv;
                const float v4[4] = {v[0], v[1], v[2], v[3]};
                sink.row(r, 16 * m + 4 * kg, v4);
            }
            if (kg == 0) sink.stats(r, lt > 0.f ? lt * fast_exp2(st.m_run[mg] - st.m_top[mg]) : 0.f, st.m_top[mg]);
        }
    }
}

// Rows [row0, row_end) of an empty range (kernels/pa_decode_fp8.py:2591-2598),
// written by the nthreads threads tid = 0 .. nthreads-1.
template <int D, class Sink>
__device__ __forceinline__ void emit_empty(int nthreads, int row0, int row_end, const Sink &sink,
                                           int tid = threadIdx.x) {
    for (int r = row0 + tid; r < row_end; r += nthreads) sink.stats(r, 0.0f, -INFINITY);
    const float zero8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int i = tid; i < (row_end - row0) * (D / 8); i += nthreads)
        sink.row(row0 + i / (D / 8), (i % (D / 8)) * 8, zero8);
}

// Attention of query rows [row0, row0 + 64) of (sequence b, kv head h) over the
// keys [tok_lo, tok_hi) of the sequence, streaming K / V through registers; the
// result of each row r = qi*g + gi goes to sink.row (normalised output) and
// sink.stats (exp sum and log2-domain max).  ctx is already clamped to the page
// row's capacity; bt_row is the sequence's page row (block-table row or
// kv_page_indices window).  Every thread of the workgroup calls this with the same
// arguments (it synchronises internally).
// The workgroup has NW = RS * NS waves.  Wave w owns query-row groups
// [rs*MTPW, (rs+1)*MTPW) of the chunk (rs = w % RS, 16 rows per group) and the
// steps ns, ns+NS, ... of the range (ns = w / RS).  Each wave loads its own steps:
// the next step's K goes into the K registers right after the QK products, its V
// right after the PV products.  Waves of the same rs merge their online-softmax
// states through LDS at the end.
template <int MTPW, int RS, int NS, bool PER_TOKEN, int D, bool V4, class Sink>
__device__ __forceinline__ void attend_range(const DecodeParams &p, const int b, const int h, const int ctx,
                                             const int tok_lo, const int tok_hi, const int32_t *bt_row,
                                             const int row0, const Sink &sink) {
    constexpr int NW = RS * NS;
    constexpr int CPL = D / 64;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rs = wave % RS;
    const int ns = wave / RS;
    const int l16 = lane & 15;
    const int kg = lane >> 4;
    const int bs = 1 << p.bs_log2;
    const int row_group0 = (row0 >> 4) + rs * MTPW;

    if (tok_lo >= tok_hi) {
        emit_empty<D>(NW * 64, row0, min(p.eqgs, row0 + kRowChunk), sink);
        return;
    }
    const float k_fac = PER_TOKEN ? p.qk_scale : p.qk_scale * p.ks[0];
    const float k_eff = logit_scale(k_fac);
    RowSet<MTPW, D> rw;
    setup_rows(rw, p, b, h, ctx, tok_lo, tok_hi, row_group0, l16, kg, k_fac < 0.0f);
    const float v_fac = PER_TOKEN ? 1.0f : p.vs[0];
    SmState<MTPW, D> st;
    st.init();

    const int ngroups = (tok_hi - tok_lo + kGroup - 1) / kGroup;
    const int nsteps = (ngroups + 3) / 4;
    const int last_group = tok_lo + (ngroups - 1) * kGroup;
    const uint8_t *kc_h = p.kc + (int64_t)h * p.s_k_head;
    const uint8_t *vc_h = p.vc + (int64_t)h * p.s_v_head;
    const int kchunk = bs * 16;  // bytes between 16-dim chunks of one (block, head)
    const int k_lane_off = l16 * 16 + (CPL * kg) * kchunk;
    // V row of (head dim d, 16-token group sub) at sub * vsub + d * vd in the tile
    const int vd = V4 ? bs : 16;
    const int vsub = V4 ? 16 : D * 16;
    const int v_lane_off = l16 * vd;

    // A lane's V / scale group is kg; K tile jt is group jt for every lane, its page
    // the entry lane row jt read (a scalar).  The page-table entries of a step are
    // read one step of the wave earlier than its K / V: vector memory waits are in
    // order, so waiting for entries read just before the step's K would also wait
    // for the V loads still in flight.
    auto page_of = [&](int step, int g) {
        const int gs = min(tok_lo + step * kStep + 16 * g, last_group);
        return bt_row[gs >> p.bs_log2];
    };
    auto k_bases = [&](int step, int ev, const uint8_t *(&kb)[4]) {
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
            const int gs = min(tok_lo + step * kStep + 16 * jt, last_group);
            const int phys = min(max(__builtin_amdgcn_readlane(ev, 16 * jt), 0), p.num_blocks - 1);
            kb[jt] = kc_h + (int64_t)phys * p.s_k_block + ((gs & (bs - 1)) >> 4) * 256;
        }
    };
    auto v_loc = [&](int step, int e, int64_t &vofs, int64_t &sofs) {
        const int gs = min(tok_lo + step * kStep + 16 * kg, last_group);
        const int phys = min(max(e, 0), p.num_blocks - 1);
        const int sub = (gs & (bs - 1)) >> 4;
        vofs = (int64_t)phys * p.s_v_block + sub * vsub + v_lane_off;
        sofs = (int64_t)phys * p.s_ks_block + (int64_t)h * p.s_ks_head + sub * 16;
    };

    // K of the step: [tile][chunk], 16 fp8 each, tile jt the step's group jt (the
    // page-per-tile layout of step_qk_softmax<..., KT = true>; the bf16 products skip
    // the padding chunk)
    uint4 kr[4][kKChunks<D>];
    uint4 vr[D / 16];  // V of the step: [dim tile], 16 tokens of one head dim
    // Per-token scales: a lane needs the 16 K and 16 V scales of its group kg, and
    // loads a quarter of each (tokens 4 (l16 & 3) .. +3, 16 bytes); the quad of
    // lanes l16 & 3 = 0..3 holds the whole group, and each step gathers it with DPP
    // quad broadcasts.  Two loads per step instead of eight lane-replicated ones:
    // the load instructions, not their bytes, made per-token scales cost c3 4%
    // (kernel 159.6 us, 152.8 us with the scale loads taken out, 155.5 us gathered).
    f32x4 ksl, vsl;
    auto load_k = [&](const uint8_t *const (&kb)[4]) {
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
#pragma unroll
            for (int c = 0; c < CPL; ++c) kr[jt][c] = ld16(kb[jt] + k_lane_off + c * kchunk);
    };
    auto load_v = [&](int64_t vofs) {
#pragma unroll
        for (int m = 0; m < D / 16; ++m) vr[m] = ld16(vc_h + vofs + m * 16 * vd);
    };
    auto load_scales = [&](int64_t sofs) {
        ksl = *reinterpret_cast<const f32x4 *>(p.ks + sofs + 4 * (l16 & 3));
        vsl = *reinterpret_cast<const f32x4 *>(p.vs + sofs + 4 * (l16 & 3));
    };

    int step = ns;
    int ev_next = 0;  // page-table entry of the wave's next step
    if (step < nsteps) {
        const int ev = page_of(step, kg);
        if (step + NS < nsteps) ev_next = page_of(step + NS, kg);
        int64_t vofs, sofs;
        v_loc(step, ev, vofs, sofs);
        const uint8_t *kb[4];
        k_bases(step, ev, kb);
        load_k(kb);
        if constexpr (PER_TOKEN) load_scales(sofs);
        load_v(vofs);
    }
    while (step < nsteps) {
        const int nxt = step + NS;
        const bool has_nxt = nxt < nsteps;
        int ev_after = 0;
        if (nxt + NS < nsteps) ev_after = page_of(nxt + NS, kg);
        const uint8_t *nkb[4] = {nullptr, nullptr, nullptr, nullptr};
        int64_t nvofs = 0, nsofs = 0;
        if (has_nxt) {
            k_bases(nxt, ev_next, nkb);
            v_loc(nxt, ev_next, nvofs, nsofs);
        }
        ev_next = ev_after;
        f32x4 ksc[4], vsc[4];  // the step's scales by tile, before the next step's loads reuse ksl / vsl
        if constexpr (PER_TOKEN) {
            quad_gather(ksl, ksc);
            quad_gather(vsl, vsc);
        }
        bf16x8 pop[MTPW][2];
        step_qk_softmax<MTPW, D, PER_TOKEN, true>(st, rw, kr, [&](int jt) { return ksc[jt]; },
                                            [&](int jt) { return vsc[jt]; }, k_eff, tok_lo + step * kStep, kg, pop,
                                            [&] {
                                                if (has_nxt) {
                                                    load_k(nkb);  // K registers are free again
                                                    if constexpr (PER_TOKEN) load_scales(nsofs);
                                                }
                                            });
        step_pv<MTPW, D>(st, vr, pop);
        if (has_nxt) load_v(nvofs);  // V registers are free again
        step = nxt;
    }

    if constexpr (NS == 1) {
        finish_rows<MTPW, D>(st, p, row_group0, l16, kg, v_fac, sink);
    } else {
        // sum the four kg-lane partial exp sums of each query row
#pragma unroll
        for (int mg = 0; mg < MTPW; ++mg) {
            float lt = st.l_run[mg];
            lt += shfl_xor_f(lt, 16);
            lt += shfl_xor_f(lt, 32);
            st.l_run[mg] = lt;
        }
        // merge through LDS in blocks of DB head dims (128, or 64 when D is an odd
        // multiple of 64): RS*16 rows x DB outputs per pass, E per thread
        constexpr int DB = D % 128 == 0 ? 128 : 64;
        constexpr int DP = DB + 4;
        __shared__ float s_o[NW][16][DP];
        __shared__ float s_m[NW][16];
        __shared__ float s_l[NW][16];
        __shared__ float s_t[NW][16];
        constexpr int E = RS * 16 * DB / (NW * 64);
        static_assert(E >= 4 && E % 4 == 0 && E * NW * 64 == RS * 16 * DB, "merge covers each row pass exactly");
        const int flat = tid * E;
        const int mrs = flat / (16 * DB);  // row split this thread merges
        const int n = (flat / DB) % 16;
        const int d0 = flat % DB;
#pragma unroll
        for (int mg = 0; mg < MTPW; ++mg) {
            if (kg == 0) {
                s_m[wave][l16] = st.m_run[mg];
                s_l[wave][l16] = st.l_run[mg];
                s_t[wave][l16] = st.m_top[mg];
            }
#pragma unroll
            for (int db = 0; db < D / DB; ++db) {
#pragma unroll
                for (int m = 0; m < DB / 16; ++m)
                    *reinterpret_cast<f32x4 *>(&s_o[wave][l16][16 * m + 4 * kg]) = st.o[mg][db * (DB / 16) + m];
                __syncthreads();
                float M = -INFINITY, Mt = -INFINITY;
#pragma unroll
                for (int j = 0; j < NS; ++j) {
                    M = fmaxf(M, s_m[j * RS + mrs][n]);
                    Mt = fmaxf(Mt, s_t[j * RS + mrs][n]);
                }
                const float Ms = M == -INFINITY ? 0.0f : M;
                float f[NS];
                float L = 0.f;
#pragma unroll
                for (int j = 0; j < NS; ++j) {
                    f[j] = fast_exp2(s_m[j * RS + mrs][n] - Ms);
                    L += s_l[j * RS + mrs][n] * f[j];
                }
                const float inv = L > 0.f ? v_fac / L : 0.f;
                const int r = ((row0 >> 4) + mrs * MTPW + mg) * 16 + n;
                if (r < p.eqgs) {
                    constexpr int EW = E < 8 ? E : 8;  // outputs per store (E is 4 with 8 waves)
#pragma unroll
                    for (int e0 = 0; e0 < E; e0 += EW) {
                        float v8[EW];
#pragma unroll
                        for (int j2 = 0; j2 < EW; ++j2) {
                            float a = 0.f;
#pragma unroll
                            for (int j = 0; j < NS; ++j) a += s_o[j * RS + mrs][n][d0 + e0 + j2] * f[j];
                            v8[j2] = a * inv;
                        }
                        sink.row(r, db * DB + d0 + e0, v8);
                    }
                    if (db == 0 && d0 == 0) sink.stats(r, L > 0.f ? L * fast_exp2(M - Mt) : 0.f, Mt);
                }
                __syncthreads();
            }
        }
    }
}

// Token range [lo, hi) of partition slot z of a sequence of ctx tokens: the 256-token
// partitions [z*pps, min((z+1)*pps, T)) with T = ceil(ctx/256), pps = ceil(T/P)
// (kernels/pa_decode_fp8.py:2311-2320); with a sliding window they start at tile
// max(ctx-ql-sw, 0)/256 (kernels/pa_decode_swa.py:1359-1368) and the first window tile
// is trimmed to the 16-token group holding the window start.  Empty when lo >= hi.
// Slot ranges are increasing in z and contiguous: an empty slot has only empty
// slots after it.
__device__ __forceinline__ void slot_tokens(const DecodeParams &p, int ctx, int z, int &lo, int &hi) {
    const int T = (ctx + kPartition - 1) / kPartition;
    const int seq_start = p.sw > 0 ? max(ctx - p.ql - p.sw, 0) : 0;
    const int first_tile = seq_start / kPartition;
    const int vis = T - first_tile;
    const int pps = vis > 0 ? (vis + p.max_parts - 1) / p.max_parts : 0;
    const int plo = first_tile + z * pps;
    const int phi = min(plo + pps, T);
    lo = plo * kPartition;
    hi = min(phi * kPartition, ctx);
    if (lo < seq_start) lo = seq_start & ~(kGroup - 1);
}

// Single-wave layout over a chain of partition slots [z0, z1) of (sequence b, kv
// head h), query rows [row0, row0 + 16*MTPW): the wave streams the steps of every
// slot in turn, its load pipeline (page-table entries two steps ahead, K / V one
// step ahead) running on across slot boundaries, and writes each slot's partial (or,
// with one slot per sequence, the output) when that slot's last step is done.  The
// per-slot state restarts there; each slot's result is exactly what a workgroup of
// its own would write.  Slots without keys (a suffix of the chain) get the empty
// partial (kernels/pa_decode_fp8.py:2591-2598).
template <int MTPW, bool PER_TOKEN, int D, bool V4>
__device__ __forceinline__ void attend_slots(const DecodeParams &p, const int b, const int h, const int ctx,
                                             const int z0, const int z1, const int32_t *bt_row, const int row0,
                                             uint8_t *merge_lds = nullptr) {
    constexpr int CPL = D / 64;
    const int lane = threadIdx.x & 63;
    const int l16 = lane & 15;
    const int kg = lane >> 4;
    const int bs = 1 << p.bs_log2;
    const int row_group0 = row0 >> 4;
    // one slot per sequence in direct mode: the final rows; otherwise the slot's partial
    const bool final_row = p.direct && p.max_parts == 1;
    auto sink_of = [&](int z) {
        SlotSink sk{p,
                    p.tmp_out + b * p.s_to_seq + h * p.s_to_head + z * p.s_to_part,
                    p.exp_sums + b * p.s_es_seq + h * p.s_es_head + z * p.s_es_part,
                    p.max_logits + b * p.s_es_seq + h * p.s_es_head + z * p.s_es_part,
                    b,
                    h,
                    final_row};
        if (merge_lds) {  // [P][eqgs][kHeadDim] bf16 rows, then [P][eqgs] exp sums and max logits
            const int rows = p.max_parts * p.eqgs;
            sk.lto = reinterpret_cast<uint16_t *>(merge_lds) + z * p.eqgs * kHeadDim;
            sk.les = reinterpret_cast<float *>(merge_lds + rows * kHeadDim * 2) + z * p.eqgs;
            sk.lml = sk.les + rows;
        }
        return sk;
    };

    // Slot geometry of the sequence (slot_tokens without its division per slot):
    // slot z covers [max(base + z * span, trim), min(base + (z + 1) * span, ctx)).
    const int T = (ctx + kPartition - 1) / kPartition;
    const int seq_start = p.sw > 0 ? max(ctx - p.ql - p.sw, 0) : 0;
    const int first_tile = seq_start / kPartition;
    const int vis = T - first_tile;
    const int pps = vis > 0 ? (vis + p.max_parts - 1) / p.max_parts : 0;
    const int base = first_tile * kPartition, span = pps * kPartition;
    const int trim = seq_start & ~(kGroup - 1);
    auto slot_lo = [&](int z) { return max(base + z * span, trim); };
    auto slot_hi = [&](int z) { return min(base + (z + 1) * span, ctx); };
    // the slots with keys: a prefix [z0, ze) of the chain (slot z has keys iff its
    // first tile exists, first_tile + z * pps < T)
    const int ze = pps > 0 ? min(z1, max(z0, (vis + pps - 1) / pps)) : z0;
    for (int z = ze; z < z1; ++z) emit_empty<D>(64, row0, min(p.eqgs, row0 + kRowChunk), sink_of(z), lane);
    if (ze == z0) return;

    const float k_fac = PER_TOKEN ? p.qk_scale : p.qk_scale * p.ks[0];
    const float k_eff = logit_scale(k_fac);
    RowSet<MTPW, D> rw;
    // the rows' own key bounds (window start, causal end), clipped per slot below
    setup_rows(rw, p, b, h, ctx, 0, ctx, row_group0, l16, kg, k_fac < 0.0f);
    int row_lo[MTPW], row_hi[MTPW];
#pragma unroll
    for (int mg = 0; mg < MTPW; ++mg) {
        row_lo[mg] = rw.lo_n[mg];
        row_hi[mg] = rw.hi_n[mg];
    }
    const int rows_lo_max = rw.lo_max, rows_hi_min = rw.hi_min;
    const float v_fac = PER_TOKEN ? 1.0f : p.vs[0];
    SmState<MTPW, D> st;
    st.init();

    // A step of the chain: its slot z (ze: past the chain), first token t0 and its
    // slot's end e (page reads clamp to token e - 1, in the slot's last 16-token group).
    // The slot has a later step iff t0 + 64 < e.  Wave-uniform.
    struct Cur {
        int z, t0, e;
    };
    auto slot_first = [&](int z) { return z < ze ? Cur{z, slot_lo(z), slot_hi(z)} : Cur{ze, 0, 1}; };
    auto advance = [&](const Cur &c) {
        if (c.z >= ze) return c;
        return c.t0 + kStep < c.e ? Cur{c.z, c.t0 + kStep, c.e} : slot_first(c.z + 1);
    };
    auto enter_slot = [&](const Cur &c) {  // the rows' key bounds within the slot
        const int lo = slot_lo(c.z);
#pragma unroll
        for (int mg = 0; mg < MTPW; ++mg) {
            rw.lo_n[mg] = max(row_lo[mg], lo);
            rw.hi_n[mg] = min(row_hi[mg], c.e);
        }
        rw.lo_max = max(rows_lo_max, lo);
        rw.hi_min = min(rows_hi_min, c.e);
    };

    const uint8_t *kc_h = p.kc + (int64_t)h * p.s_k_head;
    const uint8_t *vc_h = p.vc + (int64_t)h * p.s_v_head;
    const int kchunk = bs * 16;
    const int k_lane_off = l16 * 16 + (CPL * kg) * kchunk;
    const int vd = V4 ? bs : 16;
    const int vsub = V4 ? 16 : D * 16;
    const int v_lane_off = l16 * vd;
    auto page_of = [&](const Cur &c, int g) { return bt_row[min(c.t0 + 16 * g, c.e - 1) >> p.bs_log2]; };
    auto k_bases = [&](const Cur &c, int ev, const uint8_t *(&kb)[4]) {  // tile jt: the page lane row jt read
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
            const int gs = min(c.t0 + 16 * jt, c.e - 1);
            const int phys = min(max(__builtin_amdgcn_readlane(ev, 16 * jt), 0), p.num_blocks - 1);
            kb[jt] = kc_h + (int64_t)phys * p.s_k_block + ((gs & (bs - 1)) >> 4) * 256;
        }
    };
    auto v_loc = [&](const Cur &c, int e, int64_t &vofs, int64_t &sofs) {
        const int gs = min(c.t0 + 16 * kg, c.e - 1);
        const int phys = min(max(e, 0), p.num_blocks - 1);
        const int sub = (gs & (bs - 1)) >> 4;
        vofs = (int64_t)phys * p.s_v_block + sub * vsub + v_lane_off;
        sofs = (int64_t)phys * p.s_ks_block + (int64_t)h * p.s_ks_head + sub * 16;
    };

    uint4 kr[4][kKChunks<D>];
    uint4 vr[D / 16];
    f32x4 ksl, vsl;  // per-token scale quarters, gathered across the quad at each step
    auto load_k = [&](const uint8_t *const (&kb)[4]) {
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
#pragma unroll
            for (int c = 0; c < CPL; ++c) kr[jt][c] = ld16(kb[jt] + k_lane_off + c * kchunk);
    };
    auto load_v = [&](int64_t vofs) {
#pragma unroll
        for (int m = 0; m < D / 16; ++m) vr[m] = ld16(vc_h + vofs + m * 16 * vd);
    };
    auto load_scales = [&](int64_t sofs) {
        ksl = *reinterpret_cast<const f32x4 *>(p.ks + sofs + 4 * (l16 & 3));
        vsl = *reinterpret_cast<const f32x4 *>(p.vs + sofs + 4 * (l16 & 3));
    };

    Cur cur = slot_first(z0);
    Cur c1 = advance(cur);
    int ev_next = 0;  // page-table entry of step c1
    {
        const int ev = page_of(cur, kg);
        if (c1.z < ze) ev_next = page_of(c1, kg);
        int64_t vofs, sofs;
        v_loc(cur, ev, vofs, sofs);
        const uint8_t *kb[4];
        k_bases(cur, ev, kb);
        load_k(kb);
        if constexpr (PER_TOKEN) load_scales(sofs);
        load_v(vofs);
    }
    enter_slot(cur);
    while (cur.z < ze) {
        const Cur c2 = advance(c1);
        const bool has_nxt = c1.z < ze;
        int ev_after = 0;
        if (c2.z < ze) ev_after = page_of(c2, kg);
        const uint8_t *nkb[4] = {nullptr, nullptr, nullptr, nullptr};
        int64_t nvofs = 0, nsofs = 0;
        if (has_nxt) {
            k_bases(c1, ev_next, nkb);
            v_loc(c1, ev_next, nvofs, nsofs);
        }
        ev_next = ev_after;
        f32x4 ksc[4], vsc[4];
        if constexpr (PER_TOKEN) {
            quad_gather(ksl, ksc);
            quad_gather(vsl, vsc);
        }
        bf16x8 pop[MTPW][2];
        step_qk_softmax<MTPW, D, PER_TOKEN, true>(st, rw, kr, [&](int jt) { return ksc[jt]; },
                                            [&](int jt) { return vsc[jt]; }, k_eff, cur.t0, kg, pop, [&] {
                                                if (has_nxt) {
                                                    load_k(nkb);
                                                    if constexpr (PER_TOKEN) load_scales(nsofs);
                                                }
                                            });
        step_pv<MTPW, D>(st, vr, pop);
        if (has_nxt) load_v(nvofs);
        if (c1.z != cur.z) {  // the slot's last step: its result, then a fresh state for the next slot
            finish_rows<MTPW, D>(st, p, row_group0, l16, kg, v_fac, sink_of(cur.z));
            if (has_nxt) {
                st.init();
                enter_slot(c1);
            }
        }
        cur = c1;
        c1 = c2;
    }
}

// ------------------------------------------------------- LDS-staged K / V stream
// For layouts where every wave of the workgroup consumes every step (NS == 0),
// the workgroup streams the steps' K / V through an LDS ring: each step's 128 D
// bytes (plus its per-token scales) are loaded once per workgroup with direct
// global -> LDS loads (global_load_lds_dwordx4, 16 bytes per lane, lane i landing
// at M0 + 16 i), kStages - 1 steps ahead of the step being computed.  The loads
// are issued from inline assembly, so the compiler does not order LDS reads
// behind them; each wave waits for its own loads of a step with an explicit
// s_waitcnt vmcnt(n) (loads complete in issue order, and n counts only loads this
// wave issued later, so the wait is never short) and a barrier then publishes the
// step to every wave.  Page indices for the load addresses come from an LDS window
// of the page row, so no vector memory load of the compiler's own sits between
// the asynchronous ones.
//
// Stage layout (bytes): K [4 groups][D/16 chunks][16 tokens][16] with the group
// stride padded to 16 D + 64 (the QK operand reads of lanes 0-3 and 4-7 then hit
// different banks), V [4 groups][D dims][16 tokens], then the per-token K and V
// scales [4 groups][16] f32 each.
#ifndef PA_FP8_STAGES
#define PA_FP8_STAGES 3  // ring depth (steps in flight + 1)
#endif
#ifndef PA_FP8_KPAD
#define PA_FP8_KPAD 64  // bytes of padding after each K group
#endif
#ifndef PA_FP8_PAGE_WINDOW
#define PA_FP8_PAGE_WINDOW 256  // page-row entries held in LDS at a time
#endif
constexpr int kStages = PA_FP8_STAGES;
template <int D>
constexpr int kKGroupStride = 16 * D + PA_FP8_KPAD;
template <int D>
constexpr int kStageV = 4 * kKGroupStride<D>;
template <int D>
constexpr int kStageS = kStageV<D> + 64 * D;
template <int D>
constexpr int kStageBytes = kStageS<D> + 512;
constexpr int kPageWin = PA_FP8_PAGE_WINDOW;

typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const lds_void_t *)p;
}

// 16 bytes from gptr to LDS byte address lds_base + 16 * lane (with the
// non-temporal hint by default: each K / V byte is read once).
__device__ __forceinline__ void dma16(const void *gptr, uint32_t lds_base) {
#if PA_FP8_NT_KV
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(gptr), "s"(lds_base) : "memory", "m0");
#else
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "s"(lds_base) : "memory", "m0");
#endif
}

// 16 bytes from sbase + voff (sbase wave-uniform, in scalar registers; voff a 32-bit
// per-lane offset) to LDS byte address lds_base + 16 * lane: the SADDR form, whose
// address needs no vector arithmetic.
__device__ __forceinline__ void dma16_s(const void *sbase, uint32_t voff, uint32_t lds_base) {
#if PA_FP8_NT_KV
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(sbase), "s"(lds_base)
                 : "memory", "m0");
#else
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds_base)
                 : "memory", "m0");
#endif
}

// Wait until at most N of this wave's vector memory loads are outstanding and
// its LDS operations are done, then meet the other waves.
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
    static_assert(N >= 0 && N <= 63, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Loads steps of one (sequence, kv head) token range into an LDS ring for NW waves:
// K rows, V rows and (per-token) the scale piece of step q go to stage q % STAGES;
// each wave issues R loads per step.  A K row is 4 chunks x 16 tokens of one
// group (1 KB), a V row 64 head dims x 16 tokens of one group; a group has D/64
// of each.  issue(q) needs every wave past its last use of stage q % STAGES (the
// caller's barrier guarantees it).
template <int NW, int STAGES, bool PER_TOKEN, int D, bool V4>
struct KvStager {
    static constexpr int CPL = D / 64;       // K rows (and V rows) per 16-token group
    static constexpr int KROWS = 4 * CPL / NW;  // K rows a wave loads per step
    static constexpr int VROWS = KROWS;      // V rows (the K rows' groups)
    static constexpr int SLANES = 32 / NW;   // lanes of a wave loading 16 bytes of scales
    static constexpr int R = KROWS + VROWS + (PER_TOKEN ? 1 : 0);
    static_assert(KROWS * NW == 4 * CPL, "the waves split the rows evenly");
    static_assert(NW == 1 || NW == 2 || NW == 4, "1, 2 or 4 waves");
    static_assert((STAGES - 2) * R <= 63, "vmcnt range");

    const DecodeParams &p;
    uint8_t *ring;
    int32_t *pages;
    const int32_t *bt_row;
    const uint8_t *kc_h, *vc_h;
    int kchunk;
    uint32_t ring_addr;
    int h, row_len, tok_lo, last_group, last_page, nsteps, wbase, bs, tid, lane, wave;
    bool one_page;  // every step lies in one page (issue_one_page)
    // loop-invariant lane offsets of the one-page loads: K rows j and V rows j from the
    // step's sub-row 0 of the page, and the lane's scale piece (in floats)
    int k_lane[KROWS], v_lane[VROWS], s_lane;

    __device__ __forceinline__ void load_window(int base) {  // every wave is past its last use of the window
        wbase = base;
        const int n = min(kPageWin, last_page - base + 1);
        for (int i = tid; i < n; i += NW * 64) pages[i] = base + i < row_len ? bt_row[base + i] : 0;
        __syncthreads();
    }
    // physical block and 16-token sub-row of group g of step q
    __device__ __forceinline__ void group_loc(int q, int g, int &phys, int &sub) const {
        const int gs = min(tok_lo + q * kStep + 16 * g, last_group);
        const int e = pages[(gs >> p.bs_log2) - wbase];
        phys = min(max(e, 0), p.num_blocks - 1);
        sub = (gs & (bs - 1)) >> 4;
    }
    // Steps inside one page (pages of 64 tokens or more, the range starting on a step
    // boundary) whose four groups all hold keys: one page-window read and one scalar
    // base per cache for the step, the lanes' parts being loop-invariant offsets.
    __device__ __forceinline__ bool issue_one_page(int q) {
        const int t = tok_lo + q * kStep;
        if (!one_page || t + 3 * kGroup > last_group) return false;
        const int pg = t >> p.bs_log2;
        if (pg - wbase >= kPageWin) load_window(pg);
        const uint32_t sb = ring_addr + (uint32_t)((q % STAGES) * kStageBytes<D>);
        const int e = __builtin_amdgcn_readfirstlane(pages[pg - wbase]);
        const int64_t phys = min(max(e, 0), p.num_blocks - 1);
        const int sub0 = (t & (bs - 1)) >> 4;  // 16-token sub-row of the step's group 0
        const uint8_t *kb = kc_h + phys * p.s_k_block + sub0 * 256;
        const uint8_t *vb = vc_h + phys * p.s_v_block + sub0 * (V4 ? 16 : 16 * D);
#pragma unroll
        for (int j = 0; j < KROWS; ++j) {
            const int r = wave + NW * j;
            const int g = r / CPL, c4 = r % CPL;
            dma16_s(kb, k_lane[j], __builtin_amdgcn_readfirstlane(sb + g * kKGroupStride<D> + c4 * 1024));
        }
#pragma unroll
        for (int j = 0; j < VROWS; ++j) {
            const int r = wave + NW * j;
            const int g = r / CPL, c4 = r % CPL;
            dma16_s(vb, v_lane[j], __builtin_amdgcn_readfirstlane(sb + kStageV<D> + g * (16 * D) + c4 * 1024));
        }
        if constexpr (PER_TOKEN) {
            if (lane < SLANES) {
                const float *sbase = (wave * SLANES < 16 ? p.ks : p.vs) + phys * p.s_ks_block +
                                     (int64_t)h * p.s_ks_head + sub0 * 16;
                dma16_s(sbase, 4 * s_lane, __builtin_amdgcn_readfirstlane(sb + kStageS<D> + wave * SLANES * 16));
            }
        }
        return true;
    }
    __device__ __forceinline__ void issue(int q) {
        if (issue_one_page(q)) return;
        const int lastg_page = min(tok_lo + q * kStep + 48, last_group) >> p.bs_log2;
        if (lastg_page - wbase >= kPageWin) load_window((tok_lo + q * kStep) >> p.bs_log2);
        const uint32_t sb = ring_addr + (uint32_t)((q % STAGES) * kStageBytes<D>);
        // every page-window read first, then the loads: each load's inline asm is a
        // memory barrier to the compiler, so a window read placed between two loads
        // would be waited for on its own
        int phys[KROWS], sub[KROWS];
#pragma unroll
        for (int j = 0; j < KROWS; ++j) group_loc(q, (wave + NW * j) / CPL, phys[j], sub[j]);
        const int piece = wave * SLANES + min(lane, SLANES - 1);
        int sphys = 0, ssub = 0;
        if constexpr (PER_TOKEN) group_loc(q, (piece & 15) >> 2, sphys, ssub);
#pragma unroll
        for (int j = 0; j < KROWS; ++j) {  // K rows: (group g, chunks 4*c4 .. 4*c4+3)
            const int r = wave + NW * j;
            const int g = r / CPL, c4 = r % CPL;
            const uint8_t *src = kc_h + (int64_t)phys[j] * p.s_k_block + (4 * c4 + (lane >> 4)) * kchunk +
                                 sub[j] * 256 + (lane & 15) * 16;
            dma16(src, __builtin_amdgcn_readfirstlane(sb + g * kKGroupStride<D> + c4 * 1024));
        }
#pragma unroll
        for (int j = 0; j < VROWS; ++j) {  // V rows: (group g, dims 64*c4 .. 64*c4+63), the K rows' groups
            const int r = wave + NW * j;
            const int g = r / CPL, c4 = r % CPL;
            const uint8_t *src = vc_h + (int64_t)phys[j] * p.s_v_block + sub[j] * (V4 ? 16 : 16 * D) +
                                 (64 * c4 + lane) * (V4 ? bs : 16);
            dma16(src, __builtin_amdgcn_readfirstlane(sb + kStageV<D> + g * (16 * D) + c4 * 1024));
        }
        if constexpr (PER_TOKEN) {  // 32 pieces of 16 bytes: K scales of groups 0-3, then V scales
            if (lane < SLANES) {
                const float *src = (piece < 16 ? p.ks : p.vs) + (int64_t)sphys * p.s_ks_block +
                                   (int64_t)h * p.s_ks_head + ssub * 16 + 4 * (piece & 3);
                dma16(src, __builtin_amdgcn_readfirstlane(sb + kStageS<D> + wave * SLANES * 16));
            }
        }
    }
    __device__ __forceinline__ void prologue() {
#pragma unroll
        for (int q = 0; q < STAGES - 1; ++q)
            if (q < nsteps) issue(q);
    }
    template <int L>
    __device__ __forceinline__ void wait_later(int later) {
        if constexpr (L > 0) {
            if (later >= L) {
                wait_vm_barrier<L * R>();
                return;
            }
            wait_later<L - 1>(later);
        } else {
            wait_vm_barrier<0>();
        }
    }
    // Step n is in LDS for every wave, and every wave is done with step n-1, after
    // this wave's loads of step n landed (at most (later steps issued) * R of its
    // loads remain outstanding) and the barrier.
    __device__ __forceinline__ void wait_step(int n) { wait_later<STAGES - 2>(min(STAGES - 2, nsteps - 1 - n)); }
    __device__ __forceinline__ const uint8_t *stage(int n) const { return ring + (n % STAGES) * kStageBytes<D>; }
};

template <int NW, int STAGES, bool PER_TOKEN, int D, bool V4>
__device__ __forceinline__ void init_stager(KvStager<NW, STAGES, PER_TOKEN, D, V4> &sg, uint8_t *ring, int32_t *pages,
                                            const DecodeParams &p, int h, int tok_lo, int tok_hi,
                                            const int32_t *bt_row, int row_len) {
    sg.ring = ring;
    sg.pages = pages;
    sg.ring_addr = lds_addr(ring);
    sg.bt_row = bt_row;
    sg.row_len = row_len;
    sg.h = h;
    sg.kc_h = p.kc + (int64_t)h * p.s_k_head;
    sg.vc_h = p.vc + (int64_t)h * p.s_v_head;
    sg.bs = 1 << p.bs_log2;
    sg.kchunk = sg.bs * 16;
    sg.tok_lo = tok_lo;
    const int ngroups = (tok_hi - tok_lo + kGroup - 1) / kGroup;
    sg.nsteps = (ngroups + 3) / 4;
    sg.last_group = tok_lo + (ngroups - 1) * kGroup;
    sg.last_page = sg.last_group >> p.bs_log2;
    sg.tid = threadIdx.x;
    sg.lane = threadIdx.x & 63;
    sg.wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    using S = KvStager<NW, STAGES, PER_TOKEN, D, V4>;
    sg.one_page = sg.bs >= kStep && (tok_lo & (kStep - 1)) == 0;
#pragma unroll
    for (int j = 0; j < S::KROWS; ++j) {
        const int r = sg.wave + NW * j;
        const int g = r / S::CPL, c4 = r % S::CPL;
        sg.k_lane[j] = (4 * c4 + (sg.lane >> 4)) * sg.kchunk + g * 256 + (sg.lane & 15) * 16;
        sg.v_lane[j] = g * (V4 ? 16 : 16 * D) + (64 * c4 + sg.lane) * (V4 ? sg.bs : 16);
    }
    const int piece = sg.wave * S::SLANES + min(sg.lane, S::SLANES - 1);
    sg.s_lane = ((piece & 15) >> 2) * 16 + 4 * (piece & 3);
    sg.load_window(tok_lo >> p.bs_log2);
}

// Row-split LDS-staged layout: RS waves each own MTPW row groups of the chunk and
// all take every 64-token step from the ring.
template <int MTPW, int RS, bool PER_TOKEN, int D, bool V4, class Sink>
__device__ __forceinline__ void attend_range_staged(const DecodeParams &p, const int b, const int h, const int ctx,
                                                    const int tok_lo, const int tok_hi, const int32_t *bt_row,
                                                    const int row_len, const int row0, const Sink &sink) {
    constexpr int NW = RS;
    constexpr int CPL = D / 64;
    __shared__ __attribute__((aligned(16))) uint8_t s_ring[kStages * kStageBytes<D>];
    __shared__ int32_t s_pages[kPageWin];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15;
    const int kg = lane >> 4;
    const int row_group0 = (row0 >> 4) + wave * MTPW;

    // every wave is done with the ring and the page window of an earlier range
    wait_vm_barrier<0>();
    if (tok_lo >= tok_hi) {
        emit_empty<D>(NW * 64, row0, min(p.eqgs, row0 + kRowChunk), sink);
        return;
    }
    const float k_fac = PER_TOKEN ? p.qk_scale : p.qk_scale * p.ks[0];
    const float k_eff = logit_scale(k_fac);
    RowSetF8<MTPW, D> rw;
    setup_rows(rw, p, b, h, ctx, tok_lo, tok_hi, row_group0, l16, kg, k_fac < 0.0f);
    const float v_fac = PER_TOKEN ? 1.0f : p.vs[0];
    SmState<MTPW, D> st;
    st.init();
    KvStager<NW, kStages, PER_TOKEN, D, V4> sg{p};
    init_stager(sg, s_ring, s_pages, p, h, tok_lo, tok_hi, bt_row, row_len);
    sg.prologue();
    for (int n = 0; n < sg.nsteps; ++n) {
        sg.wait_step(n);
        // the ring loads go out ahead of the other waves' products on the SIMD
        __builtin_amdgcn_s_setprio(3);
        if (n + kStages - 1 < sg.nsteps) sg.issue(n + kStages - 1);
        __builtin_amdgcn_s_setprio(0);
        // the stage's byte offset as one scalar, so each LDS address below is one add
        const uint8_t *sk = s_ring + __builtin_amdgcn_readfirstlane((n % kStages) * kStageBytes<D>);
        uint4 kr[4][kKChunks<D>];
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
            const uint8_t *kp = sk + (l16 >> 2) * kKGroupStride<D> + (CPL * kg) * 256 + (4 * jt + (l16 & 3)) * 16;
#pragma unroll
            for (int c = 0; c < CPL; ++c) kr[jt][c] = *reinterpret_cast<const uint4 *>(kp + c * 256);
            if constexpr (kKChunks<D> > CPL) kr[jt][CPL] = make_uint4(0u, 0u, 0u, 0u);
        }
        // the scales and V are read from the stage where they are used, which keeps
        // them out of registers during the QK products and the softmax
        const uint8_t *ss = sk + kStageS<D> + kg * 64;
        auto ks_at = [&](int jt) { return *reinterpret_cast<const f32x4 *>(ss + 16 * jt); };
        auto vs_at = [&](int jt) { return *reinterpret_cast<const f32x4 *>(ss + 256 + 16 * jt); };
        bf16x8 pop[MTPW][2];
        step_qk_softmax<MTPW, D, PER_TOKEN, false>(st, rw, kr, ks_at, vs_at, k_eff, tok_lo + n * kStep, kg, pop, [] {});
        uint4 vr[D / 16];
#pragma unroll
        for (int m = 0; m < D / 16; ++m)
            vr[m] = *reinterpret_cast<const uint4 *>(sk + kStageV<D> + kg * (16 * D) + (16 * m + l16) * 16);
        step_pv<MTPW, D>(st, vr, pop);
    }
    finish_rows<MTPW, D>(st, p, row_group0, l16, kg, v_fac, sink);
}

// Layout <MTPW, RS, NS>: NS >= 1 streams K / V through registers (attend_range);
// NS == 0 stages them through LDS for RS waves that all take every step
// (attend_range_staged).
template <int RS, int NS>
constexpr int kThreads = RS * (NS > 0 ? NS : 1) * 64;

template <int MTPW, int RS, int NS, bool PER_TOKEN, int D, bool V4, class Sink>
__device__ __forceinline__ void attend(const DecodeParams &p, int b, int h, int ctx, int tok_lo, int tok_hi,
                                       const int32_t *bt_row, int row_len, int row0, const Sink &sink) {
    if constexpr (NS == 0)
        attend_range_staged<MTPW, RS, PER_TOKEN, D, V4>(p, b, h, ctx, tok_lo, tok_hi, bt_row, row_len, row0, sink);
    else
        attend_range<MTPW, RS, NS, PER_TOKEN, D, V4>(p, b, h, ctx, tok_lo, tok_hi, bt_row, row0, sink);
}

// The work item of a split-context workgroup.  The grid is (B * chunks, Hkv, Z), and
// the workgroups go to the XCDs round-robin in dispatch order (x fastest).  With
// several slot groups per sequence (Z > 1, p.spread) the linear dispatch index is
// read with the row chunk fastest, then the kv head, then the slot group, then the
// sequence: one sequence's items are consecutive and spread over every XCD.  Read as
// the grid's (x, y, z), every item of sequence b goes to XCD b mod 8 (B * Hkv is a
// multiple of 8 in practice), and a ragged batch loads the XCDs as unevenly as its
// lengths: c3 at 8 slots took 300 us that way, 204 us spread.  One workgroup per
// (sequence, kv head) keeps the grid's order, where a sequence's kv heads share their
// XCD's L2 for its page-table row (equal-length batches 0.3-0.8% faster).  The
// chained kernel keeps the grid's order (its layouts hold whole sequences or equal
// slots, and the remap cost it 1-2%).
struct SlotItem {
    int b, h, z, row0;
};
__device__ __forceinline__ SlotItem slot_item(const DecodeParams &p) {
    if (!p.spread) {
        const int b = p.chunks > 1 ? (int)(blockIdx.x / p.chunks) : (int)blockIdx.x;
        return SlotItem{b, (int)blockIdx.y, (int)blockIdx.z, ((int)blockIdx.x - b * max(p.chunks, 1)) * kRowChunk};
    }
    const uint64_t nh = gridDim.y, nz = gridDim.z, nc = p.chunks > 1 ? (uint64_t)p.chunks : 1u;
    uint64_t r = blockIdx.x + (uint64_t)gridDim.x * (blockIdx.y + nh * blockIdx.z);
    const int c = (int)(r % nc);
    r /= nc;
    const int h = (int)(r % nh);
    r /= nh;
    const int z = (int)(r % nz);
    return SlotItem{(int)(r / nz), h, z, c * kRowChunk};
}

// Split-context decode: a workgroup runs partition slot z of kv head h of sequence b,
// query rows [row0, row0 + 64) (slot_item; the row chunks of a slot are adjacent in
// dispatch order, so they read its K / V at about the same time).
template <int MTPW, int RS, int NS, bool PER_TOKEN, int D, bool V4>
__global__ __launch_bounds__((kThreads<RS, NS>), (kWavesFor<MTPW, NS, D>)) void pa_decode_partition_kernel(
    const DecodeParams p) {
    const SlotItem it = slot_item(p);
    const int b = it.b, h = it.h, z = it.z, row0 = it.row0;

    int64_t ctx64 = p.ctx[b];
    const int64_t cap = (int64_t)p.max_blocks << p.bs_log2;
    ctx64 = ctx64 < 0 ? 0 : (ctx64 > cap ? cap : ctx64);
    const int ctx = (int)ctx64;

    // ---- slot -> token range (integer planner, bit-exact with the oracle)
    int tok_lo, tok_hi;
    slot_tokens(p, ctx, z, tok_lo, tok_hi);

    const SlotSink sink{p,
                        p.tmp_out + b * p.s_to_seq + h * p.s_to_head + z * p.s_to_part,
                        p.exp_sums + b * p.s_es_seq + h * p.s_es_head + z * p.s_es_part,
                        p.max_logits + b * p.s_es_seq + h * p.s_es_head + z * p.s_es_part,
                        b,
                        h,
                        p.direct != 0};
    attend<MTPW, RS, NS, PER_TOKEN, D, V4>(p, b, h, ctx, tok_lo, tok_hi, p.bt + (int64_t)b * p.s_bt_seq,
                                           p.max_blocks, row0, sink);
}

// Chained-slot layout: workgroup (b, h, zc) has NW waves; wave w runs the slots
// [(zc * NW + w) * spw, (zc * NW + w + 1) * spw) of (sequence b, kv head h) in turn
// (attend_slots), each writing its slots' partials.  When one workgroup holds every
// slot of its (sequence, kv head) and p.direct is set, its waves then merge those
// partials into the final output themselves (the reduce's arithmetic, lse_merge_row),
// and no reduce launch follows.  Query rows: one 16-row group (ql * g <= 16).
template <int NW, bool PER_TOKEN, int D, bool V4>
__global__ __launch_bounds__(NW * 64, (kWavesPerSimd<1, D>)) void pa_decode_chain_kernel(const DecodeParams p) {
    const int b = blockIdx.x;
    const int h = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int64_t ctx64 = p.ctx[b];
    const int64_t cap = (int64_t)p.max_blocks << p.bs_log2;
    ctx64 = ctx64 < 0 ? 0 : (ctx64 > cap ? cap : ctx64);
    const int ctx = (int)ctx64;
    const int64_t zb = ((int64_t)blockIdx.z * NW + wave) * p.spw;
    const int z0 = (int)min(zb, (int64_t)p.max_parts);
    const int z1 = (int)min(zb + p.spw, (int64_t)p.max_parts);
    // the merge's copy of the partials, when the host sized the dynamic LDS for it
    extern __shared__ __attribute__((aligned(16))) uint8_t s_merge[];
    const bool lds_merge = p.direct && p.max_parts > 1 && p.merge_lds;
    attend_slots<1, PER_TOKEN, D, V4>(p, b, h, ctx, z0, z1, p.bt + (int64_t)b * p.s_bt_seq, 0,
                                      lds_merge ? s_merge : nullptr);
    if (!p.direct || p.max_parts == 1) return;
    // every slot's partial is written (in LDS, or in global memory: a workgroup-scope
    // release and acquire, the waves sharing a CU and none of them having read these
    // rows before)
    __syncthreads();
    constexpr int NB = (D + 127) / 128;
    const int rows = p.max_parts * p.eqgs;
    for (int r = wave; r < p.eqgs; r += NW) {
        const int64_t e0 = b * p.s_es_seq + h * p.s_es_head + r;
        float a0[NB], a1[NB];
        if (lds_merge) {
            const float *les = reinterpret_cast<const float *>(s_merge + rows * kHeadDim * 2);
            lse_merge_row<NB>(les + r, les + rows + r, reinterpret_cast<const uint16_t *>(s_merge) + r * kHeadDim,
                              p.eqgs, p.eqgs * kHeadDim, p.max_parts, D, lane, a0, a1);
        } else {
            lse_merge_row<NB>(p.exp_sums + e0, p.max_logits + e0, p.tmp_out + b * p.s_to_seq + h * p.s_to_head +
                              r * p.s_to_group, p.s_es_part, p.s_to_part, p.max_parts, D, lane, a0, a1);
        }
        const int qi = r / p.g, gi = r - (r / p.g) * p.g;
        const int64_t off = b * p.s_o_seq + qi * p.s_o_len + h * p.s_o_head + gi * p.s_o_group + 2 * lane;
#pragma unroll
        for (int k = 0; k < NB; ++k) {
            if (2 * lane + 128 * k >= D) continue;
            if (p.out_dtype == PA_FP8_F32) {
                float *o = reinterpret_cast<float *>(p.out) + off + 128 * k;
                *reinterpret_cast<float2 *>(o) = make_float2(a0[k], a1[k]);
            } else {
                uint16_t *o = reinterpret_cast<uint16_t *>(p.out) + off + 128 * k;
                *reinterpret_cast<uint32_t *>(o) =
                    p.out_dtype == PA_FP8_F16
                        ? uint32_t(f32_to_f16_bits(a0[k])) | (uint32_t(f32_to_f16_bits(a1[k])) << 16)
                        : uint32_t(f32_to_bf16_bits(a0[k])) | (uint32_t(f32_to_bf16_bits(a1[k])) << 16);
            }
        }
    }
}

// ---------------------------------------------------------------- worklist path
// Where a work's rows go: output[qo_start + qi, qhead] when the work holds its
// whole sequence (pidx < 0), else the f32 partial row pidx + ql + qi plus its
// log-sum-exp (kernels/pa_decode_fp8.py:1612-1643).
struct WorkSink {
    const WorklistParams &w;
    int h, qo_start, pidx;

    template <int N>
    __device__ __forceinline__ void row(int r, int d0, const float (&v)[N]) const {
        const int g = w.kv.g;
        const int qi = r / g, qhead = h * g + (r - qi * g);
        if (pidx < 0) {
            store_out<N>(w.out, w.out_dtype, (int64_t)(qo_start + qi) * w.s_out_seq + qhead * w.s_out_head + d0, v);
            return;
        }
        float *dst = w.po + (int64_t)(pidx + w.kv.ql + qi) * w.s_po_row + qhead * w.head_dim + d0;
#pragma unroll
        for (int j = 0; j < N; j += 4) *reinterpret_cast<float4 *>(dst + j) = make_float4(v[j], v[j + 1], v[j + 2], v[j + 3]);
    }
    __device__ __forceinline__ void stats(int r, float L, float m2) const {
        if (pidx < 0) return;
        const int g = w.kv.g;
        const int qi = r / g, qhead = h * g + (r - qi * g);
        w.pl[(int64_t)(pidx + w.kv.ql + qi) * w.s_pl_row + qhead] = L > 0.f ? m2 * kLn2 + __logf(L) : -INFINITY;
    }
};

// Persistent decode over the get_pa_metadata_v1 worklist: the workgroups of bin c
// run the works [work_indptr[c], work_indptr[c+1]) one after another
// (kernels/pa_decode_fp8.py:941-1721), one workgroup per chunk of 64 query rows
// (adjacent in dispatch order).  With bin_groups = G (and one chunk) the device
// takes the workgroups in G rounds of gridDim/G (one per CU each), and workgroup c
// of round a = c / (gridDim/G) runs a bin of group a of some head: a schedule
// weighted by group then gives the workgroups dispatched first, which issue ahead
// of the later ones on their CU, the larger quotas.  Every field read from the
// worklist is range-checked, so a malformed or overflowed worklist skips work
// instead of touching memory outside the tensors.
template <int MTPW, int RS, int NS, bool PER_TOKEN, int D, bool V4>
__global__ __launch_bounds__((kThreads<RS, NS>), (kWavesFor<MTPW, NS, D>)) void pa_decode_worklist_kernel(
    const WorklistParams w) {
    const DecodeParams &p = w.kv;
    int c = blockIdx.x, row0 = 0;
    if (p.chunks > 1) {
        c = blockIdx.x / p.chunks;
        row0 = (blockIdx.x - c * p.chunks) * kRowChunk;
    } else if (w.bin_groups > 1) {
        const int per_round = w.num_bins / w.bin_groups;  // workgroups per dispatch round
        const int per_group = per_round / w.num_kv_heads;  // bins of one head in one group
        const int a = c / per_round, u = c - a * per_round;
        const int k = u / per_group, j = u - k * per_group;
        c = k * (per_round * w.bin_groups / w.num_kv_heads) + a * per_group + j;
    }
    const int wbeg = max(__builtin_amdgcn_readfirstlane(w.work_indptr[c]), 0);
    const int wend = min(__builtin_amdgcn_readfirstlane(w.work_indptr[c + 1]), w.max_work);
    // A work's fields, and its sequence's page range, context length and partition
    // base, are read with scalar loads (the constant address space: the worklist is
    // read-only here) one work ahead, so the next work's set-up does not start with
    // two dependent memory round trips, and no vector memory wait covers them:
    // c3 kernel 156.3 -> 152.2 us.
    typedef __attribute__((address_space(4))) const int32_t cint;
    struct Fields {
        int b, pidx, qo_start, kv_start, kv_end, qh_start, page0, page1, ctx, pbase;
    };
    auto fields = [&](int wi) {
        Fields r;
        const cint *info = (const cint *)(w.work_info + (int64_t)wi * 8);
        r.b = info[0];
        r.pidx = info[1];
        r.qo_start = info[2];
        r.kv_start = info[4];
        r.kv_end = info[5];
        r.qh_start = info[7] & 0xffff;
        const int bb = min(max(r.b, 0), w.batch - 1);  // batch >= 1 here; out-of-range works are skipped below
        r.page0 = ((const cint *)w.kv_indptr)[bb];
        r.page1 = ((const cint *)w.kv_indptr)[bb + 1];
        r.ctx = ((const cint *)p.ctx)[bb];
        r.pbase = ((const cint *)w.partition_indptr)[bb];
        return r;
    };
    // (The LDS-staged layout reads each work's fields when it starts: the next work's
    // fields would stay live in scalar registers through every step, where that
    // layout's step has none to spare.)
    constexpr bool kAhead = NS > 0;
    Fields nxt{};
    if (kAhead && wbeg < wend) nxt = fields(wbeg);
    for (int wi = wbeg; wi < wend; ++wi) {
        const Fields f = kAhead ? nxt : fields(wi);
        if (kAhead && wi + 1 < wend) nxt = fields(wi + 1);
        const int b = f.b, pidx = f.pidx, qo_start = f.qo_start;
        const int h = f.qh_start / p.g;
        if (b < 0 || b >= w.batch || h >= w.num_kv_heads) continue;
        if (pidx < 0 ? (qo_start < 0 || qo_start > w.output_rows - p.ql)
                     : (pidx > w.partial_rows - 2 * p.ql))
            continue;
        const int page0 = f.page0, page1 = f.page1;
        if (page0 < 0 || page1 < page0 || page1 > w.num_pages) continue;
        int64_t ctx64 = f.ctx;
        const int64_t cap = (int64_t)(page1 - page0) << p.bs_log2;
        ctx64 = ctx64 < 0 ? 0 : (ctx64 > cap ? cap : ctx64);
        const int ctx = (int)ctx64;
        const int64_t lp0 = max((int64_t)f.kv_start - f.pbase, (int64_t)0);
        const int64_t lp1 = (int64_t)f.kv_end - f.pbase;
        const int tok_lo = (int)min(lp0 * kPartition, (int64_t)ctx);
        const int tok_hi = (int)max(min(lp1 * kPartition, (int64_t)ctx), (int64_t)tok_lo);
        const WorkSink sink{w, h, qo_start, pidx};
        attend<MTPW, RS, NS, PER_TOKEN, D, V4>(p, b, h, ctx, tok_lo, tok_hi, w.kv_page_indices + page0,
                                               page1 - page0, row0, sink);
    }
}

// Wave layout per number of 16-row query groups of a chunk (min(ql * g, 64) / 16,
// rounded up):
//   one group    -> <1,1,NS>: NS waves split the steps (1, 2, 4 or 8: waves_per_slot);
//   two groups   -> <2,1,4>: every wave holds both groups, four waves split the steps;
//   3 / 4 groups -> <1,4,0>: one wave per group, the workgroup's steps staged through
//                   an LDS ring that every wave reads.
// Head dims other than 128 run four waves in the one-group layout (at 256 the
// registers allow one wave per SIMD, so eight-wave workgroups would spill), and
// the 4-D value layout four or eight (the launcher's sliding-window and
// persistent paths, which read it, choose those); above 128 two row groups run
// the staged layout (two groups' accumulators per wave would spill).
template <int MTPW, int RS, int NS, bool PT, int D, bool V4>
hipError_t launch_partition(const DecodeParams &p, dim3 grid, hipStream_t s) {
    hipLaunchKernelGGL((pa_decode_partition_kernel<MTPW, RS, NS, PT, D, V4>), grid, dim3((kThreads<RS, NS>)), 0, s, p);
    return hipGetLastError();
}

template <int NW, bool PT, int D, bool V4>
hipError_t launch_chain(const DecodeParams &p, dim3 grid, hipStream_t s) {
    hipLaunchKernelGGL((pa_decode_chain_kernel<NW, PT, D, V4>), grid, dim3(NW * 64), p.merge_lds, s, p);
    return hipGetLastError();
}

template <bool PT, int D, bool V4>
hipError_t dispatch_partition_pt(const DecodeParams &p, int mtp, int waves, dim3 grid, hipStream_t s) {
    if constexpr (D == 128 && !V4) {
        if (p.spw > 0) {  // chained slots (the C ABI admits them for one row group only)
            switch (waves) {
            case 2: return launch_chain<2, PT, D, V4>(p, grid, s);
            case 4: return launch_chain<4, PT, D, V4>(p, grid, s);
            case 8: return launch_chain<8, PT, D, V4>(p, grid, s);
            default: return launch_chain<1, PT, D, V4>(p, grid, s);
            }
        }
    }
    switch (mtp) {
    case 1:
        if constexpr (D == 128) {
            if (waves == 8) return launch_partition<1, 1, 8, PT, D, V4>(p, grid, s);
            if constexpr (!V4) {
                if (waves == 1) return launch_partition<1, 1, 1, PT, D, V4>(p, grid, s);
                if (waves == 2) return launch_partition<1, 1, 2, PT, D, V4>(p, grid, s);
            }
        }
        return launch_partition<1, 1, 4, PT, D, V4>(p, grid, s);
    case 2:
        if constexpr (D <= 128) return launch_partition<2, 1, 4, PT, D, V4>(p, grid, s);
        [[fallthrough]];
    default: return launch_partition<1, 4, 0, PT, D, V4>(p, grid, s);
    }
}

template <int MTPW, int RS, int NS, bool PT, int D, bool V4>
hipError_t launch_worklist(const WorklistParams &w, dim3 grid, hipStream_t s) {
    hipLaunchKernelGGL((pa_decode_worklist_kernel<MTPW, RS, NS, PT, D, V4>), grid, dim3((kThreads<RS, NS>)), 0, s, w);
    return hipGetLastError();
}

template <bool PT, int D, bool V4>
hipError_t dispatch_worklist_pt(const WorklistParams &w, int mtp, dim3 grid, hipStream_t s) {
    switch (mtp) {
    case 1: return launch_worklist<1, 1, 4, PT, D, V4>(w, grid, s);
    case 2:
        if constexpr (D <= 128) return launch_worklist<2, 1, 4, PT, D, V4>(w, grid, s);
        [[fallthrough]];
    default: return launch_worklist<1, 4, 0, PT, D, V4>(w, grid, s);
    }
}

}  // namespace
}  // namespace pa
