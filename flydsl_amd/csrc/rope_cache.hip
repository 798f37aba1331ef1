// gfx950 fused NeoX rotary embedding + paged KV-cache writer (C ABI: pa_fp8_rope_cache).
//
// Work unit: one ROW = one (token, head) vector of Q or K.  A row is handled by
// a power-of-two group of lanes (lanes_per_row = next_pow2(D/16)); lane c owns
// head dims [8c, 8c+8) AND their rotation partners [D/2 + 8c, D/2 + 8c + 8), so
// the NeoX pair (d, d + D/2) sits in one lane and no cross-lane exchange is
// needed for the rotation (the reference gives each lane a contiguous slice and
// fetches the partner with ds_bpermute, kernels/fused_rope_cache_kernel.py:150-177).
// Every load and store of Q/K/V/outputs/cos/sin is one 16-byte vector access.
// Flash-layout head dims that are not a multiple of 16 go to
// rope_cache_narrow_kernel instead (element-wise accesses, same arithmetic).
// Rows of token t are laid out [Q heads..., K heads...] in the flat row index,
// so consecutive lanes stream consecutive bytes of Q then K.  A K row also
// reads V and writes the two cache entries of its token.
//
// Numerics follow the reference kernel (kernels/fused_rope_cache_kernel.py:214-247),
// which computes in the element dtype: every product and the final sum are
// rounded to bf16 / f16 (computed in f32 -- exact products of two 16-bit values --
// then rounded to nearest even).  fp8 cache codes come from v_cvt_pk_fp8_f32
// (round to nearest even; |x| > 464 -> NaN, as torch's float8_e4m3fn cast).
// Per-tensor scales are applied as x * v_rcp_f32(scale), the hardware reciprocal
// the reference takes (:282-283): within 1 ulp of 1/scale, exact at powers of two,
// and not always the correctly rounded quotient (one ulp off at 3.0, and at about
// 11% of scales over a log-uniform sweep), so the cache codes follow the
// reference's bytes at every scale.
#include <hip/hip_runtime.h>
#include <stdint.h>


#include "pa_common.h"
#include "pa_fp8.h"

namespace pa {
// Query / key / value rows are read once and the outputs and cache entries written
// once, so both go with the non-temporal hint (about 3% faster on a 16384-token
// prefill than plain accesses).
#ifndef PA_FP8_NT_WRITER
#define PA_FP8_NT_WRITER 1  // query / key / value row loads with the non-temporal hint
#endif
#ifndef PA_FP8_NT_WRITER_ST
#define PA_FP8_NT_WRITER_ST 1  // 16-byte output and cache stores with the non-temporal hint
#endif

namespace {

constexpr int kRopeThreads = 256;

// n / d for 0 <= n < 2^31 by multiplication (division by an invariant integer,
// Granlund and Montgomery 1994): with l = ceil(log2 d) and
// mul = floor(2^32 (2^l - d) / d) + 1, n / d = (mulhi(n, mul) + n) >> l.  The sum
// stays below 2^32 because n < 2^31.  d = 1 gives mul = 1, l = 0 (n itself); a
// power of two gives mul = 1 (a shift).
struct FastDiv {
    uint32_t mul, shift;
    int32_t d;
};

FastDiv make_fastdiv(int d) {
    uint32_t l = 0;
    while ((uint64_t(1) << l) < uint64_t(d)) ++l;
    const uint64_t m = ((uint64_t(1) << 32) * ((uint64_t(1) << l) - uint64_t(d))) / uint64_t(d) + 1;
    return FastDiv{uint32_t(m), l, d};
}

__device__ __forceinline__ int fdiv(int n, const FastDiv &f) {
    return int((__umulhi(uint32_t(n), f.mul) + uint32_t(n)) >> f.shift);
}

struct RopeParams {
    const uint16_t *q, *k, *v, *cos, *sin;
    const int32_t *pos, *slot;
    uint16_t *qo, *ko;
    uint8_t *kc, *vc;
    float *ks, *vs;
    int64_t sq_t, sq_h, sk_t, sk_h, sv_t, sv_h, sqo_t, sqo_h, sko_t, sko_h, scos, ssin;
    int64_t skc_b, skc_h, skc_t, svc_b, svc_h, svc_t, sks_b, sks_h;
    int64_t q_rows;   // num_tokens * num_q_heads
    int64_t q_tiles;  // workgroups of Q rows (the K/V workgroups follow)
    int32_t T;
    int32_t gather;   // V of the dim-major layouts may be staged through LDS
    int32_t QH, KH, D, bs, nb, max_pos;
    int32_t pos_shift, slot_shift;  // 1: int64 index tensor, low word at element 2t
    int32_t reuse, lpr_log2, chunks;
    FastDiv div_qh, div_kh, div_bs, div_d;  // the launch's divisors (all rows, slots < 2^31)
};

template <int ELEM>
__device__ __forceinline__ float to_f(uint32_t bits16) {
    if constexpr (ELEM == PA_FP8_BF16) return __uint_as_float(bits16 << 16);
    else return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// float -> 16-bit pattern, round to nearest even (v_cvt_pk_bf16_f32 / v_cvt_f16_f32)
template <int ELEM>
__device__ __forceinline__ uint32_t from_f(float f) {
    if constexpr (ELEM == PA_FP8_BF16) return __builtin_bit_cast(uint16_t, (__bf16)f);
    else return f32_to_f16_bits(f);
}

template <int ELEM>
__device__ __forceinline__ float rnd(float f) { return to_f<ELEM>(from_f<ELEM>(f)); }

template <int ELEM>
__device__ __forceinline__ void unpack8(uint4 w, float (&x)[8]) {
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        x[2 * i] = to_f<ELEM>(u[i] & 0xffffu);
        x[2 * i + 1] = to_f<ELEM>(u[i] >> 16);
    }
}

template <int ELEM>
__device__ __forceinline__ uint4 pack8(const float (&x)[8]) {
    uint32_t u[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) u[i] = from_f<ELEM>(x[2 * i]) | (from_f<ELEM>(x[2 * i + 1]) << 16);
    return make_uint4(u[0], u[1], u[2], u[3]);
}

__device__ __forceinline__ uint4 ld16v(const uint16_t *p) { return *reinterpret_cast<const uint4 *>(p); }
__device__ __forceinline__ void st16v(uint16_t *p, uint4 w) {
#if PA_FP8_NT_WRITER_ST
    __builtin_nontemporal_store(u32x4{w.x, w.y, w.z, w.w}, reinterpret_cast<u32x4 *>(p));
#else
    *reinterpret_cast<uint4 *>(p) = w;
#endif
}
// rows of the query / key / value tensors, each read once
__device__ __forceinline__ uint4 ld16row(const uint16_t *p) {
#if PA_FP8_NT_WRITER
    const u32x4 v = ld16_nt(p);
    return make_uint4(v[0], v[1], v[2], v[3]);
#else
    return ld16v(p);
#endif
}

// Eight floats -> eight e4m3fn bytes (two dwords, element i in byte i).
__device__ __forceinline__ uint2 fp8x8(const float (&x)[8]) {
    int w0 = __builtin_amdgcn_cvt_pk_fp8_f32(x[0], x[1], 0, false);
    w0 = __builtin_amdgcn_cvt_pk_fp8_f32(x[2], x[3], w0, true);
    int w1 = __builtin_amdgcn_cvt_pk_fp8_f32(x[4], x[5], 0, false);
    w1 = __builtin_amdgcn_cvt_pk_fp8_f32(x[6], x[7], w1, true);
    return make_uint2((uint32_t)w0, (uint32_t)w1);
}

// nan -> 0, +-inf -> +-448 (pertoken_quant's nan_to_num, tests/utils.py:29-73)
__device__ __forceinline__ float clean448(float x) {
    if (x != x) return 0.0f;
    if (__builtin_isinf(x)) return x > 0.0f ? 448.0f : -448.0f;
    return x;
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Two floats rounded to bf16 (nearest even) by one v_cvt_pk_bf16_f32: the packed
// pair (a in the low half) ...
__device__ __forceinline__ uint32_t bf16_pair_bits(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}
// ... and back as floats.
__device__ __forceinline__ void round_pair_bf16(float &a, float &b) {
    const uint32_t u = bf16_pair_bits(a, b);
    a = __uint_as_float(u << 16);
    b = __uint_as_float(u & 0xffff0000u);
}

// NeoX rotation of one lane's 8 (first-half) + 8 (second-half) elements, rounded
// after each product and after the sum exactly as the element-dtype arithmetic;
// w1 / w2 get the results packed as the output row's 16-bit elements.
// Contraction is off so that no product is fused with the add that follows it
// (v_fma_f16 / v_fma_mix would skip the product's rounding).  f16 computes in
// native IEEE f16 ops; bf16 in f32 with an explicit round after each step, two
// values per conversion (the rounding of each value is that of a conversion of
// its own), the final round of a pair of dims being also its packed output word.
template <int ELEM>
__device__ __forceinline__ void rotate(float (&x1)[8], float (&x2)[8], const float (&c1)[8], const float (&s1)[8],
                                       const float (&c2)[8], const float (&s2)[8], uint4 &w1, uint4 &w2) {
#pragma clang fp contract(off)
    if constexpr (ELEM == PA_FP8_F16) {
        // native IEEE f16 products and sums (v_mul_f16 / v_sub_f16 / v_add_f16)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const _Float16 a = (_Float16)x1[i], b = (_Float16)x2[i];
            const _Float16 p1 = a * (_Float16)c1[i], p2 = b * (_Float16)s1[i];
            const _Float16 p3 = b * (_Float16)c2[i], p4 = a * (_Float16)s2[i];
            x1[i] = (float)(_Float16)(p1 - p2);
            x2[i] = (float)(_Float16)(p3 + p4);
        }
        w1 = pack8<ELEM>(x1);
        w2 = pack8<ELEM>(x2);
    } else {
        uint32_t u1[4], u2[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = 2 * j;
            float p1a = x1[i] * c1[i], p2a = x2[i] * s1[i], p3a = x2[i] * c2[i], p4a = x1[i] * s2[i];
            float p1b = x1[i + 1] * c1[i + 1], p2b = x2[i + 1] * s1[i + 1];
            float p3b = x2[i + 1] * c2[i + 1], p4b = x1[i + 1] * s2[i + 1];
            round_pair_bf16(p1a, p2a);
            round_pair_bf16(p3a, p4a);
            round_pair_bf16(p1b, p2b);
            round_pair_bf16(p3b, p4b);
            u1[j] = bf16_pair_bits(p1a - p2a, p1b - p2b);  // dims i, i + 1 of the first half
            u2[j] = bf16_pair_bits(p3a + p4a, p3b + p4b);  // and of the second half
            x1[i] = __uint_as_float(u1[j] << 16);
            x1[i + 1] = __uint_as_float(u1[j] & 0xffff0000u);
            x2[i] = __uint_as_float(u2[j] << 16);
            x2[i + 1] = __uint_as_float(u2[j] & 0xffff0000u);
        }
        w1 = make_uint4(u1[0], u1[1], u1[2], u1[3]);
        w2 = make_uint4(u2[0], u2[1], u2[2], u2[3]);
    }
}

// Writes one lane's 8 + 8 values of one token into a K (IS_V = false) or V cache.
// Element offsets inside the (block, head) tile:
//   flash      pos*stride_token + d
//   x-packed K (d/16)*(bs*16) + pos*16 + d%16
//   V 4-D      d*bs + pos
//   V trans    (pos/16)*(D*16) + d*16 + pos%16
template <int FMT, int LAYOUT, bool IS_V, int ELEM>
__device__ __forceinline__ void write_cache(uint8_t *tile, int64_t stride_token, int pos, int bs, int D, int d1,
                                            int d2, const float (&x1)[8], const float (&x2)[8]) {
    constexpr int esz = FMT == PA_FP8_CACHE_ELEM ? 2 : 1;
    const bool contiguous8 = LAYOUT == PA_FP8_KV_FLASH || !IS_V;
    if (contiguous8) {
        int64_t o1, o2;
        if (LAYOUT == PA_FP8_KV_FLASH) {
            o1 = int64_t(pos) * stride_token + d1;
            o2 = int64_t(pos) * stride_token + d2;
        } else {
            o1 = int64_t(d1 >> 4) * (bs * 16) + pos * 16 + (d1 & 15);
            o2 = int64_t(d2 >> 4) * (bs * 16) + pos * 16 + (d2 & 15);
        }
        if constexpr (FMT == PA_FP8_CACHE_ELEM) {
            st16v(reinterpret_cast<uint16_t *>(tile + o1 * esz), pack8<ELEM>(x1));
            st16v(reinterpret_cast<uint16_t *>(tile + o2 * esz), pack8<ELEM>(x2));
        } else {
            *reinterpret_cast<uint2 *>(tile + o1) = fp8x8(x1);
            *reinterpret_cast<uint2 *>(tile + o2) = fp8x8(x2);
        }
        return;
    }
    // V, dim-major layouts: one element per head dim, strided
    int64_t base, step;
    if (LAYOUT == PA_FP8_KV_X_PACKED) {
        base = pos;
        step = bs;
    } else {
        base = int64_t(pos >> 4) * (int64_t(D) * 16) + (pos & 15);
        step = 16;
    }
    if constexpr (FMT == PA_FP8_CACHE_ELEM) {
        uint16_t *t16 = reinterpret_cast<uint16_t *>(tile);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            t16[base + int64_t(d1 + i) * step] = (uint16_t)from_f<ELEM>(x1[i]);
            t16[base + int64_t(d2 + i) * step] = (uint16_t)from_f<ELEM>(x2[i]);
        }
    } else {
        const uint2 b1 = fp8x8(x1), b2 = fp8x8(x2);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t w1 = i < 4 ? b1.x : b1.y, w2 = i < 4 ? b2.x : b2.y;
            tile[base + int64_t(d1 + i) * step] = (uint8_t)(w1 >> (8 * (i & 3)));
            tile[base + int64_t(d2 + i) * step] = (uint8_t)(w2 >> (8 * (i & 3)));
        }
    }
}

// One row's inputs as loaded (raw 16-byte vectors) and its indices.
struct RowIn {
    uint4 x1, x2, v1, v2, c1, s1, c2, s2;
    int t, h, slot, praw;
    bool live, is_k;
};

// Loads of one row that depend on nothing but the row (t, h, is_k, live set by the
// caller): position, the Q or K vector, and for K rows the slot and the V vector.
__device__ __forceinline__ void load_row(const RopeParams &p, int d1, int d2, RowIn &r) {
    r.slot = -1;
    if (!r.live) return;
    r.praw = p.pos[int64_t(r.t) << p.pos_shift];
    const uint16_t *x = r.is_k ? p.k + int64_t(r.t) * p.sk_t + int64_t(r.h) * p.sk_h
                               : p.q + int64_t(r.t) * p.sq_t + int64_t(r.h) * p.sq_h;
    r.x1 = ld16row(x + d1);
    r.x2 = ld16row(x + d2);
    if (r.is_k) {
        r.slot = p.slot[int64_t(r.t) << p.slot_shift];
        const uint16_t *vr = p.v + int64_t(r.t) * p.sv_t + int64_t(r.h) * p.sv_h;
        r.v1 = ld16row(vr + d1);
        r.v2 = ld16row(vr + d2);
    }
}

// The cos / sin rows of the row's position (the only loads that wait for another).
__device__ __forceinline__ void load_freqs(const RopeParams &p, int d1, int d2, RowIn &r) {
    if (!r.live) return;
    const int pos = min(max(r.praw, 0), p.max_pos - 1);
    const uint16_t *crow = p.cos + int64_t(pos) * p.scos;
    const uint16_t *srow = p.sin + int64_t(pos) * p.ssin;
    r.c1 = ld16v(crow + d1);
    r.s1 = ld16v(srow + d1);
    if (!p.reuse) {
        r.c2 = ld16v(crow + d2);
        r.s2 = ld16v(srow + d2);
    }
}

// Rotation and output store of one row; returns the rotated values in x1 / x2.
template <int ELEM>
__device__ __forceinline__ void rotate_row(const RopeParams &p, const RowIn &r, int d1, int d2, float (&x1)[8],
                                           float (&x2)[8]) {
    float c1[8], s1[8], c2[8], s2[8];
    unpack8<ELEM>(r.c1, c1);
    unpack8<ELEM>(r.s1, s1);
    if (p.reuse) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            c2[i] = c1[i];
            s2[i] = s1[i];
        }
    } else {
        unpack8<ELEM>(r.c2, c2);
        unpack8<ELEM>(r.s2, s2);
    }
    unpack8<ELEM>(r.x1, x1);
    unpack8<ELEM>(r.x2, x2);
    uint4 w1, w2;
    rotate<ELEM>(x1, x2, c1, s1, c2, s2, w1, w2);
    uint16_t *out = r.is_k ? p.ko + int64_t(r.t) * p.sko_t + int64_t(r.h) * p.sko_h
                           : p.qo + int64_t(r.t) * p.sqo_t + int64_t(r.h) * p.sqo_h;
    st16v(out + d1, w1);
    st16v(out + d2, w2);
}

// Cache element pattern of one value (16-bit element or fp8 code).
template <int FMT, int ELEM>
__device__ __forceinline__ uint32_t cache_bits(float x) {
    if constexpr (FMT == PA_FP8_CACHE_ELEM) return from_f<ELEM>(x);
    else return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x, 0.0f, 0, false) & 0xffu;
}

// K / V rows (K rows of the KV tiles): rotation, output store, cache values and
// writes.  Every thread of the wave calls this (the per-token scale exchange
// needs the whole wave).  With `vstage` the V entry goes to the workgroup's
// staging buffer (row i of the 16-token group, all head dims) instead of memory.
template <int ELEM, int FMT, int LAYOUT>
__device__ __forceinline__ void finish_kv_row(const RopeParams &p, const RowIn &r, int c, int d1, int d2,
                                              float kscale, float vscale, uint16_t *vstage) {
    float x1[8], x2[8], v1[8], v2[8];
    bool write = false;
    if (r.live) {
        rotate_row<ELEM>(p, r, d1, d2, x1, x2);
        write = r.slot >= 0 && fdiv(r.slot, p.div_bs) < p.nb;
        if (write) {
            unpack8<ELEM>(r.v1, v1);
            unpack8<ELEM>(r.v2, v2);
        }
    }
    const int blk = write ? fdiv(r.slot, p.div_bs) : 0;
    const int bpos = write ? r.slot - blk * p.bs : 0;

    if constexpr (FMT == PA_FP8_CACHE_FP8_TENSOR) {
        if (write) {
            const float rk = __builtin_amdgcn_rcpf(kscale);
            const float rv = __builtin_amdgcn_rcpf(vscale);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                x1[i] *= rk;
                x2[i] *= rk;
                v1[i] *= rv;
                v2[i] *= rv;
            }
        }
    } else if constexpr (FMT == PA_FP8_CACHE_FP8_TOKEN) {
        // amax over the row: every lane of the wave takes part in the exchange
        // (lanes without a cache write contribute 0); a row's lanes form an
        // aligned power-of-two group, so the xor butterfly stays inside it.
        float ak = 0.0f, av = 0.0f;
        if (write) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                x1[i] = clean448(x1[i]);
                x2[i] = clean448(x2[i]);
                v1[i] = clean448(v1[i]);
                v2[i] = clean448(v2[i]);
                ak = fmaxf(ak, fmaxf(fabsf(x1[i]), fabsf(x2[i])));
                av = fmaxf(av, fmaxf(fabsf(v1[i]), fabsf(v2[i])));
            }
        }
        for (int m = (1 << p.lpr_log2) >> 1; m >= 1; m >>= 1) {
            ak = fmaxf(ak, __shfl_xor(ak, m, 64));
            av = fmaxf(av, __shfl_xor(av, m, 64));
        }
        if (write) {
            float sk = ak / 448.0f, sv = av / 448.0f;
            if (sk == 0.0f) sk = 1.0f;
            if (sv == 0.0f) sv = 1.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                x1[i] = x1[i] / sk;
                x2[i] = x2[i] / sk;
                v1[i] = v1[i] / sv;
                v2[i] = v2[i] / sv;
            }
            if (c == 0) {
                const int64_t so = int64_t(blk) * p.sks_b + int64_t(r.h) * p.sks_h + bpos;
                p.ks[so] = sk;
                p.vs[so] = sv;
            }
        }
    }
    if (write) {
        constexpr int esz = FMT == PA_FP8_CACHE_ELEM ? 2 : 1;
        uint8_t *kt = p.kc + (int64_t(blk) * p.skc_b + int64_t(r.h) * p.skc_h) * esz;
        write_cache<FMT, LAYOUT, false, ELEM>(kt, p.skc_t, bpos, p.bs, p.D, d1, d2, x1, x2);
        if (vstage) {
            // staging buffer [group][D][16 tokens] of cache elements
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                vstage[(d1 + i) * 16] = (uint16_t)cache_bits<FMT, ELEM>(v1[i]);
                vstage[(d2 + i) * 16] = (uint16_t)cache_bits<FMT, ELEM>(v2[i]);
            }
        } else {
            uint8_t *vt = p.vc + (int64_t(blk) * p.svc_b + int64_t(r.h) * p.svc_h) * esz;
            write_cache<FMT, LAYOUT, true, ELEM>(vt, p.svc_t, bpos, p.bs, p.D, d1, d2, v1, v2);
        }
    }
}

// Grid: Q tiles first, then K/V tiles; a tile is 256 threads = 256 / lanes_per_row
// rows, thread tid handling chunk tid % lanes_per_row of row tid / lanes_per_row.
// Q rows are numbered t * QH + h.  K/V rows are numbered in groups of 16 tokens,
// head-major inside a group: ((t / 16) * KH + h) * 16 + t % 16, so a K/V tile holds
// whole (kv head, 16 consecutive tokens) groups.  When every group of a K/V tile
// goes to one 16-aligned run of slots (a prefill chunk), the V entries of the
// dim-major layouts are staged in LDS and each (head, dim) segment of 16 tokens is
// written with one 16-byte store (two for 16-bit caches); otherwise (decode: one
// token per sequence) each lane writes its own elements.
// Workgroups are dealt round-robin to the 8 XCDs (workgroup w runs on XCD w % 8).
// The remapped index gives XCD x its even share of the Q tiles and of the K/V
// tiles, each a contiguous range: K/V tiles move twice the bytes of Q tiles, so one
// range over both kinds would leave some XCDs all the K/V work, and cache entries
// of neighbouring tokens written element-wise merge in one L2.
template <int ELEM, int FMT, int LAYOUT>
__global__ __launch_bounds__(kRopeThreads) void rope_cache_kernel(RopeParams p) {
    __shared__ __align__(16) uint16_t vstage[kRopeThreads * 16];
    __shared__ int group_slot0[16];
    const int64_t nwg = gridDim.x, w = blockIdx.x;  // nwg = all tiles
    const int64_t x = w & 7, j = w >> 3;
    // XCD x runs n_x = ceil((nwg - x) / 8) workgroups: nq_x Q tiles from qs_x, then
    // the rest K/V tiles from ks_x (the sums of the earlier XCDs' shares)
    const int64_t nq = p.q_tiles > x ? (p.q_tiles - x + 7) >> 3 : 0;
    const int64_t qs = x * (p.q_tiles >> 3) + min(x, p.q_tiles & 7);
    const int64_t ks = x * (nwg >> 3) + min(x, nwg & 7) - qs;
    const int64_t tile = j < nq ? qs + j : p.q_tiles + ks + (j - nq);
    const int lpr_log2 = p.lpr_log2;
    const int c = int(threadIdx.x & ((1u << lpr_log2) - 1));
    const int rpp = kRopeThreads >> lpr_log2;  // rows per tile
    const int lrow = int(threadIdx.x >> lpr_log2);
    const bool lane_live = c < p.chunks;
    const int d1 = 8 * c, d2 = (p.D >> 1) + 8 * c;
    RowIn r;

    if (tile < p.q_tiles) {
        const int64_t row = tile * rpp + lrow;
        r.live = lane_live && row < p.q_rows;
        r.is_k = false;
        r.t = r.live ? fdiv(int(row), p.div_qh) : 0;
        r.h = r.live ? int(row - int64_t(r.t) * p.QH) : 0;
        load_row(p, d1, d2, r);
        load_freqs(p, d1, d2, r);
        if (r.live) {
            float x1[8], x2[8];
            rotate_row<ELEM>(p, r, d1, d2, x1, x2);
        }
        return;
    }

    float kscale = 1.0f, vscale = 1.0f;
    if constexpr (FMT == PA_FP8_CACHE_FP8_TENSOR) {
        kscale = p.ks[0];
        vscale = p.vs[0];
    }
    const int64_t krow = (tile - p.q_tiles) * rpp + lrow;
    const int64_t grp = krow >> 4;  // (token group, head) pair
    const int gi = int(krow & 15);  // token inside the group
    const int64_t tg = fdiv(int(grp), p.div_kh);
    r.h = int(grp - tg * p.KH);
    r.t = int(tg * 16 + gi);
    r.is_k = true;
    r.live = lane_live && r.t < p.T;
    load_row(p, d1, d2, r);
    load_freqs(p, d1, d2, r);

    bool stage = false;
    if (LAYOUT != PA_FP8_KV_FLASH && p.gather) {
        // stage V through LDS when every row of every group in this tile sits at
        // slot0 + i of an aligned run (slot0 = the group's first slot)
        const int slot0 = tg * 16 < p.T ? p.slot[int64_t(tg * 16) << p.slot_shift] : -1;
        const bool run = r.t < p.T && slot0 >= 0 && (slot0 & 15) == 0 && fdiv(slot0, p.div_bs) < p.nb &&
                         r.slot == slot0 + gi;
        stage = __syncthreads_and(run || !lane_live) != 0;
        if (stage && gi == 0 && c == 0) group_slot0[lrow >> 4] = slot0;
    }
    uint16_t *vs_row = stage ? vstage + (lrow >> 4) * (p.D * 16) + gi : nullptr;
    finish_kv_row<ELEM, FMT, LAYOUT>(p, r, c, d1, d2, kscale, vscale, vs_row);
    if (!stage) return;
    __syncthreads();
    // one (group, head dim) segment of 16 tokens per thread
    constexpr int esz = FMT == PA_FP8_CACHE_ELEM ? 2 : 1;
    const int segs = (rpp >> 4) * p.D;
    for (int j = threadIdx.x; j < segs; j += kRopeThreads) {
        const int g = fdiv(j, p.div_d), d = j - g * p.D;
        const int64_t gg = ((tile - p.q_tiles) * rpp >> 4) + g;
        const int h = int(gg - int64_t(fdiv(int(gg), p.div_kh)) * p.KH);
        const int slot0 = group_slot0[g];
        const int blk = fdiv(slot0, p.div_bs), pos0 = slot0 - blk * p.bs;
        const int64_t off = LAYOUT == PA_FP8_KV_X_TRANS ? int64_t(pos0 >> 4) * (int64_t(p.D) * 16) + int64_t(d) * 16
                                                        : int64_t(d) * p.bs + pos0;
        uint8_t *dst = p.vc + (int64_t(blk) * p.svc_b + int64_t(h) * p.svc_h + off) * esz;
        const uint16_t *src = vstage + (g * p.D + d) * 16;
        if constexpr (FMT == PA_FP8_CACHE_ELEM) {
            const uint4 *s4 = reinterpret_cast<const uint4 *>(src);
            reinterpret_cast<uint4 *>(dst)[0] = s4[0];
            reinterpret_cast<uint4 *>(dst)[1] = s4[1];
        } else {
            uint32_t wds[4];
#pragma unroll
            for (int q = 0; q < 4; ++q)
                wds[q] = (src[4 * q] & 0xffu) | ((src[4 * q + 1] & 0xffu) << 8) | ((src[4 * q + 2] & 0xffu) << 16) |
                         ((src[4 * q + 3] & 0xffu) << 24);
            *reinterpret_cast<uint4 *>(dst) = make_uint4(wds[0], wds[1], wds[2], wds[3]);
        }
    }
}

// Flash-layout rows of head dims that are not a multiple of 16 (the reference
// writer takes any head dim its vector-width rule admits,
// kernels/fused_rope_cache_kernel.py:79-96).  Rows are numbered as in
// rope_cache_kernel's Q range, Q rows t * QH + h then K rows t * KH + h; a row
// is handled by an aligned group of L = 2^lpr_log2 lanes (L = next_pow2(D/2),
// at most 64), lane c taking the rotation pairs (j, j + D/2) for j = c, c + L,
// ... < D/2, one 16-bit element per access (consecutive lanes, consecutive
// elements).  Same arithmetic as rotate() and finish_kv_row(), element by element.
constexpr int kNarrowPairs = 8;  // pairs per lane: D/2 <= 8 * 64

template <int ELEM>
__device__ __forceinline__ void rotate1(float &x1, float &x2, float c1, float s1, float c2, float s2) {
#pragma clang fp contract(off)
    if constexpr (ELEM == PA_FP8_F16) {
        const _Float16 a = (_Float16)x1, b = (_Float16)x2;
        const _Float16 p1 = a * (_Float16)c1, p2 = b * (_Float16)s1;
        const _Float16 p3 = b * (_Float16)c2, p4 = a * (_Float16)s2;
        x1 = (float)(_Float16)(p1 - p2);
        x2 = (float)(_Float16)(p3 + p4);
    } else {
        float p1 = x1 * c1, p2 = x2 * s1, p3 = x2 * c2, p4 = x1 * s2;
        round_pair_bf16(p1, p2);
        round_pair_bf16(p3, p4);
        float o1 = p1 - p2, o2 = p3 + p4;
        round_pair_bf16(o1, o2);
        x1 = o1;
        x2 = o2;
    }
}

template <int ELEM, int FMT>
__global__ __launch_bounds__(kRopeThreads) void rope_cache_narrow_kernel(RopeParams p) {
    const int lpr_log2 = p.lpr_log2;
    const int c = int(threadIdx.x & ((1u << lpr_log2) - 1));
    const int64_t row = int64_t(blockIdx.x) * (kRopeThreads >> lpr_log2) + (threadIdx.x >> lpr_log2);
    // whole rows leave together, so the amax exchange below stays among live lanes
    if (row >= p.q_rows + int64_t(p.T) * p.KH) return;
    const int half = p.D >> 1;
    const bool is_k = row >= p.q_rows;
    int t, h;
    if (!is_k) {
        t = fdiv(int(row), p.div_qh);
        h = int(row - int64_t(t) * p.QH);
    } else {
        const int kr = int(row - p.q_rows);
        t = fdiv(kr, p.div_kh);
        h = kr - t * p.KH;
    }
    const int pos = min(max(p.pos[int64_t(t) << p.pos_shift], 0), p.max_pos - 1);
    const uint16_t *x = is_k ? p.k + int64_t(t) * p.sk_t + int64_t(h) * p.sk_h
                             : p.q + int64_t(t) * p.sq_t + int64_t(h) * p.sq_h;
    uint16_t *out = is_k ? p.ko + int64_t(t) * p.sko_t + int64_t(h) * p.sko_h
                         : p.qo + int64_t(t) * p.sqo_t + int64_t(h) * p.sqo_h;
    const uint16_t *crow = p.cos + int64_t(pos) * p.scos;
    const uint16_t *srow = p.sin + int64_t(pos) * p.ssin;
    const int coff = p.reuse ? 0 : half;  // column of the second half's cos / sin
    float x1[kNarrowPairs], x2[kNarrowPairs];
#pragma unroll
    for (int i = 0; i < kNarrowPairs; ++i) {
        const int j = c + (i << lpr_log2);
        x1[i] = x2[i] = 0.0f;
        if (j < half) {
            x1[i] = to_f<ELEM>(x[j]);
            x2[i] = to_f<ELEM>(x[j + half]);
            rotate1<ELEM>(x1[i], x2[i], to_f<ELEM>(crow[j]), to_f<ELEM>(srow[j]), to_f<ELEM>(crow[j + coff]),
                          to_f<ELEM>(srow[j + coff]));
            out[j] = (uint16_t)from_f<ELEM>(x1[i]);
            out[j + half] = (uint16_t)from_f<ELEM>(x2[i]);
        }
    }
    if (!is_k) return;

    const int slot = p.slot[int64_t(t) << p.slot_shift];
    const bool write = slot >= 0 && fdiv(slot, p.div_bs) < p.nb;  // uniform over the row's lanes
    const int blk = write ? fdiv(slot, p.div_bs) : 0;
    const int bpos = write ? slot - blk * p.bs : 0;
    const uint16_t *vr = p.v + int64_t(t) * p.sv_t + int64_t(h) * p.sv_h;
    float v1[kNarrowPairs], v2[kNarrowPairs];
#pragma unroll
    for (int i = 0; i < kNarrowPairs; ++i) {
        const int j = c + (i << lpr_log2);
        v1[i] = v2[i] = 0.0f;
        if (write && j < half) {
            v1[i] = to_f<ELEM>(vr[j]);
            v2[i] = to_f<ELEM>(vr[j + half]);
        }
    }
    float sk = 1.0f, sv = 1.0f;
    if constexpr (FMT == PA_FP8_CACHE_FP8_TENSOR) {
        sk = __builtin_amdgcn_rcpf(p.ks[0]);  // applied as x * rcp(scale)
        sv = __builtin_amdgcn_rcpf(p.vs[0]);
    } else if constexpr (FMT == PA_FP8_CACHE_FP8_TOKEN) {
        float ak = 0.0f, av = 0.0f;
#pragma unroll
        for (int i = 0; i < kNarrowPairs; ++i) {
            x1[i] = clean448(x1[i]);
            x2[i] = clean448(x2[i]);
            v1[i] = clean448(v1[i]);
            v2[i] = clean448(v2[i]);
            ak = fmaxf(ak, fmaxf(fabsf(x1[i]), fabsf(x2[i])));
            av = fmaxf(av, fmaxf(fabsf(v1[i]), fabsf(v2[i])));
        }
        for (int m = (1 << lpr_log2) >> 1; m >= 1; m >>= 1) {
            ak = fmaxf(ak, __shfl_xor(ak, m, 64));
            av = fmaxf(av, __shfl_xor(av, m, 64));
        }
        sk = ak / 448.0f;
        sv = av / 448.0f;
        if (sk == 0.0f) sk = 1.0f;
        if (sv == 0.0f) sv = 1.0f;
        if (write && c == 0) {
            const int64_t so = int64_t(blk) * p.sks_b + int64_t(h) * p.sks_h + bpos;
            p.ks[so] = sk;
            p.vs[so] = sv;
        }
    }
    if (!write) return;
    constexpr int esz = FMT == PA_FP8_CACHE_ELEM ? 2 : 1;
    uint8_t *kt = p.kc + (int64_t(blk) * p.skc_b + int64_t(bpos) * p.skc_t + int64_t(h) * p.skc_h) * esz;
    uint8_t *vt = p.vc + (int64_t(blk) * p.svc_b + int64_t(bpos) * p.svc_t + int64_t(h) * p.svc_h) * esz;
#pragma unroll
    for (int i = 0; i < kNarrowPairs; ++i) {
        const int j = c + (i << lpr_log2);
        if (j >= half) continue;
        float k1 = x1[i], k2 = x2[i], w1 = v1[i], w2 = v2[i];
        if constexpr (FMT == PA_FP8_CACHE_FP8_TENSOR) {
            k1 *= sk;
            k2 *= sk;
            w1 *= sv;
            w2 *= sv;
        } else if constexpr (FMT == PA_FP8_CACHE_FP8_TOKEN) {
            k1 = k1 / sk;
            k2 = k2 / sk;
            w1 = w1 / sv;
            w2 = w2 / sv;
        }
        if constexpr (FMT == PA_FP8_CACHE_ELEM) {
            uint16_t *k16 = reinterpret_cast<uint16_t *>(kt), *v16 = reinterpret_cast<uint16_t *>(vt);
            k16[j] = (uint16_t)from_f<ELEM>(k1);
            k16[j + half] = (uint16_t)from_f<ELEM>(k2);
            v16[j] = (uint16_t)from_f<ELEM>(w1);
            v16[j + half] = (uint16_t)from_f<ELEM>(w2);
        } else {
            kt[j] = (uint8_t)cache_bits<FMT, ELEM>(k1);
            kt[j + half] = (uint8_t)cache_bits<FMT, ELEM>(k2);
            vt[j] = (uint8_t)cache_bits<FMT, ELEM>(w1);
            vt[j + half] = (uint8_t)cache_bits<FMT, ELEM>(w2);
        }
    }
}

template <int ELEM>
hipError_t launch_narrow(const RopeParams &p, int fmt, dim3 grid, hipStream_t s) {
    switch (fmt) {
    case PA_FP8_CACHE_ELEM:
        hipLaunchKernelGGL((rope_cache_narrow_kernel<ELEM, PA_FP8_CACHE_ELEM>), grid, dim3(kRopeThreads), 0, s, p);
        break;
    case PA_FP8_CACHE_FP8_TENSOR:
        hipLaunchKernelGGL((rope_cache_narrow_kernel<ELEM, PA_FP8_CACHE_FP8_TENSOR>), grid, dim3(kRopeThreads), 0, s,
                           p);
        break;
    default:
        hipLaunchKernelGGL((rope_cache_narrow_kernel<ELEM, PA_FP8_CACHE_FP8_TOKEN>), grid, dim3(kRopeThreads), 0, s,
                           p);
        break;
    }
    return hipGetLastError();
}

template <int ELEM, int FMT>
hipError_t launch_layout(const RopeParams &p, int layout, dim3 grid, hipStream_t s) {
    switch (layout) {
    case PA_FP8_KV_FLASH:
        hipLaunchKernelGGL((rope_cache_kernel<ELEM, FMT, PA_FP8_KV_FLASH>), grid, dim3(kRopeThreads), 0, s, p);
        break;
    case PA_FP8_KV_X_PACKED:
        hipLaunchKernelGGL((rope_cache_kernel<ELEM, FMT, PA_FP8_KV_X_PACKED>), grid, dim3(kRopeThreads), 0, s, p);
        break;
    default:
        hipLaunchKernelGGL((rope_cache_kernel<ELEM, FMT, PA_FP8_KV_X_TRANS>), grid, dim3(kRopeThreads), 0, s, p);
        break;
    }
    return hipGetLastError();
}

template <int ELEM>
hipError_t launch_format(const RopeParams &p, int fmt, int layout, dim3 grid, hipStream_t s) {
    switch (fmt) {
    case PA_FP8_CACHE_ELEM: return launch_layout<ELEM, PA_FP8_CACHE_ELEM>(p, layout, grid, s);
    case PA_FP8_CACHE_FP8_TENSOR: return launch_layout<ELEM, PA_FP8_CACHE_FP8_TENSOR>(p, layout, grid, s);
    default: return launch_layout<ELEM, PA_FP8_CACHE_FP8_TOKEN>(p, layout, grid, s);
    }
}

inline bool aligned(const void *ptr, uintptr_t a) { return (reinterpret_cast<uintptr_t>(ptr) & (a - 1)) == 0; }

// pa_fp8_rope_cache for flash-layout head dims that are not a multiple of 16 (the
// caller has checked the head dim, shape and layout fields): 16-bit tensors
// need only 2-byte alignment and any non-negative strides.
int rope_cache_narrow(const pa_fp8_rope_cache_args *a, void *hip_stream) {
    const void *p16[] = {a->query, a->key, a->value, a->cos_cache, a->sin_cache, a->query_out, a->key_out};
    for (const void *ptr : p16)
        if (!aligned(ptr, 2)) return PA_FP8_ERR_SHAPE;
    const int64_t st[] = {a->stride_q_token,  a->stride_q_head,   a->stride_k_token,  a->stride_k_head,
                          a->stride_v_token,  a->stride_v_head,   a->stride_qo_token, a->stride_qo_head,
                          a->stride_ko_token, a->stride_ko_head,  a->stride_cos_pos,  a->stride_sin_pos,
                          a->stride_kc_block, a->stride_kc_head,  a->stride_kc_token, a->stride_vc_block,
                          a->stride_vc_head,  a->stride_vc_token};
    for (int64_t s : st)
        if (s < 0) return PA_FP8_ERR_SHAPE;
    if (a->cache_format == PA_FP8_CACHE_ELEM && (!aligned(a->key_cache, 2) || !aligned(a->value_cache, 2)))
        return PA_FP8_ERR_SHAPE;
    if (a->cache_format == PA_FP8_CACHE_FP8_TOKEN && (a->stride_ks_block < 0 || a->stride_ks_head < 0))
        return PA_FP8_ERR_SHAPE;
    if (a->num_tokens == 0) return PA_FP8_OK;
    const int half = a->head_dim / 2;
    int lpr_log2 = 0;
    while ((1 << lpr_log2) < half && lpr_log2 < 6) ++lpr_log2;
    RopeParams p{};
    p.q = static_cast<const uint16_t *>(a->query);
    p.k = static_cast<const uint16_t *>(a->key);
    p.v = static_cast<const uint16_t *>(a->value);
    p.cos = static_cast<const uint16_t *>(a->cos_cache);
    p.sin = static_cast<const uint16_t *>(a->sin_cache);
    p.pos = static_cast<const int32_t *>(a->positions);
    p.slot = static_cast<const int32_t *>(a->slot_mapping);
    p.qo = static_cast<uint16_t *>(a->query_out);
    p.ko = static_cast<uint16_t *>(a->key_out);
    p.kc = static_cast<uint8_t *>(a->key_cache);
    p.vc = static_cast<uint8_t *>(a->value_cache);
    p.ks = a->key_scale;
    p.vs = a->value_scale;
    p.sq_t = a->stride_q_token;
    p.sq_h = a->stride_q_head;
    p.sk_t = a->stride_k_token;
    p.sk_h = a->stride_k_head;
    p.sv_t = a->stride_v_token;
    p.sv_h = a->stride_v_head;
    p.sqo_t = a->stride_qo_token;
    p.sqo_h = a->stride_qo_head;
    p.sko_t = a->stride_ko_token;
    p.sko_h = a->stride_ko_head;
    p.scos = a->stride_cos_pos;
    p.ssin = a->stride_sin_pos;
    p.skc_b = a->stride_kc_block;
    p.skc_h = a->stride_kc_head;
    p.skc_t = a->stride_kc_token;
    p.svc_b = a->stride_vc_block;
    p.svc_h = a->stride_vc_head;
    p.svc_t = a->stride_vc_token;
    p.sks_b = a->stride_ks_block;
    p.sks_h = a->stride_ks_head;
    p.QH = a->num_q_heads;
    p.KH = a->num_kv_heads;
    p.D = a->head_dim;
    p.bs = a->block_size;
    p.nb = a->num_blocks;
    p.max_pos = a->max_pos;
    p.pos_shift = a->positions_i64 ? 1 : 0;
    p.slot_shift = a->slots_i64 ? 1 : 0;
    p.reuse = a->reuse_freqs_front_part ? 1 : 0;
    p.lpr_log2 = lpr_log2;
    p.T = a->num_tokens;
    p.q_rows = int64_t(a->num_tokens) * a->num_q_heads;
    const int64_t rows = p.q_rows + int64_t(a->num_tokens) * a->num_kv_heads;
    const int64_t rpp = kRopeThreads >> lpr_log2;
    const int64_t blocks = (rows + rpp - 1) / rpp;
    // rows, K rows and slots are divided as 31-bit values
    if (blocks > 0x7fffffffLL || blocks * rpp > 0x7fffffffLL) return PA_FP8_ERR_SHAPE;
    p.div_qh = make_fastdiv(a->num_q_heads);
    p.div_kh = make_fastdiv(a->num_kv_heads);
    p.div_bs = make_fastdiv(a->block_size);
    p.div_d = make_fastdiv(a->head_dim);
    const dim3 grid((unsigned)blocks);
    hipStream_t s = static_cast<hipStream_t>(hip_stream);
    const hipError_t e = a->elem_dtype == PA_FP8_BF16 ? launch_narrow<PA_FP8_BF16>(p, a->cache_format, grid, s)
                                                      : launch_narrow<PA_FP8_F16>(p, a->cache_format, grid, s);
    return e == hipSuccess ? PA_FP8_OK : PA_FP8_ERR_HIP + int(e);
}

__global__ __launch_bounds__(256) void hw_reciprocal_kernel(const float *x, float *y, int64_t n) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) y[i] = __builtin_amdgcn_rcpf(x[i]);
}

}  // namespace
}  // namespace pa

extern "C" int pa_fp8_rope_cache(const pa_fp8_rope_cache_args *a, void *hip_stream) {
    using namespace pa;
    if (!a) return PA_FP8_ERR_NULL_POINTER;
    // per-token tensors may be empty (NULL) when there are no tokens
    if (a->num_tokens != 0 && (!a->query || !a->key || !a->value || !a->positions || !a->slot_mapping ||
                               !a->query_out || !a->key_out))
        return PA_FP8_ERR_NULL_POINTER;
    if (!a->cos_cache || !a->sin_cache || !a->key_cache || !a->value_cache) return PA_FP8_ERR_NULL_POINTER;
    if (a->elem_dtype != PA_FP8_BF16 && a->elem_dtype != PA_FP8_F16) return PA_FP8_ERR_DTYPE;
    if (a->cache_format < PA_FP8_CACHE_ELEM || a->cache_format > PA_FP8_CACHE_FP8_TOKEN) return PA_FP8_ERR_LAYOUT;
    if (a->kv_layout < PA_FP8_KV_FLASH || a->kv_layout > PA_FP8_KV_X_TRANS) return PA_FP8_ERR_LAYOUT;
    if (a->cache_format != PA_FP8_CACHE_ELEM && (!a->key_scale || !a->value_scale)) return PA_FP8_ERR_NULL_POINTER;
    const int D = a->head_dim;
    // head dims off the 16-dim grid: flash layout only, element-wise accesses
    const bool narrow = a->kv_layout == PA_FP8_KV_FLASH && D % 16 != 0;
    if (narrow ? (D < 2 || D > 1024 || D % 2 != 0) : (D < 16 || D > 1024 || D % 16 != 0)) return PA_FP8_ERR_HEAD_DIM;
    if (a->num_tokens < 0 || a->num_q_heads < 1 || a->num_kv_heads < 1 || a->block_size < 1 || a->num_blocks < 1 ||
        a->max_pos < 1)
        return PA_FP8_ERR_SHAPE;
    if (int64_t(a->num_q_heads) + a->num_kv_heads > (1 << 20)) return PA_FP8_ERR_SHAPE;
    if (a->kv_layout == PA_FP8_KV_X_TRANS && a->block_size % 16 != 0) return PA_FP8_ERR_LAYOUT;
    if (narrow) return rope_cache_narrow(a, hip_stream);
    // 16-byte vector rows for every 16-bit tensor
    const void *p16[] = {a->query, a->key, a->value, a->cos_cache, a->sin_cache, a->query_out, a->key_out};
    for (const void *ptr : p16)
        if (!aligned(ptr, 16)) return PA_FP8_ERR_SHAPE;
    const int64_t s16[] = {a->stride_q_token,  a->stride_q_head,  a->stride_k_token,  a->stride_k_head,
                           a->stride_v_token,  a->stride_v_head,  a->stride_qo_token, a->stride_qo_head,
                           a->stride_ko_token, a->stride_ko_head, a->stride_cos_pos,  a->stride_sin_pos};
    for (int64_t s : s16)
        if (s < 0 || s % 8 != 0) return PA_FP8_ERR_SHAPE;
    // caches: 16-byte (16-bit cache) or 8-byte (fp8) runs of 8 head dims
    const uintptr_t ca = a->cache_format == PA_FP8_CACHE_ELEM ? 16 : 8;
    if (!aligned(a->key_cache, ca) || !aligned(a->value_cache, ca)) return PA_FP8_ERR_SHAPE;
    const int64_t sc[] = {a->stride_kc_block, a->stride_kc_head, a->stride_vc_block, a->stride_vc_head};
    for (int64_t s : sc)
        if (s < 0 || s % 8 != 0) return PA_FP8_ERR_SHAPE;
    if (a->kv_layout == PA_FP8_KV_FLASH && (a->stride_kc_token < 0 || a->stride_kc_token % 8 != 0 ||
                                            a->stride_vc_token < 0 || a->stride_vc_token % 8 != 0))
        return PA_FP8_ERR_SHAPE;
    if (a->cache_format == PA_FP8_CACHE_FP8_TOKEN && (a->stride_ks_block < 0 || a->stride_ks_head < 0))
        return PA_FP8_ERR_SHAPE;
    if (a->num_tokens == 0) return PA_FP8_OK;

    const int chunks = D / 16;
    int lpr_log2 = 0;
    while ((1 << lpr_log2) < chunks) ++lpr_log2;
    RopeParams p;
    p.q = static_cast<const uint16_t *>(a->query);
    p.k = static_cast<const uint16_t *>(a->key);
    p.v = static_cast<const uint16_t *>(a->value);
    p.cos = static_cast<const uint16_t *>(a->cos_cache);
    p.sin = static_cast<const uint16_t *>(a->sin_cache);
    p.pos = static_cast<const int32_t *>(a->positions);
    p.slot = static_cast<const int32_t *>(a->slot_mapping);
    p.qo = static_cast<uint16_t *>(a->query_out);
    p.ko = static_cast<uint16_t *>(a->key_out);
    p.kc = static_cast<uint8_t *>(a->key_cache);
    p.vc = static_cast<uint8_t *>(a->value_cache);
    p.ks = a->key_scale;
    p.vs = a->value_scale;
    p.sq_t = a->stride_q_token;
    p.sq_h = a->stride_q_head;
    p.sk_t = a->stride_k_token;
    p.sk_h = a->stride_k_head;
    p.sv_t = a->stride_v_token;
    p.sv_h = a->stride_v_head;
    p.sqo_t = a->stride_qo_token;
    p.sqo_h = a->stride_qo_head;
    p.sko_t = a->stride_ko_token;
    p.sko_h = a->stride_ko_head;
    p.scos = a->stride_cos_pos;
    p.ssin = a->stride_sin_pos;
    p.skc_b = a->stride_kc_block;
    p.skc_h = a->stride_kc_head;
    p.skc_t = a->stride_kc_token;
    p.svc_b = a->stride_vc_block;
    p.svc_h = a->stride_vc_head;
    p.svc_t = a->stride_vc_token;
    p.sks_b = a->stride_ks_block;
    p.sks_h = a->stride_ks_head;
    p.QH = a->num_q_heads;
    p.KH = a->num_kv_heads;
    p.D = D;
    p.bs = a->block_size;
    p.nb = a->num_blocks;
    p.max_pos = a->max_pos;
    p.pos_shift = a->positions_i64 ? 1 : 0;
    p.slot_shift = a->slots_i64 ? 1 : 0;
    p.reuse = a->reuse_freqs_front_part ? 1 : 0;
    p.lpr_log2 = lpr_log2;
    p.chunks = chunks;
    const int64_t rpp = kRopeThreads >> lpr_log2;
    p.T = a->num_tokens;
    p.q_rows = int64_t(a->num_tokens) * a->num_q_heads;
    p.q_tiles = (p.q_rows + rpp - 1) / rpp;
    const int64_t kv_rows = (int64_t(a->num_tokens) + 15) / 16 * 16 * a->num_kv_heads;
    const int64_t blocks = p.q_tiles + (kv_rows + rpp - 1) / rpp;
    // row indices, (token group, head) indices and slots are divided as 31-bit values
    if (blocks > 0x7fffffffLL || (p.q_tiles + 1) * rpp > 0x7fffffffLL || kv_rows + rpp > 0x7fffffffLL)
        return PA_FP8_ERR_SHAPE;
    p.div_qh = make_fastdiv(a->num_q_heads);
    p.div_kh = make_fastdiv(a->num_kv_heads);
    p.div_bs = make_fastdiv(a->block_size);
    p.div_d = make_fastdiv(D);
    // staged V writes: whole 16-token groups per workgroup, 16-aligned runs inside a
    // page, 16-byte aligned (block, head) tiles
    const int64_t esz = a->cache_format == PA_FP8_CACHE_ELEM ? 2 : 1;
    p.gather = rpp >= 16 && a->block_size % 16 == 0 && aligned(a->value_cache, 16) &&
               (a->stride_vc_block * esz) % 16 == 0 && (a->stride_vc_head * esz) % 16 == 0;
    const dim3 grid((unsigned)blocks);
    hipStream_t s = static_cast<hipStream_t>(hip_stream);
    const hipError_t e = a->elem_dtype == PA_FP8_BF16
                             ? launch_format<PA_FP8_BF16>(p, a->cache_format, a->kv_layout, grid, s)
                             : launch_format<PA_FP8_F16>(p, a->cache_format, a->kv_layout, grid, s);
    return e == hipSuccess ? PA_FP8_OK : PA_FP8_ERR_HIP + int(e);
}

extern "C" int pa_fp8_hw_reciprocal(const float *x, float *y, int64_t n, void *hip_stream) {
    if (n < 0) return PA_FP8_ERR_SHAPE;
    if (n > 0 && (x == nullptr || y == nullptr)) return PA_FP8_ERR_NULL_POINTER;
    if (n == 0) return PA_FP8_OK;
    if ((n + 255) / 256 > 0x7fffffffLL) return PA_FP8_ERR_SHAPE;
    hipLaunchKernelGGL(pa::hw_reciprocal_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(hip_stream), x, y, n);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? PA_FP8_OK : PA_FP8_ERR_HIP + int(e);
}
