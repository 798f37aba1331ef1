// Shared device helpers for the gfx950 paged-attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kHeadDim = 128;           // D
constexpr int kPartition = 256;         // tokens per context partition (reference KV_COMPUTE_BLOCK)
constexpr int kGroup = 16;              // tokens per MFMA token group
constexpr int kStep = 64;               // tokens per wave step (4 groups)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kSlack = 8.0f;          // log2 headroom before the online-softmax reference max is raised

// Four fp8 e4m3fn bytes -> four bf16 (exact: every e4m3fn value is a bf16 value).
__device__ __forceinline__ bf16x4 fp8x4_to_bf16x4(uint32_t w) {
    bf16x2 lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
    bf16x2 hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true);
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3);
}

// Eight fp8 bytes (two dwords, little-endian byte order) -> bf16x8.
__device__ __forceinline__ bf16x8 fp8x8_to_bf16x8(uint32_t w0, uint32_t w1) {
    bf16x4 a = fp8x4_to_bf16x4(w0);
    bf16x4 b = fp8x4_to_bf16x4(w1);
    return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

__device__ __forceinline__ f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

typedef int i32x8 __attribute__((ext_vector_type(8)));

// C[16x16] += A[16x128] B[128x16] 2^(sb - 127): fp8 e4m3fn operands, f32
// accumulation, B's E8M0 block scale from byte 0 of sb, A's 2^0
// (v_mfma_scale_f32_16x16x128_f8f6f4).  Lane l holds row / column l % 16; its
// bytes j < 16 are k = 16 (l / 16) + j and its bytes j >= 16 are
// k = 64 + 16 (l / 16) + j - 16.  The scale of column c, k block q
// (k in [32 q, 32 q + 32)) comes from lane c + 16 q, so it covers bytes of two
// lanes, and only a scale that varies with the column alone (the same in lanes
// c, c + 16, c + 32, c + 48) is exact.  Any placement of k that A and B share
// gives the same product, so the operands only keep A and B alike.  (Layout and
// scale lanes measured on the GPU against host products.)
__device__ __forceinline__ f32x4 mfma_fp8_k128(i32x8 a, i32x8 b, f32x4 c, int sb) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, sb);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float shfl_xor_f(float v, int mask) { return __shfl_xor(v, mask, 64); }

// max(a, b) as one v_max_f32 (the compiler's fmaxf adds a NaN-quieting move per
// operand that comes from another lane; the values here are finite or -inf).
__device__ __forceinline__ float max_raw(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// max of v over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (the four 16-lane rows), with
// the gfx950 row swaps (v_permlane16_swap / v_permlane32_swap: no lane-index
// arithmetic, no LDS): each swap hands every lane its partner row's value.
__device__ __forceinline__ float rows4_max(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const float m = max_raw(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    return max_raw(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// Lane J of each quad of lanes (4q .. 4q+3) to the whole quad: a DPP quad_perm
// broadcast (a VALU move, no LDS).
template <int J>
__device__ __forceinline__ float quad_bcast(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), J * 0x55, 0xf, 0xf, true));
}

// out[j] = piece of quad lane j, for j = 0..3.
__device__ __forceinline__ void quad_gather(const f32x4 &piece, f32x4 (&out)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        out[0][i] = quad_bcast<0>(piece[i]);
        out[1][i] = quad_bcast<1>(piece[i]);
        out[2][i] = quad_bcast<2>(piece[i]);
        out[3][i] = quad_bcast<3>(piece[i]);
    }
}

// 16 bytes with the non-temporal hint (data read once).
__device__ __forceinline__ u32x4 ld16_nt(const void *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}

// K / V are read once per decode step, and loading them with the non-temporal hint
// keeps them from displacing what is reused (page rows, scales, queries): c2
// 94.6 -> 87.9 us, c4 50.2 -> 46.0 us, c3 and c5 2-3% faster.
#ifndef PA_FP8_NT_KV
#define PA_FP8_NT_KV 1  // K / V loads with the non-temporal hint
#endif
__device__ __forceinline__ uint4 ld16(const uint8_t *p) {
#if PA_FP8_NT_KV
    const u32x4 v = ld16_nt(p);
    return make_uint4(v[0], v[1], v[2], v[3]);
#else
    return *reinterpret_cast<const uint4 *>(p);
#endif
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }

// float -> bf16 bits, round to nearest even (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return uint16_t(u >> 16);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    _Float16 h = (_Float16)f;
    return __builtin_bit_cast(uint16_t, h);
}

// Log-sum-exp merge of the P partials of R query rows (the first nrows <= R of them):
// lane owns head dims 2*lane, 2*lane+1 of each 128-dim block (a0 / a1 per row and
// block; NB blocks).  es / ml point at row 0's exp_sum / max_logit of slot 0 (row q at
// + q * s_es_row), to at row 0's bf16 partial row of slot 0 (row q at + q * s_to_row).
// out = sum_z w_z to_z with w_z = s_z e^(m_z - M) / sum_z s_z e^(m_z - M), M = max_z m_z
// (kernels/pa_decode_swa.py:954-1130).  Both the reduce kernel and the chained
// kernel's in-workgroup merge run this, so their outputs are identical; each row's
// arithmetic is the same whatever R and nrows are, the rows only share the memory
// round trips.  Each slot's weight is computed in its own lane and broadcast with
// readlane; the rows of kMergeChunk slots with nonzero weights are loaded together
// (one memory round trip per chunk) and added in slot order.  A slot of weight 0 (an
// empty slot, whose row may hold anything) is neither loaded nor added.
constexpr int kMergeChunk = 8;
template <int NB, int R>
__device__ __forceinline__ void lse_merge_rows(const float *es, const float *ml, const uint16_t *to, int64_t s_es_row,
                                               int64_t s_to_row, int64_t s_es_part, int64_t s_to_part, int P,
                                               int head_dim, int lane, int nrows, float (&a0)[R][NB],
                                               float (&a1)[R][NB]) {
    constexpr int CH = R > 1 ? kMergeChunk / 2 : kMergeChunk;  // slots per chunk (registers: R * CH * NB)
    // the first 64 slots' exp_sums and max_logits, one per lane, loaded once for all
    // three passes (later slots are read again where a pass needs them)
    float es0[R], ml0[R], Ms[R], inv[R];
#pragma unroll
    for (int q = 0; q < R; ++q) {
        const bool in = q < nrows && lane < P;
        es0[q] = in ? es[q * s_es_row + lane * s_es_part] : 0.f;
        ml0[q] = in ? ml[q * s_es_row + lane * s_es_part] : 0.f;
    }
#pragma unroll
    for (int q = 0; q < R; ++q) {
        Ms[q] = 0.f;
        if (q >= nrows) continue;
        const float *mq = ml + q * s_es_row;
        float mloc = -INFINITY;
        if (lane < P) mloc = fmaxf(mloc, ml0[q]);
        for (int z = lane + 64; z < P; z += 64) mloc = fmaxf(mloc, mq[z * s_es_part]);
#pragma unroll
        for (int sh = 32; sh >= 1; sh >>= 1) mloc = fmaxf(mloc, shfl_xor_f(mloc, sh));
        Ms[q] = mloc == -INFINITY ? 0.0f : mloc;
    }
#pragma unroll
    for (int q = 0; q < R; ++q) {
        inv[q] = 0.f;
        if (q >= nrows) continue;
        const float *eq = es + q * s_es_row, *mq = ml + q * s_es_row;
        float wl = 0.f;
        if (lane < P) wl += es0[q] * fast_exp2((ml0[q] - Ms[q]) * kLog2e);
        for (int z = lane + 64; z < P; z += 64) {
            const float mz = mq[z * s_es_part];
            wl += eq[z * s_es_part] * fast_exp2((mz - Ms[q]) * kLog2e);
        }
#pragma unroll
        for (int sh = 32; sh >= 1; sh >>= 1) wl += shfl_xor_f(wl, sh);
        inv[q] = wl > 0.f ? 1.0f / wl : 0.0f;
    }
#pragma unroll
    for (int q = 0; q < R; ++q)
#pragma unroll
        for (int k = 0; k < NB; ++k) a0[q][k] = a1[q][k] = 0.f;
    for (int z0 = 0; z0 < P; z0 += 64) {
        const int z = z0 + lane, n = min(P - z0, 64);
        float wz[R];
#pragma unroll
        for (int q = 0; q < R; ++q) {
            const float *eq = es + q * s_es_row, *mq = ml + q * s_es_row;
            const float ez = z0 == 0 ? es0[q] : (z < P ? eq[z * s_es_part] : 0.f);
            const float mz = z0 == 0 ? ml0[q] : (z < P ? mq[z * s_es_part] : 0.f);
            wz[q] = q < nrows && z < P ? ez * fast_exp2((mz - Ms[q]) * kLog2e) * inv[q] : 0.f;
        }
        for (int j0 = 0; j0 < n; j0 += CH) {
            float w[R][CH];
            uint32_t two[R][CH][NB];
#pragma unroll
            for (int q = 0; q < R; ++q)
#pragma unroll
                for (int j = 0; j < CH; ++j)
                    w[q][j] = q < nrows && j0 + j < n
                                  ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wz[q]),
                                                                                        j0 + j))
                                  : 0.f;
#pragma unroll
            for (int q = 0; q < R; ++q)
#pragma unroll
                for (int j = 0; j < CH; ++j)
#pragma unroll
                    for (int k = 0; k < NB; ++k)
                        two[q][j][k] = w[q][j] != 0.f && 2 * lane + 128 * k < head_dim
                                           ? *reinterpret_cast<const uint32_t *>(to + q * s_to_row +
                                                                                 (z0 + j0 + j) * s_to_part + 128 * k +
                                                                                 2 * lane)
                                           : 0u;
#pragma unroll
            for (int q = 0; q < R; ++q)
#pragma unroll
                for (int j = 0; j < CH; ++j) {
                    if (w[q][j] == 0.f) continue;
#pragma unroll
                    for (int k = 0; k < NB; ++k) {
                        if (2 * lane + 128 * k >= head_dim) continue;
                        a0[q][k] += w[q][j] * bf16_bits_to_f32(uint16_t(two[q][j][k] & 0xffffu));
                        a1[q][k] += w[q][j] * bf16_bits_to_f32(uint16_t(two[q][j][k] >> 16));
                    }
                }
        }
    }
}

// One row of lse_merge_rows.
template <int NB>
__device__ __forceinline__ void lse_merge_row(const float *es, const float *ml, const uint16_t *to, int64_t s_es_part,
                                              int64_t s_to_part, int P, int head_dim, int lane, float (&a0)[NB],
                                              float (&a1)[NB]) {
    float r0[1][NB], r1[1][NB];
    lse_merge_rows<NB, 1>(es, ml, to, 0, 0, s_es_part, s_to_part, P, head_dim, lane, 1, r0, r1);
#pragma unroll
    for (int k = 0; k < NB; ++k) {
        a0[k] = r0[0][k];
        a1[k] = r1[0][k];
    }
}

}  // namespace pa
