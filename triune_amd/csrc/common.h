// common.h -- device helpers shared by the GLA / Gated DeltaNet kernels (gfx950, wave64).
//
// MFMA fragment conventions used throughout (v_mfma_f32_16x16x32_bf16):
//   lane l = 16*g4 + r16  (g4 = l >> 4 in 0..3, r16 = l & 15)
//   A operand (16 x 32, M x K):  lane holds row m = r16, eight K slots (g4, j), j = 0..7
//   B operand (32 x 16, K x N):  lane holds column n = r16, the same eight K slots (g4, j)
//   C/D (16 x 16):               lane holds rows 4*g4 + i (i = 0..3) of column r16
// Any bijection between K slots and the contracted index is valid as long as the A and B
// operands use the same one; the kernels pick the one that lets accumulator tiles feed the
// next product without moving data between lanes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace triune {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

enum DType : int { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };

__device__ __forceinline__ f32x4 mfma(const bf16x8& a, const bf16x8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

__device__ __forceinline__ float bf2f(__bf16 x) { return (float)x; }

// ---------------------------------------------------------------------------------------
// Splitting fp32 values into sums of bf16 parts: x ~= p0 + p1 (+ p2).  Each part is the
// round-to-nearest bf16 of the remaining residual, so N parts carry ~8N mantissa bits.
// ---------------------------------------------------------------------------------------
template <int N>
struct Split8 {
    bf16x8 p[N];
};

// Round-to-nearest bf16 of (a, b) in one packed conversion: a in bits 0-15, b in bits 16-31.
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a, b}, b2));
}

// The two floats a packed bf16 pair stands for.
__device__ __forceinline__ float pk_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float pk_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

// Splits r[0..2W) into N packed planes w[n][0..W): pair by pair, one packed conversion gives
// both the stored part and the value the residual subtracts.
template <int N, int W>
__device__ __forceinline__ void split_pairs(float (&r)[2 * W], uint32_t (&w)[N][W]) {
#pragma unroll
    for (int n = 0; n < N; ++n) {
#pragma unroll
        for (int j = 0; j < W; ++j) {
            w[n][j] = pk_bf16(r[2 * j], r[2 * j + 1]);
            if (n + 1 < N) {
                r[2 * j] -= pk_lo(w[n][j]);
                r[2 * j + 1] -= pk_hi(w[n][j]);
            }
        }
    }
}

template <int N>
__device__ __forceinline__ Split8<N> split8(const float (&x)[8]) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    float r[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = x[j];
    uint32_t w[N][4];
    split_pairs<N, 4>(r, w);
    Split8<N> s;
#pragma unroll
    for (int n = 0; n < N; ++n) s.p[n] = __builtin_bit_cast(bf16x8, u32x4{w[n][0], w[n][1], w[n][2], w[n][3]});
    return s;
}

// Products of split operands: sum over part pairs (ia, ib) with ia + ib < NS.
// NA / NB are the number of parts each operand carries (an operand exactly representable
// in bf16 has one part).
template <int NA, int NB, int NS>
__device__ __forceinline__ f32x4 mfma_split(const Split8<NA>& a, const Split8<NB>& b, f32x4 c) {
#pragma unroll
    for (int ia = 0; ia < NA; ++ia)
#pragma unroll
        for (int ib = 0; ib < NB; ++ib)
            if (ia + ib < NS) c = mfma(a.p[ia], b.p[ib], c);
    return c;
}

// ---------------------------------------------------------------------------------------
// Element loads: eight consecutive elements starting at p (16-byte aligned for 16-bit types,
// 32-byte for fp32), returned as float, or zeros when !valid.
// ---------------------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void load8(const T* p, bool valid, float (&x)[8]);

template <>
__device__ __forceinline__ void load8<__bf16>(const __bf16* p, bool valid, float (&x)[8]) {
    if (valid) {
        uint4 u = *reinterpret_cast<const uint4*>(p);
        uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            x[2 * j] = __uint_as_float(w[j] << 16);
            x[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = 0.f;
    }
}

template <>
__device__ __forceinline__ void load8<_Float16>(const _Float16* p, bool valid, float (&x)[8]) {
    if (valid) {
        f16x8 h = *reinterpret_cast<const f16x8*>(p);
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = (float)h[j];
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = 0.f;
    }
}

template <>
__device__ __forceinline__ void load8<float>(const float* p, bool valid, float (&x)[8]) {
    if (valid) {
        float4 a = reinterpret_cast<const float4*>(p)[0];
        float4 b = reinterpret_cast<const float4*>(p)[1];
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = 0.f;
    }
}

// Runtime-typed variant (gates may be fp32 while q/k/v are 16-bit).
__device__ __forceinline__ void load8_dt(const void* p, int dt, bool valid, float (&x)[8]) {
    if (dt == DT_F32) load8<float>(reinterpret_cast<const float*>(p), valid, x);
    else if (dt == DT_BF16) load8<__bf16>(reinterpret_cast<const __bf16*>(p), valid, x);
    else load8<_Float16>(reinterpret_cast<const _Float16*>(p), valid, x);
}

__device__ __forceinline__ int dt_size(int dt) { return dt == DT_F32 ? 4 : 2; }

// Store eight consecutive floats as dtype dt.
__device__ __forceinline__ void store8_dt(void* p, int dt, const float (&x)[8]) {
    if (dt == DT_F32) {
        float4* q = reinterpret_cast<float4*>(p);
        q[0] = make_float4(x[0], x[1], x[2], x[3]);
        q[1] = make_float4(x[4], x[5], x[6], x[7]);
    } else if (dt == DT_BF16) {
        bf16x8 h;
#pragma unroll
        for (int j = 0; j < 8; ++j) h[j] = (__bf16)x[j];
        *reinterpret_cast<bf16x8*>(p) = h;
    } else {
        f16x8 h;
#pragma unroll
        for (int j = 0; j < 8; ++j) h[j] = (_Float16)x[j];
        *reinterpret_cast<f16x8*>(p) = h;
    }
}

// Store four consecutive floats as dtype dt.
__device__ __forceinline__ void store4_dt(void* p, int dt, float a, float b, float c, float d) {
    if (dt == DT_F32) {
        *reinterpret_cast<float4*>(p) = make_float4(a, b, c, d);
    } else if (dt == DT_BF16) {
        bf16x4 h = {(__bf16)a, (__bf16)b, (__bf16)c, (__bf16)d};
        *reinterpret_cast<bf16x4*>(p) = h;
    } else {
        typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
        f16x4 h = {(_Float16)a, (_Float16)b, (_Float16)c, (_Float16)d};
        *reinterpret_cast<f16x4*>(p) = h;
    }
}

// Store four floats as dtype dt at byte offset off of a buffer resource: a store whose offset
// lies past the resource's records is dropped, so lanes (or whole waves) with nothing to store
// still issue it and every wave keeps the same count of memory operations in flight.
__device__ __forceinline__ void buffer_store4_dt(__amdgpu_buffer_rsrc_t r, int off, int dt, const f32x4& x) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
    if (dt == DT_F32) {
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), r, off, 0, 0);
    } else if (dt == DT_BF16) {
        const bf16x4 h = {(__bf16)x[0], (__bf16)x[1], (__bf16)x[2], (__bf16)x[3]};
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, h), r, off, 0, 0);
    } else {
        const f16x4 h = {(_Float16)x[0], (_Float16)x[1], (_Float16)x[2], (_Float16)x[3]};
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, h), r, off, 0, 0);
    }
}

// ---------------------------------------------------------------------------------------
// Lane helpers (wave64).
// ---------------------------------------------------------------------------------------
// Value of x in lane (lane - n) of the same 16-lane row, or 0 for the first n lanes of the
// row (DPP row_shr with bound_ctrl).
template <int N>
__device__ __forceinline__ float row_shr(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x110 + N, 0xf, 0xf, true));
}

// Value of x in lane (lane + n) of the same 16-lane row, or 0 for the last n lanes of the row
// (DPP row_shl with bound_ctrl).
template <int N>
__device__ __forceinline__ float row_shl(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x100 + N, 0xf, 0xf, true));
}

// Inclusive prefix sum across the 16 lanes of each row.
__device__ __forceinline__ float row_inclusive_scan(float x) {
    x += row_shr<1>(x);
    x += row_shr<2>(x);
    x += row_shr<4>(x);
    x += row_shr<8>(x);
    return x;
}

// Sum over the 16 lanes of a DPP row, in every lane of it: quad swaps (lane ^ 1, lane ^ 2), then
// the half-row mirror (quad q <-> quad q ^ 1) and the row mirror (half <-> half).
template <int CTRL>
__device__ __forceinline__ float dpp_add(float x) {
    return x + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float dpp_sum16(float x) {
    x = dpp_add<0xB1>(x);   // quad_perm [1, 0, 3, 2]
    x = dpp_add<0x4E>(x);   // quad_perm [2, 3, 0, 1]
    x = dpp_add<0x141>(x);  // row_half_mirror
    return dpp_add<0x140>(x);  // row_mirror
}

// Rotation by N lanes within each 16-lane DPP row (lane p reads lane p - N of its row).
template <int N>
__device__ __forceinline__ float row_ror(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x120 + N, 0xf, 0xf, false));
}

// Whole-row exchanges (VALU, no LDS).  With rows x0..x3 of 16 lanes: swap16 returns
// lo = [x0, x0, x2, x2] and hi = [x1, x1, x3, x3]; swap32 returns lo = [x0, x1, x0, x1] and
// hi = [x2, x3, x2, x3].
struct RowPair {
    float lo, hi;
};
__device__ __forceinline__ RowPair swap16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return {__uint_as_float(r[0]), __uint_as_float(r[1])};
}
__device__ __forceinline__ RowPair swap32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return {__uint_as_float(r[0]), __uint_as_float(r[1])};
}

// x + (the value of lane ^ SH): through whole-row swaps for SH = 16 and 32 (VALU), otherwise
// through an LDS-pipe shuffle.  Both lanes of a pair get the same, identically rounded sum.
template <int SH>
__device__ __forceinline__ float xor_sum(float x) {
    if constexpr (SH == 16) {
        const RowPair p = swap16(x);
        return p.lo + p.hi;
    } else if constexpr (SH == 32) {
        const RowPair p = swap32(x);
        return p.lo + p.hi;
    } else {
        return x + __shfl_xor(x, SH);
    }
}

// Sum over the lanes l ^ (SH * 2^k) of a wave (SH a power of two): every lane of the group
// gets it.
template <int SH>
__device__ __forceinline__ float xor_group_sum(float x) {
    if constexpr (SH < 64) return xor_group_sum<SH * 2>(xor_sum<SH>(x));
    return x;
}

// Value held by lane src_lane.
__device__ __forceinline__ float lane_bcast(float x, int src_lane) {
    return __int_as_float(__builtin_amdgcn_ds_bpermute(src_lane << 2, __float_as_int(x)));
}

constexpr float LOG2E = 1.4426950408889634f;

__device__ __forceinline__ float fast_exp(float x) {
    // exp(x) = 2^(x log2 e); v_exp_f32 is accurate to ~1 ulp over the range used here.
    return __builtin_amdgcn_exp2f(x * LOG2E);
}

// The GLA input pre-processing (VectorisedGLA, triune/model/attention.py:14-79): elu(x) + 1,
// logsigmoid, and the inverse of a row's L2 norm with the reference's floor.
__device__ __forceinline__ float elu1(float x) { return x >= 0.f ? x + 1.f : fast_exp(x); }

// min(x, 0) - log(1 + e^-|x|) with the hardware exp2 / log2: for e^-|x| below 2^-24 the log term
// rounds to 0, an absolute error under 6e-8.
__device__ __forceinline__ float logsigmoid(float x) {
    // min(x, 0) as one integer min (a float with the sign bit set keeps its bits, others map to +0)
    const float lo = __int_as_float(min(__float_as_int(x), 0));
    return lo - 0.6931471805599453f * __builtin_amdgcn_logf(1.f + fast_exp(-fabsf(x)));
}

__device__ __forceinline__ float sigmoid(float x) {
    const float e = fast_exp(-fabsf(x));
    return x >= 0.f ? 1.f / (1.f + e) : e / (1.f + e);
}

// The hardware reciprocal square root (about 1 ulp), as the reference's tl.rsqrt (attention.py:42).
__device__ __forceinline__ float inv_norm(float sumsq) { return __builtin_amdgcn_rsqf(fmaxf(sumsq, 1e-12f)); }

}  // namespace triune
