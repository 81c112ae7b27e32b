// recurrent_scan.hip -- exclusive affine scan over a sequence of [Dk, Dv] states.
//
// For each (outer o, head h) and n = 0..N_o-1, with s starting at init (or zero):
//   s_all[n] = s ;   s = decay[n] (row-broadcast over Dv) * s + kv[n]
// and fin = s after the last step.  This is the forward of the reference's
// FusedRecurrentScan (triune/kernels/fast_gla.py:34-64 kernel, :109-149 wrapper), and the
// prefill's inter-segment carry (decay given as a log, kv = segment-local states, s_all
// written in place of kv).  Arithmetic in fp32; kv / s_all / fin may be fp32, bf16 or fp16.
#include <type_traits>

#include "kernels.h"

namespace triune {

__device__ __forceinline__ float ld_dt(const void* p, int dt, int64_t i) {
    if (dt == DT_F32) return reinterpret_cast<const float*>(p)[i];
    if (dt == DT_BF16) return (float)reinterpret_cast<const __bf16*>(p)[i];
    return (float)reinterpret_cast<const _Float16*>(p)[i];
}

__device__ __forceinline__ void ld4_dt(const void* p, int dt, int64_t i, float (&x)[4]) {
    if (dt == DT_F32) {
        float4 a = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + i);
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    } else if (dt == DT_BF16) {
        bf16x4 a = *reinterpret_cast<const bf16x4*>(reinterpret_cast<const __bf16*>(p) + i);
        x[0] = (float)a[0]; x[1] = (float)a[1]; x[2] = (float)a[2]; x[3] = (float)a[3];
    } else {
        typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
        f16x4 a = *reinterpret_cast<const f16x4*>(reinterpret_cast<const _Float16*>(p) + i);
        x[0] = (float)a[0]; x[1] = (float)a[1]; x[2] = (float)a[2]; x[3] = (float)a[3];
    }
}

__device__ __forceinline__ void st4_dt(void* p, int dt, int64_t i, const float (&x)[4]) {
    if (dt == DT_F32) store4_dt(reinterpret_cast<float*>(p) + i, dt, x[0], x[1], x[2], x[3]);
    else if (dt == DT_BF16) store4_dt(reinterpret_cast<__bf16*>(p) + i, dt, x[0], x[1], x[2], x[3]);
    else store4_dt(reinterpret_cast<_Float16*>(p) + i, dt, x[0], x[1], x[2], x[3]);
}

template <typename T>
__device__ __forceinline__ void ld4_t(const void* p, int64_t i, float (&x)[4]) {
    const T* q = reinterpret_cast<const T*>(p) + i;
    if constexpr (std::is_same<T, float>::value) {
        const float4 a = *reinterpret_cast<const float4*>(q);
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    } else {
        typedef T t4 __attribute__((ext_vector_type(4)));
        const t4 a = *reinterpret_cast<const t4*>(q);
        x[0] = (float)a[0]; x[1] = (float)a[1]; x[2] = (float)a[2]; x[3] = (float)a[3];
    }
}

template <typename T>
__device__ __forceinline__ void st4_t(void* p, int64_t i, const float (&x)[4]) {
    T* q = reinterpret_cast<T*>(p) + i;
    if constexpr (std::is_same<T, float>::value) {
        *reinterpret_cast<float4*>(q) = make_float4(x[0], x[1], x[2], x[3]);
    } else {
        typedef T t4 __attribute__((ext_vector_type(4)));
        *reinterpret_cast<t4*>(q) = t4{(T)x[0], (T)x[1], (T)x[2], (T)x[3]};
    }
}

// grid: (ceil(Dk*Dv/4 / SCAN_TPB), H, n_outer), block SCAN_TPB; each thread owns 4 consecutive
// elements.  Small blocks spread the (outer, head) rows over many CUs.  The grid holds only
// B*H*Dk*Dv/256 waves (384 at the config-1 chunk-state shape), so each thread keeps the loads
// of SCAN_U steps in flight (32 steps x 16 bytes per lane) before the dependent chain consumes
// them; the steps' stores go out before the next batch's loads.
constexpr int SCAN_TPB = 64;
constexpr int SCAN_U = 32;
__global__ __launch_bounds__(SCAN_TPB) void recurrent_scan_kernel(ScanParams a) {
    const int64_t DD = (int64_t)a.Dk * a.Dv;
    const int64_t e = ((int64_t)blockIdx.x * SCAN_TPB + threadIdx.x) * 4;
    if (e >= DD) return;
    const int64_t h = blockIdx.y, o = blockIdx.z;
    const int row = (int)(e / a.Dv);
    int64_t n0 = 0, N = a.N;
    if (a.seg_off) {
        n0 = a.seg_off[o];
        N = (int64_t)a.seg_off[o + 1] - n0;
    }
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    if (a.init) {
        const float* ip = a.init + o * a.i_so + h * a.i_sh + e;
        float4 v = *reinterpret_cast<const float4*>(ip);
        s[0] = v.x; s[1] = v.y; s[2] = v.z; s[3] = v.w;
    } else if (a.init_any) {
        ld4_dt(a.init_any, a.init_dt, o * a.i_so + h * a.i_sh + e, s);
    }
    const int64_t kv_base = o * a.kv_so + h * a.kv_sh + e;
    const int64_t sa_base = o * a.sa_so + h * a.sa_sh + e;
    const int64_t d_base = o * a.d_so + h * a.d_sh + row;
    constexpr int U = SCAN_U;
    for (int64_t n = 0; n < N; n += U) {  // a partial last batch re-reads its last step (not used)
        float x[U][4], d[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = n0 + (n + u < N ? n + u : N - 1);
            ld4_dt(a.kv, a.kv_dt, kv_base + i * a.kv_sn, x[u]);
            d[u] = ld_dt(a.dec, a.dec_dt, d_base + i * a.d_sn);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (n + u >= N) break;  // uniform
            const float dd = a.dec_is_log ? expf(d[u]) : d[u];
            if (a.s_all) st4_dt(a.s_all, a.sa_dt, sa_base + (n0 + n + u) * a.sa_sn, s);
#pragma unroll
            for (int c = 0; c < 4; ++c) s[c] = s[c] * dd + x[u][c];
        }
    }
    if (a.fin) st4_dt(a.fin, a.fin_dt, o * a.f_so + h * a.f_sh + e, s);
}

// The same scan with the dtypes fixed at compile time (kv in KT, s_all / fin in OT, decay factors
// in fp32), so every load of a batch is one unconditional vector access and the compiler's waits
// track them exactly.
template <typename KT, typename OT>
__global__ __launch_bounds__(SCAN_TPB) void recurrent_scan_typed_kernel(ScanParams a) {
    const int64_t DD = (int64_t)a.Dk * a.Dv;
    const int64_t e = ((int64_t)blockIdx.x * SCAN_TPB + threadIdx.x) * 4;
    if (e >= DD) return;
    const int64_t h = blockIdx.y, o = blockIdx.z;
    const int row = (int)(e / a.Dv);
    const int64_t N = a.N;
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    if (a.init) {
        const float4 v = *reinterpret_cast<const float4*>(a.init + o * a.i_so + h * a.i_sh + e);
        s[0] = v.x; s[1] = v.y; s[2] = v.z; s[3] = v.w;
    } else if (a.init_any) {
        ld4_dt(a.init_any, a.init_dt, o * a.i_so + h * a.i_sh + e, s);
    }
    const int64_t kv_base = o * a.kv_so + h * a.kv_sh + e;
    const int64_t sa_base = o * a.sa_so + h * a.sa_sh + e;
    const float* dec = reinterpret_cast<const float*>(a.dec) + o * a.d_so + h * a.d_sh + row;
    constexpr int U = SCAN_U;
    for (int64_t n = 0; n < N; n += U) {
        float x[U][4], d[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = n + u < N ? n + u : N - 1;
            ld4_t<KT>(a.kv, kv_base + i * a.kv_sn, x[u]);
            d[u] = dec[i * a.d_sn];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (n + u >= N) break;  // uniform
            st4_t<OT>(a.s_all, sa_base + (n + u) * a.sa_sn, s);
#pragma unroll
            for (int c = 0; c < 4; ++c) s[c] = s[c] * d[u] + x[u][c];
        }
    }
    st4_t<OT>(a.fin, o * a.f_so + h * a.f_sh + e, s);
}

// The prefill's carry over segments: fp32 kv and s_all (the same buffer), fp32 log-decay, fp32
// init / fin.  All U loads of a block of steps are issued before the dependent chain runs, so a
// typical sequence (at most U segments) pays one memory latency; the chain itself is four
// independent FMA lanes per step with exp on the hardware exp2.  The steps go through buffer
// instructions: per block of steps one resource based at the block's lowest step (the first, or
// with a negative step stride, as the backward's reverse scan has, the last) at the workgroup's
// first element (kv) or the decays, the lane's offset in the vector register and the step's
// distance from the base in the scalar offset, so no step costs vector address arithmetic.
template <int U>
__global__ __launch_bounds__(SCAN_TPB) void seg_scan_f32_kernel(ScanParams a) {
    const int64_t DD = (int64_t)a.Dk * a.Dv;
    const int64_t eb = (int64_t)blockIdx.x * SCAN_TPB * 4;  // the workgroup's first element
    const int t = (int)threadIdx.x;
    const int64_t e = eb + 4 * t;
    if (e >= DD) return;
    const int64_t h = blockIdx.y, o = blockIdx.z;
    const int row = (int)(e / a.Dv);
    int64_t n0 = 0, N = a.N;
    if (a.seg_off) {
        n0 = a.seg_off[o];
        N = (int64_t)a.seg_off[o + 1] - n0;
    }
    int64_t srow = o;  // row of init / fin
    bool has_row = true;
    if (a.slots) {
        const int32_t sl = a.slots[o];
        has_row = sl >= 0 && sl < a.n_slots;
        srow = has_row ? sl : 0;
    }
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    if (a.init && has_row) s = *reinterpret_cast<const float4*>(a.init + srow * a.i_so + h * a.i_sh + e);
    float* kv = const_cast<float*>(reinterpret_cast<const float*>(a.kv)) + o * a.kv_so + h * a.kv_sh + eb;
    float* dec = const_cast<float*>(reinterpret_cast<const float*>(a.dec)) + o * a.d_so + h * a.d_sh;
    const bool kneg = a.kv_sn < 0, dneg = a.d_sn < 0;
    const int32_t kst = (int32_t)((kneg ? -a.kv_sn : a.kv_sn) * 4);  // bytes per step
    const int32_t dst = (int32_t)((dneg ? -a.d_sn : a.d_sn) * 4);
    const int32_t kvo = 16 * t, dvo = 4 * row;
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    for (int64_t n = 0; n < N; n += U) {
        const int32_t last = (int32_t)(N - n < U ? N - n : U) - 1;  // the block's last step
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
            kv + (n0 + n + (kneg ? last : 0)) * a.kv_sn, (short)0, 0x7fffffff, 0x00020000);
        const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc(
            dec + (n0 + n + (dneg ? last : 0)) * a.d_sn, (short)0, 0x7fffffff, 0x00020000);
        auto koff = [&](int32_t u) { return (kneg ? last - u : u) * kst; };
        auto doff = [&](int32_t u) { return (dneg ? last - u : u) * dst; };
        float4 x[U];
        float d[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int32_t uu = u < last ? u : last;  // a short block re-reads its last step
            x[u] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rk, kvo, koff(uu), 0));
            d[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rd, dvo, doff(uu), 0));
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (u <= last) {
                const float dd = fast_exp(d[u]);
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, s), rk, kvo, koff(u), 0);  // exclusive prefix
                s.x = s.x * dd + x[u].x;
                s.y = s.y * dd + x[u].y;
                s.z = s.z * dd + x[u].z;
                s.w = s.w * dd + x[u].w;
            }
        }
    }
    if (a.fin && has_row) *reinterpret_cast<float4*>(reinterpret_cast<float*>(a.fin) + srow * a.f_so + h * a.f_sh + e) = s;
}

__device__ __forceinline__ void st1_dt(void* p, int dt, int64_t i, float x) {
    if (dt == DT_F32) reinterpret_cast<float*>(p)[i] = x;
    else if (dt == DT_BF16) reinterpret_cast<__bf16*>(p)[i] = (__bf16)x;
    else reinterpret_cast<_Float16*>(p)[i] = (_Float16)x;
}

// Backward of the exclusive scan (reference: _recurrent_scan_bwd, fast_gla.py:67-107, and
// FusedRecurrentScan.backward :151-203), for each (outer o, head h), walking n = N-1 .. 0:
//   d_kv[n] = d ;  d_decay[n][i] = sum_j d[i][j] * s_all[n][i][j] ;  d = d_s_all[n] + decay[n] * d
// from d = d_fin, and d_init = d at the end.  The reference sums d_decay over Dv afterwards
// (d_decay * s_prev per element, then .sum(-1)); here the LPR lanes of a row reduce it in
// registers.  grid: (ceil(Dk / (64 / LPR)), H, n_outer), one wave per block; lane = row-in-block
// * LPR + c holds columns 4c .. 4c+3 of its row (LPR = smallest power of two >= Dv / 4).
__global__ __launch_bounds__(64) void recurrent_scan_bwd_kernel(ScanBwdParams a, int lpr) {
    const int lane = threadIdx.x;
    const int row = blockIdx.x * (64 / lpr) + lane / lpr;
    const int j0 = (lane % lpr) * 4;
    const bool act = row < a.Dk && j0 < a.Dv;
    const int64_t DD = (int64_t)a.Dk * a.Dv, N = a.N;
    const int64_t bh = (int64_t)blockIdx.z * a.H + blockIdx.y;
    const int64_t e = act ? (int64_t)row * a.Dv + j0 : 0;
    const int64_t r = act ? row : 0;
    float d[4] = {0.f, 0.f, 0.f, 0.f};
    if (a.d_fin && act) ld4_dt(a.d_fin, a.df_dt, bh * DD + e, d);
    constexpr int U = SCAN_U;
    for (int64_t nn = N; nn > 0; nn -= U) {
        float ds[U][4], sp[U][4], dc[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t n = nn - 1 - u >= 0 ? nn - 1 - u : 0;
            const int64_t i5 = (bh * N + n) * DD + e;
            if (a.d_s_all) {
                ld4_dt(a.d_s_all, a.dsa_dt, i5, ds[u]);
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c) ds[u][c] = 0.f;
            }
            const float4 s4 = *reinterpret_cast<const float4*>(a.s_all + i5);
            sp[u][0] = s4.x; sp[u][1] = s4.y; sp[u][2] = s4.z; sp[u][3] = s4.w;
            dc[u] = ld_dt(a.dec, a.dec_dt, (bh * N + n) * a.Dk + r);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t n = nn - 1 - u;
            if (n < 0) break;  // uniform
            const int64_t i5 = (bh * N + n) * DD + e;
            if (act) st4_dt(a.d_kv, a.out_dt, i5, d);
            float part = act ? d[0] * sp[u][0] + d[1] * sp[u][1] + d[2] * sp[u][2] + d[3] * sp[u][3] : 0.f;
            for (int off = lpr >> 1; off >= 1; off >>= 1) part += __shfl_xor(part, off);
            if (act && j0 == 0) st1_dt(a.d_dec, a.out_dt, (bh * N + n) * a.Dk + row, part);
#pragma unroll
            for (int c = 0; c < 4; ++c) d[c] = ds[u][c] + dc[u] * d[c];
        }
    }
    if (act) st4_dt(a.d_init, a.out_dt, bh * DD + e, d);
}

// The backward with the dtypes fixed at compile time: upstream gradient of s_all and every output
// in GT, decay factors in fp32 (same work split as recurrent_scan_bwd_kernel).  LPR16: a row's
// partial products are summed over its 16 lanes (one DPP row, Dv = 64) without LDS round trips.
template <typename GT, bool LPR16>
__global__ __launch_bounds__(64) void recurrent_scan_bwd_typed_kernel(ScanBwdParams a, int lpr) {
    const int lane = threadIdx.x;
    const int row = blockIdx.x * (64 / lpr) + lane / lpr;
    const int j0 = (lane % lpr) * 4;
    const bool act = row < a.Dk && j0 < a.Dv;
    const int64_t DD = (int64_t)a.Dk * a.Dv, N = a.N;
    const int64_t bh = (int64_t)blockIdx.z * a.H + blockIdx.y;
    const int64_t e = act ? (int64_t)row * a.Dv + j0 : 0;
    const int64_t r = act ? row : 0;
    const float* dec = reinterpret_cast<const float*>(a.dec);
    float d[4] = {0.f, 0.f, 0.f, 0.f};
    if (a.d_fin && act) ld4_dt(a.d_fin, a.df_dt, bh * DD + e, d);
    constexpr int U = SCAN_U;
    for (int64_t nn = N; nn > 0; nn -= U) {
        float ds[U][4], sp[U][4], dc[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t n = nn - 1 - u >= 0 ? nn - 1 - u : 0;
            const int64_t i5 = (bh * N + n) * DD + e;
            if (a.d_s_all) {
                ld4_t<GT>(a.d_s_all, i5, ds[u]);
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c) ds[u][c] = 0.f;
            }
            const float4 s4 = *reinterpret_cast<const float4*>(a.s_all + i5);
            sp[u][0] = s4.x; sp[u][1] = s4.y; sp[u][2] = s4.z; sp[u][3] = s4.w;
            dc[u] = dec[(bh * N + n) * a.Dk + r];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t n = nn - 1 - u;
            if (n < 0) break;  // uniform
            const int64_t i5 = (bh * N + n) * DD + e;
            if (act) st4_t<GT>(a.d_kv, i5, d);
            float part = act ? d[0] * sp[u][0] + d[1] * sp[u][1] + d[2] * sp[u][2] + d[3] * sp[u][3] : 0.f;
            if constexpr (LPR16) {
                part = dpp_sum16(part);
            } else {
                for (int off = lpr >> 1; off >= 1; off >>= 1) part += __shfl_xor(part, off);
            }
            if (act && j0 == 0) reinterpret_cast<GT*>(a.d_dec)[(bh * N + n) * a.Dk + row] = (GT)part;
#pragma unroll
            for (int c = 0; c < 4; ++c) d[c] = ds[u][c] + dc[u] * d[c];
        }
    }
    if (act) st4_t<GT>(a.d_init, bh * DD + e, d);
}

hipError_t launch_recurrent_scan_bwd(const ScanBwdParams& a, hipStream_t stream) {
    int lpr = 1;
    while (lpr * 4 < a.Dv) lpr <<= 1;
    if (lpr > 64) return hipErrorInvalidValue;
    const int rpb = 64 / lpr;
    dim3 grid((unsigned)((a.Dk + rpb - 1) / rpb), (unsigned)a.H, (unsigned)a.n_outer);
    const bool typed = a.dec_dt == DT_F32 && (!a.d_s_all || a.dsa_dt == a.out_dt);
    if (typed && lpr == 16) {
        if (a.out_dt == DT_F32) hipLaunchKernelGGL((recurrent_scan_bwd_typed_kernel<float, true>), grid, dim3(64), 0, stream, a, lpr);
        else if (a.out_dt == DT_BF16) hipLaunchKernelGGL((recurrent_scan_bwd_typed_kernel<__bf16, true>), grid, dim3(64), 0, stream, a, lpr);
        else hipLaunchKernelGGL((recurrent_scan_bwd_typed_kernel<_Float16, true>), grid, dim3(64), 0, stream, a, lpr);
    } else if (typed && a.out_dt == DT_F32) hipLaunchKernelGGL((recurrent_scan_bwd_typed_kernel<float, false>), grid, dim3(64), 0, stream, a, lpr);
    else if (typed && a.out_dt == DT_BF16) hipLaunchKernelGGL((recurrent_scan_bwd_typed_kernel<__bf16, false>), grid, dim3(64), 0, stream, a, lpr);
    else if (typed && a.out_dt == DT_F16) hipLaunchKernelGGL((recurrent_scan_bwd_typed_kernel<_Float16, false>), grid, dim3(64), 0, stream, a, lpr);
    else hipLaunchKernelGGL(recurrent_scan_bwd_kernel, grid, dim3(64), 0, stream, a, lpr);
    return hipGetLastError();
}

hipError_t launch_recurrent_scan(const ScanParams& a, hipStream_t stream) {
    const int64_t DD = (int64_t)a.Dk * a.Dv;
    dim3 grid((unsigned)((DD / 4 + SCAN_TPB - 1) / SCAN_TPB), (unsigned)a.H, (unsigned)a.n_outer);
    const bool prefill_carry = a.kv_dt == DT_F32 && a.dec_dt == DT_F32 && a.dec_is_log && a.s_all == a.kv &&
                               a.sa_dt == DT_F32 && a.sa_so == a.kv_so && a.sa_sh == a.kv_sh &&
                               a.sa_sn == a.kv_sn && !a.init_any && (!a.fin || a.fin_dt == DT_F32);
    if (a.slots && !prefill_carry) return hipErrorInvalidValue;
    if (prefill_carry) {
        hipLaunchKernelGGL(seg_scan_f32_kernel<24>, grid, dim3(SCAN_TPB), 0, stream, a);
        return hipGetLastError();
    }
    // dense steps, fp32 decay factors, s_all and fin both present in one dtype that is kv's or fp32
    const bool typed = !a.seg_off && a.dec_dt == DT_F32 && !a.dec_is_log && a.s_all && a.fin &&
                       a.sa_dt == a.fin_dt && (a.sa_dt == a.kv_dt || a.sa_dt == DT_F32);
    if (typed) {
        const int k = a.kv_dt, t = a.sa_dt;
        if (k == DT_F32) hipLaunchKernelGGL((recurrent_scan_typed_kernel<float, float>), grid, dim3(SCAN_TPB), 0, stream, a);
        else if (k == DT_BF16 && t == DT_BF16) hipLaunchKernelGGL((recurrent_scan_typed_kernel<__bf16, __bf16>), grid, dim3(SCAN_TPB), 0, stream, a);
        else if (k == DT_BF16) hipLaunchKernelGGL((recurrent_scan_typed_kernel<__bf16, float>), grid, dim3(SCAN_TPB), 0, stream, a);
        else if (t == DT_F16) hipLaunchKernelGGL((recurrent_scan_typed_kernel<_Float16, _Float16>), grid, dim3(SCAN_TPB), 0, stream, a);
        else hipLaunchKernelGGL((recurrent_scan_typed_kernel<_Float16, float>), grid, dim3(SCAN_TPB), 0, stream, a);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(recurrent_scan_kernel, grid, dim3(SCAN_TPB), 0, stream, a);
    return hipGetLastError();
}

}  // namespace triune
