// gla_prep.hip -- GLA input pre-processing on gfx950, and the decode step fused with it.
//
// Pre-processing of the reference's VectorisedGLA (triune/model/attention.py:14-79, the
// _fused_qkv_g_prep_inplace_kernel Triton kernel; the unfused form is attention.py:509-528):
//   q, k <- RoPE(normalize(elu(x) + 1))   per (token, head) row of HD elements
//   g    <- logsigmoid(g)
// with normalize(a) = a / sqrt(max(sum(a^2), 1e-12)) and RoPE pairing element d with d + HD/2:
//   out[d]        = a[d] cos[t][d]        - a[d + HD/2] sin[t][d]
//   out[d + HD/2] = a[d + HD/2] cos[t][d + HD/2] + a[d] sin[t][d + HD/2]          (d < HD/2)
// The fused decode step (attention.py:81-179, _fused_qkvg_decode_step_kernel) applies the same
// pre-processing to one token per sequence and then the GLA step with decay sigmoid(g)
// (= exp(logsigmoid(g))):  S <- diag(sigmoid(g)) S + k v^T ,  o = S^T q.
//
// gla_prep_kernel: memory-bound, in place.  A row is covered by HD/8 consecutive lanes holding 8
// elements each (16-byte accesses for 16-bit types); the sum of squares is reduced and the RoPE
// partner exchanged with lane shuffles inside the row's lane group.
// gla_fused_decode_kernel: the decode kernel's layout (a 256-thread block per (b, h) row, thread
// = RPT key rows x 4 value columns); every wave forms the two norms itself from one element per
// lane, so no barrier separates the pre-processing from the state update.
#include "kernels.h"

namespace triune {

template <typename T>
using V4 = T __attribute__((ext_vector_type(4)));

// Eight consecutive elements as floats / back (16-bit: one 16-byte access; fp32: two).
template <typename T>
__device__ __forceinline__ void ld8(const T* p, float (&x)[8]) {
    const V4<T> a = *reinterpret_cast<const V4<T>*>(p);
    const V4<T> b = *reinterpret_cast<const V4<T>*>(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        x[i] = (float)a[i];
        x[4 + i] = (float)b[i];
    }
}

template <typename T>
__device__ __forceinline__ void st8(T* p, const float (&x)[8]) {
    V4<T> a, b;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        a[i] = (T)x[i];
        b[i] = (T)x[4 + i];
    }
    *reinterpret_cast<V4<T>*>(p) = a;
    *reinterpret_cast<V4<T>*>(p + 4) = b;
}

__device__ __forceinline__ float elu1(float x) { return x >= 0.f ? x + 1.f : expf(x); }

__device__ __forceinline__ float logsigmoid(float x) { return fminf(x, 0.f) - log1pf(expf(-fabsf(x))); }

__device__ __forceinline__ float sigmoid(float x) {
    const float e = expf(-fabsf(x));
    return x >= 0.f ? 1.f / (1.f + e) : e / (1.f + e);
}

__device__ __forceinline__ float inv_norm(float sumsq) { return 1.f / sqrtf(fmaxf(sumsq, 1e-12f)); }

// ---------------------------------------------------------------------------------------
// In-place pre-processing of qkv [B, T, 3, H, HD] (q, k; v untouched) and g [B, T, H, HD].
// ---------------------------------------------------------------------------------------
template <int HD, typename TIO, typename TCS>
__global__ __launch_bounds__(256) void gla_prep_kernel(PrepParams a) {
    constexpr int LPR = HD / 8;  // lanes per row
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63;
    const int64_t nrows = a.B * a.T * a.H;
    const int64_t row = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW + lane / LPR;
    const bool ok = row < nrows;
    const int64_t r = ok ? row : nrows - 1;  // past the end: a valid row is read, nothing stored
    const int c = lane % LPR;                 // this lane's 8 elements: 8c .. 8c+7
    const int64_t h = r % a.H, bt = r / a.H, t = bt % a.T, b = bt / a.T;
    TIO* qp = reinterpret_cast<TIO*>(a.qkv) + b * a.qkv_sb + t * a.qkv_st + h * a.qkv_sh + 8 * c;
    TIO* kp = qp + a.qkv_sp;
    TIO* gp = reinterpret_cast<TIO*>(a.g) + b * a.g_sb + t * a.g_st + h * a.g_sh + 8 * c;
    float q[8], k[8], g[8];
    ld8(qp, q);
    ld8(kp, k);
    ld8(gp, g);
    float sq = 0.f, sk = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        q[i] = elu1(q[i]);
        k[i] = elu1(k[i]);
        sq += q[i] * q[i];
        sk += k[i] * k[i];
        g[i] = logsigmoid(g[i]);
    }
#pragma unroll
    for (int m = 1; m < LPR; m <<= 1) {
        sq += __shfl_xor(sq, m);
        sk += __shfl_xor(sk, m);
    }
    const float iq = inv_norm(sq), ik = inv_norm(sk);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        q[i] *= iq;
        k[i] *= ik;
    }
    if (a.use_rope) {
        const TCS* cp = reinterpret_cast<const TCS*>(a.cos) + t * a.cs_st + 8 * c;
        const TCS* sp = reinterpret_cast<const TCS*>(a.sin) + t * a.cs_st + 8 * c;
        float cs[8], sn[8];
        ld8(cp, cs);
        ld8(sp, sn);
        const float sgn = c < LPR / 2 ? -1.f : 1.f;  // first half: a cos - a' sin; second: a cos + a' sin
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float qo = __shfl_xor(q[i], LPR / 2), ko = __shfl_xor(k[i], LPR / 2);
            q[i] = q[i] * cs[i] + sgn * qo * sn[i];
            k[i] = k[i] * cs[i] + sgn * ko * sn[i];
        }
    }
    if (ok) {
        st8(qp, q);
        st8(kp, k);
        st8(gp, g);
    }
}

// ---------------------------------------------------------------------------------------
// Fused decode: qkvg [B, 4, H, HD] (q, k, v, g raw), cos/sin [HD] of the step's position,
// state [B, H, HD, HD] in TS (fp32 or the I/O type), o [B, H, HD].
// ---------------------------------------------------------------------------------------
template <int HD, typename TIO, typename TCS, typename TS>
__global__ __launch_bounds__(256) void gla_fused_decode_kernel(FusedDecodeParams a) {
    constexpr int RPT = HD * HD / (4 * 256) > 4 ? HD * HD / (4 * 256) : 4;  // key rows per thread
    constexpr int CG = HD / 4;                                            // column groups
    constexpr int TPB = HD * HD / (4 * RPT);
    constexpr int WAVES = TPB / 64;
    constexpr int EPL = HD / 64 > 0 ? HD / 64 : 1;  // norm elements per lane
    static_assert(TPB == 256 || TPB == 64 || TPB == 128, "fused decode tiling");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int cg = tid % CG, rg = tid / CG, r0 = rg * RPT;
    const uint32_t H32 = (uint32_t)a.H;
    const int64_t b = blockIdx.x / H32, h = blockIdx.x % H32;
    const TIO* base = reinterpret_cast<const TIO*>(a.qkvg) + b * a.x_sb + h * a.x_sh;
    const TIO* qr = base;
    const TIO* kr = base + a.x_sp;
    const TIO* vr = base + 2 * a.x_sp;
    const TIO* gr = base + 3 * a.x_sp;
    const int64_t srow = (int64_t)blockIdx.x * HD * HD;

    // state first (the large loads), then the row inputs
    f32x4 st[RPT];
    const TS* sin_p = reinterpret_cast<const TS*>(a.state_in) + srow + (int64_t)r0 * HD + 4 * cg;
#pragma unroll
    for (int m = 0; m < RPT; ++m) {
        if (a.has_init) {
            const V4<TS> x = __builtin_nontemporal_load(reinterpret_cast<const V4<TS>*>(sin_p + m * HD));
            st[m] = f32x4{(float)x[0], (float)x[1], (float)x[2], (float)x[3]};
        } else {
            st[m] = zero4();
        }
    }
    // norms: every wave reduces the whole row from EPL elements per lane
    float sq = 0.f, sk = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
        const int d = lane + 64 * e;
        if (d < HD) {
            const float qa = elu1((float)qr[d]), ka = elu1((float)kr[d]);
            sq += qa * qa;
            sk += ka * ka;
        }
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        sq += __shfl_xor(sq, m);
        sk += __shfl_xor(sk, m);
    }
    const float iq = inv_norm(sq), ik = inv_norm(sk);
    // this thread's key rows r0 .. r0+RPT-1 (and their RoPE partners), decays, value columns
    float qv[RPT], kv[RPT], dv[RPT], vv[4];
#pragma unroll
    for (int m = 0; m < RPT; ++m) {
        const int d = r0 + m;
        float qn = elu1((float)qr[d]) * iq, kn = elu1((float)kr[d]) * ik;
        if (a.use_rope) {
            const int dp = d < HD / 2 ? d + HD / 2 : d - HD / 2;
            const float qo = elu1((float)qr[dp]) * iq, ko = elu1((float)kr[dp]) * ik;
            const float cs = (float)reinterpret_cast<const TCS*>(a.cos)[d];
            const float sn = (float)reinterpret_cast<const TCS*>(a.sin)[d];
            const float sgn = d < HD / 2 ? -1.f : 1.f;
            qn = qn * cs + sgn * qo * sn;
            kn = kn * cs + sgn * ko * sn;
        }
        qv[m] = qn;
        kv[m] = kn;
        dv[m] = sigmoid((float)gr[d]);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) vv[c] = (float)vr[4 * cg + c];

    float o4[4] = {0.f, 0.f, 0.f, 0.f};
    TS* sout_p = reinterpret_cast<TS*>(a.state_out) + srow + (int64_t)r0 * HD + 4 * cg;
#pragma unroll
    for (int m = 0; m < RPT; ++m) {
        f32x4 s = st[m];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            s[c] = dv[m] * s[c] + kv[m] * vv[c];
            o4[c] += qv[m] * s[c];
        }
        if (a.save_final) {
            const V4<TS> y = V4<TS>{(TS)s[0], (TS)s[1], (TS)s[2], (TS)s[3]};
            __builtin_nontemporal_store(y, reinterpret_cast<V4<TS>*>(sout_p + m * HD));
        }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int sh = CG; sh < 64; sh <<= 1) o4[c] += __shfl_xor(o4[c], sh);
    __shared__ f32x4 red[WAVES][CG];
    if (lane < CG) red[wave][cg] = f32x4{o4[0], o4[1], o4[2], o4[3]};
    __syncthreads();
    if (tid < CG) {
        f32x4 s = red[0][cg];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) s += red[w][cg];
        store4_dt(reinterpret_cast<char*>(a.o) + (b * a.o_sb + h * a.o_sh + 4 * cg) * dt_size(a.o_dt), a.o_dt, s[0], s[1],
                  s[2], s[3]);
    }
}

// ---------------------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------------------
template <int HD, typename TIO, typename TCS>
static hipError_t launch_prep_t(const PrepParams& a, hipStream_t stream) {
    constexpr int RPB = 4 * (64 / (HD / 8));  // rows per 256-thread block
    const int64_t rows = a.B * a.T * a.H;
    hipLaunchKernelGGL((gla_prep_kernel<HD, TIO, TCS>), dim3((unsigned)((rows + RPB - 1) / RPB)), dim3(256), 0, stream,
                       a);
    return hipGetLastError();
}

template <typename TIO, typename TCS>
static hipError_t launch_prep_hd(const PrepParams& a, int HD, hipStream_t stream) {
    if (HD == 64) return launch_prep_t<64, TIO, TCS>(a, stream);
    if (HD == 128) return launch_prep_t<128, TIO, TCS>(a, stream);
    return launch_prep_t<32, TIO, TCS>(a, stream);
}

template <typename TIO>
static hipError_t launch_prep_cs(const PrepParams& a, int HD, int cs_dt, hipStream_t stream) {
    if (cs_dt == DT_F32) return launch_prep_hd<TIO, float>(a, HD, stream);
    if (cs_dt == DT_BF16) return launch_prep_hd<TIO, __bf16>(a, HD, stream);
    return launch_prep_hd<TIO, _Float16>(a, HD, stream);
}

hipError_t launch_gla_prep(const PrepParams& a, int HD, int io_dt, int cs_dt, hipStream_t stream) {
    if (HD != 32 && HD != 64 && HD != 128) return hipErrorInvalidValue;
    if (io_dt == DT_F32) return launch_prep_cs<float>(a, HD, cs_dt, stream);
    if (io_dt == DT_BF16) return launch_prep_cs<__bf16>(a, HD, cs_dt, stream);
    return launch_prep_cs<_Float16>(a, HD, cs_dt, stream);
}

template <int HD, typename TIO, typename TCS, typename TS>
static hipError_t launch_fdec_t(const FusedDecodeParams& a, hipStream_t stream) {
    constexpr int RPT = HD * HD / (4 * 256) > 4 ? HD * HD / (4 * 256) : 4;
    constexpr int TPB = HD * HD / (4 * RPT);
    hipLaunchKernelGGL((gla_fused_decode_kernel<HD, TIO, TCS, TS>), dim3((unsigned)(a.B * a.H)), dim3(TPB), 0, stream, a);
    return hipGetLastError();
}

template <int HD, typename TIO, typename TCS>
static hipError_t launch_fdec_s(const FusedDecodeParams& a, int s_dt, hipStream_t stream) {
    if (s_dt == DT_F32) return launch_fdec_t<HD, TIO, TCS, float>(a, stream);
    return launch_fdec_t<HD, TIO, TCS, TIO>(a, stream);  // state in the I/O type (checked by the caller)
}

template <int HD, typename TIO>
static hipError_t launch_fdec_cs(const FusedDecodeParams& a, int cs_dt, int s_dt, hipStream_t stream) {
    if (cs_dt == DT_F32) return launch_fdec_s<HD, TIO, float>(a, s_dt, stream);
    return launch_fdec_s<HD, TIO, TIO>(a, s_dt, stream);  // tables in the I/O type (checked by the caller)
}

template <typename TIO>
static hipError_t launch_fdec_hd(const FusedDecodeParams& a, int HD, int cs_dt, int s_dt, hipStream_t stream) {
    if (HD == 64) return launch_fdec_cs<64, TIO>(a, cs_dt, s_dt, stream);
    if (HD == 128) return launch_fdec_cs<128, TIO>(a, cs_dt, s_dt, stream);
    return launch_fdec_cs<32, TIO>(a, cs_dt, s_dt, stream);
}

hipError_t launch_gla_fused_decode(const FusedDecodeParams& a, int HD, int io_dt, int cs_dt, int s_dt,
                                   hipStream_t stream) {
    if (HD != 32 && HD != 64 && HD != 128) return hipErrorInvalidValue;
    if (io_dt == DT_F32) return launch_fdec_hd<float>(a, HD, cs_dt, s_dt, stream);
    if (io_dt == DT_BF16) return launch_fdec_hd<__bf16>(a, HD, cs_dt, s_dt, stream);
    return launch_fdec_hd<_Float16>(a, HD, cs_dt, s_dt, stream);
}

}  // namespace triune
