// gdn.hip -- Gated DeltaNet forward, the reference variant, token-serial form.
//
// Reference: triune/kernels/fast_gla.py:781-836 (fast_recurrent_gated_deltanet) and
// :383-477 (Triton per-token kernel):
//   u_t = v_t - S_{t-1}^T k_t                  (prediction from the un-decayed state)
//   S_t = diag(exp(min(g_t, 0))) S_{t-1} + beta_t . (k_t u_t^T)
//   o_t = S_t^T q_t
// beta: none (1), one scalar per (token, head), per key dim (scales rows; the reference's
// PyTorch path) or per value dim (scales columns; the reference's Triton path).
//
// Value columns of S evolve independently, so a wave owns a slice of DVS columns of one
// (b, h) and walks the tokens; lane (rg, c) holds rows rg*RPT .. rg*RPT+RPT-1 of column c.
#include "kernels.h"

namespace triune {

__device__ __forceinline__ float ld1(const void* p, int dt, int64_t i) {
    if (dt == DT_F32) return reinterpret_cast<const float*>(p)[i];
    if (dt == DT_BF16) return (float)reinterpret_cast<const __bf16*>(p)[i];
    return (float)reinterpret_cast<const _Float16*>(p)[i];
}

template <int DK, int DV, int DVS>
__global__ __launch_bounds__(64) void gdn_tokenwise_kernel(GdnParams a) {
    constexpr int RG = 64 / DVS, RPT = DK / RG;
    static_assert(RPT % 8 == 0, "rows per lane must be a multiple of 8");
    const int lane = threadIdx.x;
    const int c = lane % DVS, rg = lane / DVS, r0 = rg * RPT;
    const int64_t bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
    const int col = blockIdx.x * DVS + c;

    float S[RPT];
    if (a.s0) {
        const float* p = a.s0 + bh * (int64_t)(DK * DV) + (int64_t)r0 * DV + col;
#pragma unroll
        for (int m = 0; m < RPT; ++m) S[m] = p[(int64_t)m * DV];
    } else {
#pragma unroll
        for (int m = 0; m < RPT; ++m) S[m] = 0.f;
    }
    const int isz = dt_size(a.io_dt), gsz = dt_size(a.g_dt);
    for (int64_t t = 0; t < a.T; ++t) {
        float kq[RPT], qq[RPT], gd[RPT];
        const char* kp = reinterpret_cast<const char*>(a.k) + (b * a.k_sb + t * a.k_st + h * a.k_sh + r0) * isz;
        const char* qp = reinterpret_cast<const char*>(a.q) + (b * a.q_sb + t * a.q_st + h * a.q_sh + r0) * isz;
        const char* gp = reinterpret_cast<const char*>(a.g) + (b * a.g_sb + t * a.g_st + h * a.g_sh + r0) * gsz;
#pragma unroll
        for (int m = 0; m < RPT; m += 8) {
            float x[8];
            load8_dt(kp + m * isz, a.io_dt, true, x);
#pragma unroll
            for (int j = 0; j < 8; ++j) kq[m + j] = x[j];
            load8_dt(qp + m * isz, a.io_dt, true, x);
#pragma unroll
            for (int j = 0; j < 8; ++j) qq[m + j] = x[j];
            load8_dt(gp + m * gsz, a.g_dt, true, x);
#pragma unroll
            for (int j = 0; j < 8; ++j) gd[m + j] = expf(fminf(x[j], 0.f));
        }
        const float vc = ld1(a.v, a.io_dt, b * a.v_sb + t * a.v_st + h * a.v_sh + col);
        float bcol = 1.f;
        float brow[RPT];
#pragma unroll
        for (int m = 0; m < RPT; ++m) brow[m] = 1.f;
        const int64_t bbase = b * a.b_sb + t * a.b_st + h * a.b_sh;
        if (a.beta_kind == BETA_HEAD) bcol = ld1(a.beta, a.beta_dt, bbase);
        else if (a.beta_kind == BETA_VALUE) bcol = ld1(a.beta, a.beta_dt, bbase + col);
        else if (a.beta_kind == BETA_KEY) {
#pragma unroll
            for (int m = 0; m < RPT; ++m) brow[m] = ld1(a.beta, a.beta_dt, bbase + r0 + m);
        }
        float pred = 0.f;
#pragma unroll
        for (int m = 0; m < RPT; ++m) pred += kq[m] * S[m];
#pragma unroll
        for (int sh = DVS; sh < 64; sh <<= 1) pred += __shfl_xor(pred, sh);
        const float uc = (vc - pred) * bcol;
        float oc = 0.f;
#pragma unroll
        for (int m = 0; m < RPT; ++m) {
            S[m] = gd[m] * S[m] + brow[m] * kq[m] * uc;
            oc += qq[m] * S[m];
        }
#pragma unroll
        for (int sh = DVS; sh < 64; sh <<= 1) oc += __shfl_xor(oc, sh);
        if (rg == 0) {
            const int64_t off = b * a.o_sb + t * a.o_st + h * a.o_sh + col;
            if (a.o_dt == DT_F32) reinterpret_cast<float*>(a.o)[off] = oc;
            else if (a.o_dt == DT_BF16) reinterpret_cast<__bf16*>(a.o)[off] = (__bf16)oc;
            else reinterpret_cast<_Float16*>(a.o)[off] = (_Float16)oc;
        }
    }
    if (a.s_final) {
        float* p = a.s_final + bh * (int64_t)(DK * DV) + (int64_t)r0 * DV + col;
#pragma unroll
        for (int m = 0; m < RPT; ++m) p[(int64_t)m * DV] = S[m];
    }
}

template <int DK, int DV, int DVS>
static hipError_t launch_gdn_t(const GdnParams& a, hipStream_t stream) {
    dim3 grid(DV / DVS, (unsigned)(a.B * a.H));
    hipLaunchKernelGGL((gdn_tokenwise_kernel<DK, DV, DVS>), grid, dim3(64), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_gdn_tokenwise(const GdnParams& a, int Dk, int Dv, hipStream_t stream) {
    if (Dk == 64 && Dv == 64) return launch_gdn_t<64, 64, 8>(a, stream);
    if (Dk == 128 && Dv == 128) return launch_gdn_t<128, 128, 8>(a, stream);
    if (Dk == 32 && Dv == 32) return launch_gdn_t<32, 32, 16>(a, stream);
    return hipErrorInvalidValue;
}

}  // namespace triune
