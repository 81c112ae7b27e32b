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

// ---------------------------------------------------------------------------------------
// One decode step (T == 1) of many rows: the reference's single-token branch
// (fast_gla.py:873-884: prediction from the un-decayed state, decay exp(min(g, 0))), with beta
// per head, per key dim or per value dim as in the chunked forms, and the fp32 state streamed
// once (s0 read, s_final written, nontemporal float4).  The thread layout is the GLA decode
// step's (gla_decode.hip): a 256-thread block takes one state row (b, h) at a time, thread
// (rg, cg) owning rows rg*RPT .. rg*RPT+RPT-1 and columns 4*cg .. 4*cg+3, and walks rows
// blockIdx.x, + gridDim.x, ...  A row loads its q, k, g, v, beta at its top; the next row's
// state loads are issued after the prediction's reduction and complete before this row's state
// is stored (a wave's state reads and writes do not overlap: at the config-2 shape 9.3 us per
// step, against 11.1-11.7 us with the next row's reads in flight during this row's stores).  Two
// reductions over the row groups per row: the prediction S^T k (before the update; every thread
// needs its four columns of it) and the readout S'^T q.  beta (BK != NONE) is fp32.
// ---------------------------------------------------------------------------------------
template <typename T>
using DVec4 = T __attribute__((ext_vector_type(4)));

template <int DK, int DV, int RPT, typename TIO, typename TG, int BK>
__global__ __launch_bounds__(DK * DV / (4 * RPT)) void gdn_decode_kernel(GdnParams a, uint32_t rows) {
    constexpr int TPB = DK * DV / (4 * RPT), CG = DV / 4, WAVES = TPB / 64;
    static_assert(TPB % 64 == 0 && CG <= 64 && RPT % 4 == 0, "unsupported decode tiling");
    const int tid = threadIdx.x;
    const int cg = tid % CG, rg = tid / CG, r0 = rg * RPT, wave = tid / 64;
    const uint32_t H32 = (uint32_t)a.H;  // rows = B * H < 2^31
    __shared__ f32x4 redp[2][WAVES][CG], redo[2][WAVES][CG];
    // A row's inputs in their storage types until used.
    struct In {
        f32x4 st[RPT];
        DVec4<TIO> q[RPT / 4], k[RPT / 4], v;
        DVec4<TG> g[RPT / 4];
        f32x4 bk[BK == BETA_KEY ? RPT / 4 : 1];  // beta per key row (BETA_KEY) or value column (BETA_VALUE)
        float bh;                                // beta per head
    };
    // The state goes through a buffer resource over the row (no records without s0, or when
    // `live` is false past the last row: the loads then read zeros and touch no memory), so every
    // path issues the same loads.
    const int32_t soff = (r0 * DV + 4 * cg) * 4;
    auto fetch_small = [&](In& x, uint32_t row) {
        const int64_t b = row / H32, h = row % H32;
        const TIO* q = reinterpret_cast<const TIO*>(a.q) + b * a.q_sb + h * a.q_sh + r0;
        const TIO* k = reinterpret_cast<const TIO*>(a.k) + b * a.k_sb + h * a.k_sh + r0;
        const TG* g = reinterpret_cast<const TG*>(a.g) + b * a.g_sb + h * a.g_sh + r0;
#pragma unroll
        for (int i = 0; i < RPT / 4; ++i) {
            x.q[i] = reinterpret_cast<const DVec4<TIO>*>(q)[i];
            x.k[i] = reinterpret_cast<const DVec4<TIO>*>(k)[i];
            x.g[i] = reinterpret_cast<const DVec4<TG>*>(g)[i];
        }
        x.v = *reinterpret_cast<const DVec4<TIO>*>(reinterpret_cast<const TIO*>(a.v) + b * a.v_sb + h * a.v_sh + 4 * cg);
        const float* bp = reinterpret_cast<const float*>(a.beta) + b * a.b_sb + h * a.b_sh;
        if constexpr (BK == BETA_HEAD) x.bh = bp[0];
        if constexpr (BK == BETA_KEY) {
#pragma unroll
            for (int i = 0; i < RPT / 4; ++i) x.bk[i] = reinterpret_cast<const f32x4*>(bp + r0)[i];
        }
        if constexpr (BK == BETA_VALUE) x.bk[0] = *reinterpret_cast<const f32x4*>(bp + 4 * cg);
    };
    auto fetch_state = [&](In& x, uint32_t srow, bool live) {
        const bool on = live && a.s0 != nullptr;
        const auto r = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.s0) + (on ? (int64_t)srow * (DK * DV) : 0),
                                                         (short)0, on ? DK * DV * 4 : 0, 0x00020000);
#pragma unroll
        for (int m = 0; m < RPT; ++m)
            x.st[m] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, soff + m * DV * 4, 0, 2));
    };
    auto step = [&](In& cur, In& nxt, uint32_t row, int buf) {
        fetch_small(cur, row);
        const uint32_t nrow = row + gridDim.x;
        const bool more = nrow < rows;
        const int64_t b = row / H32, h = row % H32;
        // prediction S^T k for this thread's four columns
        float p4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < RPT; ++m) {
            const float km = (float)cur.k[m / 4][m % 4];
#pragma unroll
            for (int c = 0; c < 4; ++c) p4[c] += km * cur.st[m][c];
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) p4[c] = xor_group_sum<CG>(p4[c]);
        if ((tid % 64) < CG) redp[buf][wave][cg] = f32x4{p4[0], p4[1], p4[2], p4[3]};
        // barriers order LDS only: the loads and stores in flight need not complete before them
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        f32x4 pred = redp[buf][0][cg];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) pred += redp[buf][w][cg];
        fetch_state(nxt, nrow, more);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        const f32x4 bvc = BK == BETA_VALUE ? cur.bk[0] : f32x4{1.f, 1.f, 1.f, 1.f};
        float y[4];  // the written values u (beta per value column: beta (.) u)
#pragma unroll
        for (int c = 0; c < 4; ++c) y[c] = bvc[c] * ((float)cur.v[c] - pred[c]);
        f32x4 ns[RPT];
        float o4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < RPT; ++m) {
            const float d = expf(fminf((float)cur.g[m / 4][m % 4], 0.f));
            float wm = (float)cur.k[m / 4][m % 4];
            if constexpr (BK == BETA_HEAD) wm *= cur.bh;
            if constexpr (BK == BETA_KEY) wm *= cur.bk[m / 4][m % 4];
            const float qm = (float)cur.q[m / 4][m % 4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                ns[m][c] = d * cur.st[m][c] + wm * y[c];
                o4[c] += qm * ns[m][c];
            }
        }
        {
            // no records without s_final: the stores are issued all the same and dropped
            const bool on = a.s_final != nullptr;
            const auto r = __builtin_amdgcn_make_buffer_rsrc(a.s_final + (on ? (int64_t)row * (DK * DV) : 0), (short)0,
                                                             on ? DK * DV * 4 : 0, 0x00020000);
            typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
            for (int m = 0; m < RPT; ++m)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, ns[m]), r, soff + m * DV * 4, 0, 2);
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) o4[c] = xor_group_sum<CG>(o4[c]);
        if ((tid % 64) < CG) redo[buf][wave][cg] = f32x4{o4[0], o4[1], o4[2], o4[3]};
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        // the readout: threads tid < CG store columns 4*cg .. 4*cg+3; the others issue the same
        // store past the row's records (dropped)
        {
            f32x4 sum = redo[buf][0][cg];
#pragma unroll
            for (int w = 1; w < WAVES; ++w) sum += redo[buf][w][cg];
            const int ob = dt_size(a.o_dt);
            const auto rout = __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<char*>(a.o) + (b * a.o_sb + h * a.o_sh) * ob,
                                                                (short)0, DV * ob, 0x00020000);
            buffer_store4_dt(rout, tid < CG ? 4 * cg * ob : DV * ob, a.o_dt, sum);
        }
    };
    // Two input sets used in turn, so no loaded state is ever copied between registers.
    In A, B;
    uint32_t row = blockIdx.x;
    fetch_state(A, row, true);
    while (row < rows) {
        step(A, B, row, 0);
        row += gridDim.x;
        if (row >= rows) break;
        step(B, A, row, 1);
        row += gridDim.x;
    }
}

// 256 threads: 4 rows per thread at D = 64, 16 at D = 128 (as the GLA decode step).
template <int D, typename TIO, typename TG, int BK>
static hipError_t launch_gdn_decode_t(const GdnParams& a, int max_blocks, hipStream_t stream) {
    constexpr int RPT = (D * D / (4 * 256)) > 4 ? (D * D / (4 * 256)) : 4;
    constexpr int TPB = D * D / (4 * RPT);
    const uint32_t rows = (uint32_t)(a.B * a.H);
    const uint32_t blocks = rows < (uint32_t)max_blocks ? rows : (uint32_t)max_blocks;
    hipLaunchKernelGGL((gdn_decode_kernel<D, D, RPT, TIO, TG, BK>), dim3(blocks), dim3(TPB), 0, stream, a, rows);
    return hipGetLastError();
}

template <int D, typename TIO, typename TG>
static hipError_t launch_gdn_decode_b(const GdnParams& a, int max_blocks, hipStream_t stream) {
    switch (a.beta_kind) {
        case BETA_HEAD: return launch_gdn_decode_t<D, TIO, TG, BETA_HEAD>(a, max_blocks, stream);
        case BETA_KEY: return launch_gdn_decode_t<D, TIO, TG, BETA_KEY>(a, max_blocks, stream);
        case BETA_VALUE: return launch_gdn_decode_t<D, TIO, TG, BETA_VALUE>(a, max_blocks, stream);
        default: return launch_gdn_decode_t<D, TIO, TG, BETA_NONE>(a, max_blocks, stream);
    }
}

template <int D>
static hipError_t launch_gdn_decode_d(const GdnParams& a, int max_blocks, hipStream_t stream) {
    const bool g32 = a.g_dt == DT_F32;
    if (a.io_dt == DT_BF16) {
        if (g32) return launch_gdn_decode_b<D, __bf16, float>(a, max_blocks, stream);
        if (a.g_dt == DT_BF16) return launch_gdn_decode_b<D, __bf16, __bf16>(a, max_blocks, stream);
    } else if (a.io_dt == DT_F16) {
        if (g32) return launch_gdn_decode_b<D, _Float16, float>(a, max_blocks, stream);
        if (a.g_dt == DT_F16) return launch_gdn_decode_b<D, _Float16, _Float16>(a, max_blocks, stream);
    } else if (a.io_dt == DT_F32 && g32) {
        return launch_gdn_decode_b<D, float, float>(a, max_blocks, stream);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_gdn_decode(const GdnParams& a, int D, int max_blocks, hipStream_t stream) {
    if (D == 64) return launch_gdn_decode_d<64>(a, max_blocks, stream);
    if (D == 128) return launch_gdn_decode_d<128>(a, max_blocks, stream);
    return hipErrorInvalidValue;
}

hipError_t launch_gdn_tokenwise(const GdnParams& a, int Dk, int Dv, hipStream_t stream) {
    if (Dk == 64 && Dv == 64) return launch_gdn_t<64, 64, 8>(a, stream);
    if (Dk == 128 && Dv == 128) return launch_gdn_t<128, 128, 8>(a, stream);
    if (Dk == 32 && Dv == 32) return launch_gdn_t<32, 32, 16>(a, stream);
    return hipErrorInvalidValue;
}

}  // namespace triune
