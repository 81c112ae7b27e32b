// gdn_bwd.hip -- gradients of the Gated DeltaNet reference variant (token-serial, recomputed from
// checkpoints).
//
// The reference differentiates fast_recurrent_gated_deltanet (triune/kernels/fast_gla.py:781-836)
// with autograd whenever a gradient is needed (fast_chunk_gated_deltanet, :885-904).  Per token,
// with P = S_{t-1}, a = exp(min(g, 0)), W = w uu^T (w_i = rs_i k_i, uu_j = cs_j u_j: rs, cs the row
// and column beta factors, 1 where the kind has none), u = v - P^T k, S_t = diag(a) P + W,
// o = S_t^T q, and D the gradient reaching S_t:
//   D += q do^T ;  dq_i = sum_j S_t[i][j] do_j
//   c_j = sum_i D[i][j] w_i ;  du_j = cs_j c_j ;  dv_j = du_j ;  dpred_j = -du_j
//   e_i = sum_j D[i][j] uu_j ;  dk_i = rs_i e_i + sum_j P[i][j] dpred_j
//   dbeta: head sum_j u_j c_j ; key k_i e_i ; value u_j c_j
//   dg_i = a_i sum_j D[i][j] P[i][j] where g_i <= 0 (torch.clamp(max=0) passes its gradient there)
//   D <- diag(a) D + k dpred^T ;  ds0 = D after token 0.
//
// Value columns evolve independently in the forward, so a wave owns 8 columns of one (b, h)
// (lane (rg, c): rows rg*RPT .. rg*RPT+RPT-1 of column c, RPT = D/8) and walks the tokens:
//   gdn_ckpt_kernel   forward from s0, storing the state before every L-th token (L = 1024/D or
//                     2048/D);
//   gdn_bwd_kernel    sub-chunks of L tokens last to first: the sub-chunk's inputs are staged in
//                     LDS, its L states before each token recomputed from the checkpoint into LDS,
//                     then the tokens walked backwards; sums over key rows stay in the wave, sums
//                     over value columns (dq, dk, dg, key-beta) are reduced over the wave's 8
//                     columns (a reduce-scatter inside each half DPP row) and written per column
//                     slice;
//   gdn_slice_sum_kernel adds the D/8 slices and writes the gradient in its dtype.
//
// Segments (beta none, per head or per key dim).  D's recurrence does not involve S: per token
// D <- F_t^T (D + q do^T) with F_t = diag(a) - w cs k^T the forward's linear map on a state column
// (S_t = F_t P + w (cs v)^T).  Over a segment of tokens the forward map is S_end = M S_start + N
// (M = F_last ... F_first) and the backward one D_first = M^T D_last + D_loc.  With NSEG segments of
// segc sub-chunks, walked in parallel:
//   gdn_segmap_kernel  per segment: M (walking the identity's columns with v = 0) and N (from zero);
//   gdn_carry_kernel   S_start[s+1] = M_s S_start[s] + N_s into the checkpoints; then, reversed,
//                      D_end[s-1] = M_s^T D_end[s] + D_loc[s] from D_end[NSEG-1] = dS_final;
//   gdn_dloc_kernel    per segment s >= 1: D_loc[s], the walk of D from zero;
//   gdn_ckpt_kernel / gdn_bwd_kernel  per segment from S_start[s] and D_end[s]; the gradient
//                      kernel (about 50 KB of LDS per wave against 13 KB for the others) walks
//                      coarser segments made of whole ones.
// Beta per value column has a map per column (cs_j differs), so it keeps one segment.
#include "kernels.h"

namespace triune {

namespace {

// value columns per wave: 8 (the lane's serial work per token is D/8 rows of one column)
constexpr int GB_CW = 8;

// SL: tokens per sub-chunk (the checkpoint interval), 1024/D or 2048/D (see gdn_bwd_chunk_tokens)
template <int D, int CW, int SL>
struct GbLay {
    static constexpr int NRG = 64 / CW;         // row groups
    static constexpr int RPT = D / NRG;         // rows per lane
    static constexpr int L = SL;
    static constexpr int RPL = RPT / CW;        // rows per lane after the column reduce-scatter (D / 64)
};

// Rows [t0, t0 + nv) of a token tensor (element strides sb, st, sh; W elements from col0) into LDS
// as fp32 [L][W]; rows past nv are zero.  DECAY (the gate): each g is stored as its decay factor
// exp(g) where g <= 0 and as -1 where the clamp min(g, 0) holds it (decay 1, no gradient), so the
// walks take |x| as the decay and x >= 0 as the clamp's pass flag, one exp per element and
// sub-chunk instead of one per lane and token.
template <int L, int W, bool DECAY = false>
__device__ __forceinline__ void stage_rows(float* dst, const void* base, int dt, int64_t sb, int64_t st, int64_t sh,
                                           int64_t b, int64_t t0, int64_t h, int col0, int nv) {
    constexpr int CPR = W / 8;
    const int lane = threadIdx.x;
    const int es = dt_size(dt);
#pragma unroll
    for (int p = lane; p < L * CPR; p += 64) {
        const int tt = p / CPR, c8 = (p % CPR) * 8;
        float x[8];
        const int64_t off = b * sb + (t0 + tt) * st + h * sh + col0 + c8;
        load8_dt(reinterpret_cast<const char*>(base) + off * es, dt, tt < nv, x);
        if constexpr (DECAY) {
#pragma unroll
            for (int i = 0; i < 8; ++i) x[i] = x[i] > 0.f ? -1.f : fast_exp(fminf(x[i], 0.f));
        }
        float4* d4 = reinterpret_cast<float4*>(dst + tt * W + c8);
        d4[0] = make_float4(x[0], x[1], x[2], x[3]);
        d4[1] = make_float4(x[4], x[5], x[6], x[7]);
    }
}

// beta per (token, head) for rows [t0, t0 + nv) into dst[L] (zero past nv).
template <int L>
__device__ __forceinline__ void stage_head_beta(float* dst, const GdnParams& a, int64_t b, int64_t t0, int64_t h,
                                                int nv) {
    const int lane = threadIdx.x;
    if (lane < L) {
        float x = 0.f;
        if (lane < nv) {
            const int64_t off = b * a.b_sb + (t0 + lane) * a.b_st + h * a.b_sh;
            if (a.beta_dt == DT_F32) x = reinterpret_cast<const float*>(a.beta)[off];
            else if (a.beta_dt == DT_BF16) x = (float)reinterpret_cast<const __bf16*>(a.beta)[off];
            else x = (float)reinterpret_cast<const _Float16*>(a.beta)[off];
        }
        dst[lane] = x;
    }
}

template <int N>
__device__ __forceinline__ void lds_read(const float* p, float (&x)[N]) {
#pragma unroll
    for (int m = 0; m < N; m += 4) {
        const float4 v = *reinterpret_cast<const float4*>(p + m);
        x[m] = v.x; x[m + 1] = v.y; x[m + 2] = v.z; x[m + 3] = v.w;
    }
}

// Sum over the row groups (lanes c, c + CW, c + 2 CW, ...) in every lane; lane ^ 8 inside a DPP
// row is the rotation by 8.
template <int CW>
__device__ __forceinline__ float rg_sum(float x) {
    if constexpr (CW == 8) x += row_ror<8>(x);
    return xor_sum<32>(xor_sum<16>(x));
}

// Sum over the CW lanes of a column group (a DPP row for 16, a half row for 8) in every lane.
template <int CW>
__device__ __forceinline__ float cw_sum(float x) {
    x = dpp_add<0xB1>(x);   // quad_perm [1, 0, 3, 2]
    x = dpp_add<0x4E>(x);   // quad_perm [2, 3, 0, 1]
    x = dpp_add<0x141>(x);  // row_half_mirror
    if constexpr (CW == 16) x = dpp_add<0x140>(x);  // row_mirror
    return x;
}

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// One butterfly step of the reduce-scatter over the CW lanes of a column group: the partner
// (lane ^ m, m = 15, 7, 3, 1 through row_mirror, row_half_mirror and two quad permutes) differs in
// bit BIT; a lane keeps the half of its N values that its BIT selects and adds the partner's copy.
template <int RB, int N, int CTRL, int BIT>
__device__ __forceinline__ void rs_step(float (&x)[RB], int c) {
    const bool up = (c >> BIT) & 1;
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
        const float lo = x[i], hi = x[i + N / 2];
        const float send = up ? lo : hi, keep = up ? hi : lo;
        x[i] = keep + dpp_mov<CTRL>(send);
    }
}

// Reduce-scatter over the CW columns of a group: on entry x[0..RPT) holds this lane's terms of
// rows r0 .. r0+RPT; on exit x[0..RPT/CW) holds the sums over the CW lanes of rows
// r0 + c*RPT/CW + [0, RPT/CW).
template <int RPT, int CW>
__device__ __forceinline__ void col_reduce_scatter(float (&x)[RPT], int c) {
    static_assert(RPT % CW == 0, "rows per lane");
    constexpr int N0 = CW == 16 ? RPT : 2 * RPT;  // CW = 8 starts at the half-row mirror
    if constexpr (CW == 16) rs_step<RPT, N0, 0x140, 3>(x, c);  // row_mirror: lane ^ 15
    rs_step<RPT, N0 / 2, 0x141, 2>(x, c);  // row_half_mirror: lane ^ 7
    rs_step<RPT, N0 / 4, 0x1B, 1>(x, c);   // quad_perm [3, 2, 1, 0]: lane ^ 3
    rs_step<RPT, N0 / 8, 0xB1, 0>(x, c);   // quad_perm [1, 0, 3, 2]: lane ^ 1
}

// One forward token on the lane's RPT rows of column c (gg: the staged decay factors, see
// stage_rows): returns u_j (before beta); S updated.
template <int RPT, int CW, int BK>
__device__ __forceinline__ float gb_forward_token(float (&S)[RPT], const float* kq, const float* gg,
                                                  const float* brow, float vj, float bc) {
    float pred = 0.f;
#pragma unroll
    for (int m = 0; m < RPT; ++m) pred = fmaf(kq[m], S[m], pred);
    pred = rg_sum<CW>(pred);
    const float u = vj - pred;
    const float uu = (BK == BETA_HEAD || BK == BETA_VALUE) ? bc * u : u;
#pragma unroll
    for (int m = 0; m < RPT; ++m) {
        const float d = fabsf(gg[m]);
        const float w = BK == BETA_KEY ? brow[m] * kq[m] : kq[m];
        S[m] = fmaf(d, S[m], w * uu);
    }
    return u;
}

}  // namespace


template <int D, int SL, int BK>
__global__ __launch_bounds__(64) void gdn_ckpt_kernel(GdnBwdParams p) {
    using Ly = GbLay<D, GB_CW, SL>;
    constexpr int RPT = Ly::RPT, L = Ly::L;
    const GdnParams& a = p.f;
    __shared__ __attribute__((aligned(16))) float sK[L * D];
    __shared__ __attribute__((aligned(16))) float sG[L * D];
    __shared__ __attribute__((aligned(16))) float sV[L * GB_CW];
    __shared__ __attribute__((aligned(16))) float sB[BK == BETA_KEY ? L * D : (BK == BETA_VALUE ? L * GB_CW : L)];
    const int lane = threadIdx.x, c = lane % GB_CW, rg = lane / GB_CW, r0 = rg * RPT;
    const int64_t bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
    const int col0 = blockIdx.x * GB_CW, col = col0 + c;
    float S[RPT];
    const int64_t DD = (int64_t)D * D;
    const int64_t seg = blockIdx.z, sc0 = seg * p.segc, sc1 = sc0 + p.segc < p.nc ? sc0 + p.segc : p.nc;
    if (seg > 0) {  // the segment's start state, written by the carry
        const float* s = p.ckpt + (bh * p.nc + sc0) * DD + (int64_t)r0 * D + col;
#pragma unroll
        for (int m = 0; m < RPT; ++m) S[m] = s[(int64_t)m * D];
    } else if (a.s0) {
        const float* s = a.s0 + bh * DD + (int64_t)r0 * D + col;
#pragma unroll
        for (int m = 0; m < RPT; ++m) S[m] = s[(int64_t)m * D];
    } else {
#pragma unroll
        for (int m = 0; m < RPT; ++m) S[m] = 0.f;
    }
    for (int64_t sc = sc0; sc < sc1; ++sc) {
        const int64_t t0 = sc * L;
        const int nv = (int)(a.T - t0 < L ? a.T - t0 : L);
        float* ck = p.ckpt + (bh * p.nc + sc) * DD + (int64_t)r0 * D + col;
        if (sc > sc0 || seg == 0) {
#pragma unroll
            for (int m = 0; m < RPT; ++m) ck[(int64_t)m * D] = S[m];
        }
        if (sc + 1 == sc1) break;  // the segment's last sub-chunk's tokens are not needed here
        __syncthreads();
        stage_rows<L, D>(sK, a.k, a.io_dt, a.k_sb, a.k_st, a.k_sh, b, t0, h, 0, nv);
        stage_rows<L, D, true>(sG, a.g, a.g_dt, a.g_sb, a.g_st, a.g_sh, b, t0, h, 0, nv);
        stage_rows<L, GB_CW>(sV, a.v, a.io_dt, a.v_sb, a.v_st, a.v_sh, b, t0, h, col0, nv);
        if constexpr (BK == BETA_HEAD) stage_head_beta<L>(sB, a, b, t0, h, nv);
        if constexpr (BK == BETA_KEY) stage_rows<L, D>(sB, a.beta, a.beta_dt, a.b_sb, a.b_st, a.b_sh, b, t0, h, 0, nv);
        if constexpr (BK == BETA_VALUE)
            stage_rows<L, GB_CW>(sB, a.beta, a.beta_dt, a.b_sb, a.b_st, a.b_sh, b, t0, h, col0, nv);
        __syncthreads();
        for (int tt = 0; tt < nv; ++tt) {
            float kq[RPT], gg[RPT], br[RPT];
            lds_read<RPT>(sK + tt * D + r0, kq);
            lds_read<RPT>(sG + tt * D + r0, gg);
            if constexpr (BK == BETA_KEY) lds_read<RPT>(sB + tt * D + r0, br);
            const float bc = BK == BETA_HEAD ? sB[tt] : (BK == BETA_VALUE ? sB[tt * GB_CW + c] : 1.f);
            gb_forward_token<RPT, GB_CW, BK>(S, kq, gg, br, sV[tt * GB_CW + c], bc);
        }
    }
}

template <int D, int SL, int BK>
__global__ __launch_bounds__(64) void gdn_bwd_kernel(GdnBwdParams p) {
    using Ly = GbLay<D, GB_CW, SL>;
    constexpr int RPT = Ly::RPT, L = Ly::L, RPL = Ly::RPL;
    const GdnParams& a = p.f;
    __shared__ __attribute__((aligned(16))) float sQ[L * D];
    __shared__ __attribute__((aligned(16))) float sK[L * D];
    __shared__ __attribute__((aligned(16))) float sG[L * D];
    __shared__ __attribute__((aligned(16))) float sV[L * GB_CW];
    __shared__ __attribute__((aligned(16))) float sDO[L * GB_CW];
    __shared__ __attribute__((aligned(16))) float sB[BK == BETA_KEY ? L * D : (BK == BETA_VALUE ? L * GB_CW : L)];
    __shared__ __attribute__((aligned(16))) float sP[L * 64 * RPT];  // [token][RPT/4][lane] float4
    __shared__ __attribute__((aligned(16))) float sU[L * 64];
    const int lane = threadIdx.x, c = lane % GB_CW, rg = lane / GB_CW, r0 = rg * RPT;
    const int64_t bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
    const int slice = blockIdx.x, nsl = gridDim.x;
    const int col0 = slice * GB_CW, col = col0 + c;
    const int64_t DD = (int64_t)D * D;
    const int64_t BTH = a.B * a.T * a.H;
    float dS[RPT];
    const int64_t seg = blockIdx.z, sc0 = seg * p.bsegc, sc1 = sc0 + p.bsegc < p.nc ? sc0 + p.bsegc : p.nc;
    const int64_t last = (seg + 1) * p.bsegr < p.nseg ? (seg + 1) * p.bsegr - 1 : p.nseg - 1;  // its last segment
    const float* dsi = p.nseg > 1 ? p.seg_de + (bh * p.nseg + last) * DD : (p.dsf ? p.dsf + bh * DD : nullptr);
    if (dsi) {
        const float* s = dsi + (int64_t)r0 * D + col;
#pragma unroll
        for (int m = 0; m < RPT; ++m) dS[m] = s[(int64_t)m * D];
    } else {
#pragma unroll
        for (int m = 0; m < RPT; ++m) dS[m] = 0.f;
    }
    for (int64_t sc = sc1 - 1; sc >= sc0; --sc) {
        const int64_t t0 = sc * L;
        const int nv = (int)(a.T - t0 < L ? a.T - t0 : L);
        __syncthreads();  // the previous sub-chunk's reads of the staging arrays are done
        stage_rows<L, D>(sQ, a.q, a.io_dt, a.q_sb, a.q_st, a.q_sh, b, t0, h, 0, nv);
        stage_rows<L, D>(sK, a.k, a.io_dt, a.k_sb, a.k_st, a.k_sh, b, t0, h, 0, nv);
        stage_rows<L, D, true>(sG, a.g, a.g_dt, a.g_sb, a.g_st, a.g_sh, b, t0, h, 0, nv);
        stage_rows<L, GB_CW>(sV, a.v, a.io_dt, a.v_sb, a.v_st, a.v_sh, b, t0, h, col0, nv);
        if (p.dout) stage_rows<L, GB_CW>(sDO, p.dout, p.do_dt, p.do_sb, p.do_st, p.do_sh, b, t0, h, col0, nv);
        if constexpr (BK == BETA_HEAD) stage_head_beta<L>(sB, a, b, t0, h, nv);
        if constexpr (BK == BETA_KEY) stage_rows<L, D>(sB, a.beta, a.beta_dt, a.b_sb, a.b_st, a.b_sh, b, t0, h, 0, nv);
        if constexpr (BK == BETA_VALUE)
            stage_rows<L, GB_CW>(sB, a.beta, a.beta_dt, a.b_sb, a.b_st, a.b_sh, b, t0, h, col0, nv);
        float S[RPT];
        {
            const float* ck = p.ckpt + (bh * p.nc + sc) * DD + (int64_t)r0 * D + col;
#pragma unroll
            for (int m = 0; m < RPT; ++m) S[m] = ck[(int64_t)m * D];
        }
        __syncthreads();
        // recompute: the state before each token of the sub-chunk, and u
        for (int tt = 0; tt < nv; ++tt) {
#pragma unroll
            for (int m = 0; m < RPT; m += 4)
                *reinterpret_cast<float4*>(sP + ((tt * (RPT / 4) + m / 4) * 64 + lane) * 4) =
                    make_float4(S[m], S[m + 1], S[m + 2], S[m + 3]);
            float kq[RPT], gg[RPT], br[RPT];
            lds_read<RPT>(sK + tt * D + r0, kq);
            lds_read<RPT>(sG + tt * D + r0, gg);
            if constexpr (BK == BETA_KEY) lds_read<RPT>(sB + tt * D + r0, br);
            const float bc = BK == BETA_HEAD ? sB[tt] : (BK == BETA_VALUE ? sB[tt * GB_CW + c] : 1.f);
            sU[tt * 64 + lane] = gb_forward_token<RPT, GB_CW, BK>(S, kq, gg, br, sV[tt * GB_CW + c], bc);
        }
        __syncthreads();
        for (int tt = nv - 1; tt >= 0; --tt) {
            const int64_t t = t0 + tt;
            float qq[RPT], kq[RPT], gg[RPT], br[RPT], P[RPT];
            lds_read<RPT>(sQ + tt * D + r0, qq);
            lds_read<RPT>(sK + tt * D + r0, kq);
            lds_read<RPT>(sG + tt * D + r0, gg);
            if constexpr (BK == BETA_KEY) lds_read<RPT>(sB + tt * D + r0, br);
#pragma unroll
            for (int m = 0; m < RPT; m += 4) {
                const float4 v4 = *reinterpret_cast<const float4*>(sP + ((tt * (RPT / 4) + m / 4) * 64 + lane) * 4);
                P[m] = v4.x; P[m + 1] = v4.y; P[m + 2] = v4.z; P[m + 3] = v4.w;
            }
            const float u = sU[tt * 64 + lane];
            const float bc = BK == BETA_HEAD ? sB[tt] : (BK == BETA_VALUE ? sB[tt * GB_CW + c] : 1.f);
            const float uu = (BK == BETA_HEAD || BK == BETA_VALUE) ? bc * u : u;
            const float doj = p.dout ? sDO[tt * GB_CW + c] : 0.f;
            float dec[RPT], w[RPT];
            float xq[RPT], xk[RPT], xg[RPT], xb[RPT];
            float cpart = 0.f;
#pragma unroll
            for (int m = 0; m < RPT; ++m) {
                dec[m] = fabsf(gg[m]);
                w[m] = BK == BETA_KEY ? br[m] * kq[m] : kq[m];
                const float st = fmaf(dec[m], P[m], w[m] * uu);  // S_t
                xq[m] = st * doj;
                dS[m] = fmaf(qq[m], doj, dS[m]);
                cpart = fmaf(dS[m], w[m], cpart);
            }
            const float cj = rg_sum<GB_CW>(cpart);
            const float du = (BK == BETA_HEAD || BK == BETA_VALUE) ? bc * cj : cj;
            const float dpred = -du;
#pragma unroll
            for (int m = 0; m < RPT; ++m) {
                const float e = dS[m] * uu;
                xk[m] = fmaf(P[m], dpred, BK == BETA_KEY ? br[m] * e : e);
                if constexpr (BK == BETA_KEY) xb[m] = kq[m] * e;
                xg[m] = dS[m] * P[m];
                dS[m] = fmaf(dec[m], dS[m], kq[m] * dpred);
            }
            if (rg == 0) {
                const int64_t off = ((b * a.T + t) * a.H + h) * D + col;
                if (a.io_dt == DT_F32) reinterpret_cast<float*>(p.dv)[off] = du;
                else if (a.io_dt == DT_BF16) reinterpret_cast<__bf16*>(p.dv)[off] = (__bf16)du;
                else reinterpret_cast<_Float16*>(p.dv)[off] = (_Float16)du;
                if constexpr (BK == BETA_VALUE) {
                    const float db = u * cj;
                    if (p.dbeta_dt == DT_F32) reinterpret_cast<float*>(p.dbeta_v)[off] = db;
                    else if (p.dbeta_dt == DT_BF16) reinterpret_cast<__bf16*>(p.dbeta_v)[off] = (__bf16)db;
                    else reinterpret_cast<_Float16*>(p.dbeta_v)[off] = (_Float16)db;
                }
            }
            if constexpr (BK == BETA_HEAD) {
                const float db = cw_sum<GB_CW>(u * cj);  // the same in every row group
                if (lane == 0) p.part_bh[(int64_t)slice * BTH + (b * a.T + t) * a.H + h] = db;
            }
            col_reduce_scatter<RPT, GB_CW>(xq, c);
            col_reduce_scatter<RPT, GB_CW>(xk, c);
            col_reduce_scatter<RPT, GB_CW>(xg, c);
            if constexpr (BK == BETA_KEY) col_reduce_scatter<RPT, GB_CW>(xb, c);
            // lane (rg, c) now holds rows rg*RPT + c*RPL + [0, RPL): row = lane * RPL + i
            const int64_t tok = ((b * a.T + t) * a.H + h) * D + lane * RPL;
            float* pq = p.part + ((int64_t)0 * nsl + slice) * BTH * D + tok;
            float* pk = p.part + ((int64_t)1 * nsl + slice) * BTH * D + tok;
            float* pg = p.part + ((int64_t)2 * nsl + slice) * BTH * D + tok;
#pragma unroll
            for (int i = 0; i < RPL; ++i) {
                const int row = lane * RPL + i;
                const float gr = sG[tt * D + row];
                pq[i] = xq[i];
                pk[i] = xk[i];
                pg[i] = gr >= 0.f ? xg[i] * gr : 0.f;  // gr: exp(g) where g <= 0, else -1
                if constexpr (BK == BETA_KEY) p.part[((int64_t)3 * nsl + slice) * BTH * D + tok + i] = xb[i];
            }
        }
    }
    if (p.ds0 && seg == 0) {
        float* s = p.ds0 + bh * DD + (int64_t)r0 * D + col;
#pragma unroll
        for (int m = 0; m < RPT; ++m) s[(int64_t)m * D] = dS[m];
    }
}

// Segment maps: grid (2 D / 8, B * H, NSEG).  Slices below D / 8 walk columns of the identity
// with v = 0 (-> M_s), the others the value columns from zero (-> N_s).  Not for beta per value.
template <int D, int SL, int BK>
__global__ __launch_bounds__(64) void gdn_segmap_kernel(GdnBwdParams p) {
    using Ly = GbLay<D, GB_CW, SL>;
    constexpr int RPT = Ly::RPT, L = Ly::L;
    static_assert(BK != BETA_VALUE, "beta per value column has a map per column");
    const GdnParams& a = p.f;
    __shared__ __attribute__((aligned(16))) float sK[L * D];
    __shared__ __attribute__((aligned(16))) float sG[L * D];
    __shared__ __attribute__((aligned(16))) float sV[L * GB_CW];
    __shared__ __attribute__((aligned(16))) float sB[BK == BETA_KEY ? L * D : L];
    const int lane = threadIdx.x, c = lane % GB_CW, rg = lane / GB_CW, r0 = rg * RPT;
    const int64_t bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
    const bool ident = blockIdx.x < D / GB_CW;
    const int col0 = (ident ? (int)blockIdx.x : (int)blockIdx.x - D / GB_CW) * GB_CW, col = col0 + c;
    const int64_t DD = (int64_t)D * D;
    const int64_t seg = blockIdx.z, sc0 = seg * p.segc, sc1 = sc0 + p.segc < p.nc ? sc0 + p.segc : p.nc;
    float S[RPT];
#pragma unroll
    for (int m = 0; m < RPT; ++m) S[m] = ident && r0 + m == col ? 1.f : 0.f;
    for (int64_t sc = sc0; sc < sc1; ++sc) {
        const int64_t t0 = sc * L;
        const int nv = (int)(a.T - t0 < L ? a.T - t0 : L);
        __syncthreads();
        stage_rows<L, D>(sK, a.k, a.io_dt, a.k_sb, a.k_st, a.k_sh, b, t0, h, 0, nv);
        stage_rows<L, D, true>(sG, a.g, a.g_dt, a.g_sb, a.g_st, a.g_sh, b, t0, h, 0, nv);
        if (!ident) stage_rows<L, GB_CW>(sV, a.v, a.io_dt, a.v_sb, a.v_st, a.v_sh, b, t0, h, col0, nv);
        if constexpr (BK == BETA_HEAD) stage_head_beta<L>(sB, a, b, t0, h, nv);
        if constexpr (BK == BETA_KEY) stage_rows<L, D>(sB, a.beta, a.beta_dt, a.b_sb, a.b_st, a.b_sh, b, t0, h, 0, nv);
        __syncthreads();
        for (int tt = 0; tt < nv; ++tt) {
            float kq[RPT], gg[RPT], br[RPT];
            lds_read<RPT>(sK + tt * D + r0, kq);
            lds_read<RPT>(sG + tt * D + r0, gg);
            if constexpr (BK == BETA_KEY) lds_read<RPT>(sB + tt * D + r0, br);
            const float bc = BK == BETA_HEAD ? sB[tt] : 1.f;
            gb_forward_token<RPT, GB_CW, BK>(S, kq, gg, br, ident ? 0.f : sV[tt * GB_CW + c], bc);
        }
    }
    float* o = (ident ? p.seg_m : p.seg_n) + (bh * p.nseg + seg) * DD + (int64_t)r0 * D + col;
#pragma unroll
    for (int m = 0; m < RPT; ++m) o[(int64_t)m * D] = S[m];
}

// D_loc[s] for segments s >= 1: grid (D / 8, B * H, NSEG - 1), the walk of D alone from zero.
template <int D, int SL, int BK>
__global__ __launch_bounds__(64) void gdn_dloc_kernel(GdnBwdParams p) {
    using Ly = GbLay<D, GB_CW, SL>;
    constexpr int RPT = Ly::RPT, L = Ly::L;
    static_assert(BK != BETA_VALUE, "beta per value column has a map per column");
    const GdnParams& a = p.f;
    __shared__ __attribute__((aligned(16))) float sQ[L * D];
    __shared__ __attribute__((aligned(16))) float sK[L * D];
    __shared__ __attribute__((aligned(16))) float sG[L * D];
    __shared__ __attribute__((aligned(16))) float sDO[L * GB_CW];
    __shared__ __attribute__((aligned(16))) float sB[BK == BETA_KEY ? L * D : L];
    const int lane = threadIdx.x, c = lane % GB_CW, rg = lane / GB_CW, r0 = rg * RPT;
    const int64_t bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
    const int col0 = blockIdx.x * GB_CW, col = col0 + c;
    const int64_t DD = (int64_t)D * D;
    const int64_t seg = (int64_t)blockIdx.z + 1, sc0 = seg * p.segc, sc1 = sc0 + p.segc < p.nc ? sc0 + p.segc : p.nc;
    float dS[RPT];
#pragma unroll
    for (int m = 0; m < RPT; ++m) dS[m] = 0.f;
    for (int64_t sc = sc1 - 1; sc >= sc0; --sc) {
        const int64_t t0 = sc * L;
        const int nv = (int)(a.T - t0 < L ? a.T - t0 : L);
        __syncthreads();
        stage_rows<L, D>(sQ, a.q, a.io_dt, a.q_sb, a.q_st, a.q_sh, b, t0, h, 0, nv);
        stage_rows<L, D>(sK, a.k, a.io_dt, a.k_sb, a.k_st, a.k_sh, b, t0, h, 0, nv);
        stage_rows<L, D, true>(sG, a.g, a.g_dt, a.g_sb, a.g_st, a.g_sh, b, t0, h, 0, nv);
        if (p.dout) stage_rows<L, GB_CW>(sDO, p.dout, p.do_dt, p.do_sb, p.do_st, p.do_sh, b, t0, h, col0, nv);
        if constexpr (BK == BETA_HEAD) stage_head_beta<L>(sB, a, b, t0, h, nv);
        if constexpr (BK == BETA_KEY) stage_rows<L, D>(sB, a.beta, a.beta_dt, a.b_sb, a.b_st, a.b_sh, b, t0, h, 0, nv);
        __syncthreads();
        for (int tt = nv - 1; tt >= 0; --tt) {
            float qq[RPT], kq[RPT], gg[RPT], br[RPT];
            lds_read<RPT>(sQ + tt * D + r0, qq);
            lds_read<RPT>(sK + tt * D + r0, kq);
            lds_read<RPT>(sG + tt * D + r0, gg);
            if constexpr (BK == BETA_KEY) lds_read<RPT>(sB + tt * D + r0, br);
            const float bc = BK == BETA_HEAD ? sB[tt] : 1.f;
            const float doj = p.dout ? sDO[tt * GB_CW + c] : 0.f;
            float cpart = 0.f;
#pragma unroll
            for (int m = 0; m < RPT; ++m) {
                dS[m] = fmaf(qq[m], doj, dS[m]);
                cpart = fmaf(dS[m], BK == BETA_KEY ? br[m] * kq[m] : kq[m], cpart);
            }
            const float cj = rg_sum<GB_CW>(cpart);
            const float dpred = -(BK == BETA_HEAD ? bc * cj : cj);
#pragma unroll
            for (int m = 0; m < RPT; ++m) dS[m] = fmaf(fabsf(gg[m]), dS[m], kq[m] * dpred);
        }
    }
    float* o = p.seg_dl + (bh * p.nseg + seg) * DD + (int64_t)r0 * D + col;
#pragma unroll
    for (int m = 0; m < RPT; ++m) o[(int64_t)m * D] = dS[m];
}

// Carry over segments, grid (D / 16, B * H), 256 threads; thread (i0, j) holds rows i0 + 16 m of
// column cb + j.  Forward (REV false): X = S_start[0] (s0 or zero), X <- M_s X + N_s into the
// checkpoint of segment s + 1.  REV: X = dS_final (or zero) into D_end[NSEG-1], X <- M_s^T X +
// D_loc[s] into D_end[s-1].  M_s is staged in LDS each step, X through LDS.
template <int D, bool REV>
__global__ __launch_bounds__(256) void gdn_carry_kernel(GdnBwdParams p) {
    constexpr int NR = D / 16;
    __shared__ __attribute__((aligned(16))) float sM[D * D];
    __shared__ __attribute__((aligned(16))) float sX[D * 16];
    const int t = threadIdx.x, j = t & 15, i0 = t >> 4;
    const int64_t bh = blockIdx.y, DD = (int64_t)D * D;
    const int cb = blockIdx.x * 16;
    auto el = [&](int m) { return (int64_t)(i0 + 16 * m) * D + cb + j; };
    float x[NR];
    const float* x0 = REV ? (p.dsf ? p.dsf + bh * DD : nullptr) : (p.f.s0 ? p.f.s0 + bh * DD : nullptr);
#pragma unroll
    for (int m = 0; m < NR; ++m) x[m] = x0 ? x0[el(m)] : 0.f;
    if constexpr (REV) {
#pragma unroll
        for (int m = 0; m < NR; ++m) p.seg_de[(bh * p.nseg + p.nseg - 1) * DD + el(m)] = x[m];
    }
    for (int64_t n = 1; n < p.nseg; ++n) {
        const int64_t s = REV ? p.nseg - n : n - 1;  // the segment whose map is applied
        const float4* M4 = reinterpret_cast<const float4*>(p.seg_m + (bh * p.nseg + s) * DD);
        const float* Y = (REV ? p.seg_dl : p.seg_n) + (bh * p.nseg + s) * DD;
        __syncthreads();  // the previous step's reads of sM and sX are done
#pragma unroll
        for (int e = t; e < D * D / 4; e += 256) reinterpret_cast<float4*>(sM)[e] = M4[e];
#pragma unroll
        for (int m = 0; m < NR; ++m) sX[(i0 + 16 * m) * 16 + j] = x[m];
        float y[NR];
#pragma unroll
        for (int m = 0; m < NR; ++m) y[m] = Y[el(m)];
        __syncthreads();
#pragma unroll
        for (int m = 0; m < NR; ++m) {
            const int i = i0 + 16 * m;
            float acc = y[m];
#pragma unroll 16
            for (int kk = 0; kk < D; ++kk) acc = fmaf(REV ? sM[kk * D + i] : sM[i * D + kk], sX[kk * 16 + j], acc);
            x[m] = acc;
        }
        float* out = REV ? p.seg_de + (bh * p.nseg + s - 1) * DD : p.ckpt + (bh * p.nc + (s + 1) * p.segc) * DD;
#pragma unroll
        for (int m = 0; m < NR; ++m) out[el(m)] = x[m];
    }
}

// out[i] = sum_s src[s * stride + i] for i < n (0 when src is null), written as dtype dt (contiguous).
__global__ __launch_bounds__(256) void gdn_slice_sum_kernel(const float* src, int nsl, int64_t stride, int64_t n,
                                                            void* out, int dt) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float s = 0.f;
    if (src)
        for (int k = 0; k < nsl; ++k) s += src[k * stride + i];
    if (dt == DT_F32) reinterpret_cast<float*>(out)[i] = s;
    else if (dt == DT_BF16) reinterpret_cast<__bf16*>(out)[i] = (__bf16)s;
    else reinterpret_cast<_Float16*>(out)[i] = (_Float16)s;
}

// Tokens per sub-chunk: 2048/D where every wave has a CU of its own (the longer sub-chunk halves
// the staging round trips; its LDS, about 100 KB, leaves one workgroup per CU), else 1024/D
// (about 50 KB: three per CU, so every wave stays resident).
int gdn_bwd_chunk_tokens(int D, int64_t waves, int64_t cus) { return waves <= cus ? 2048 / D : 1024 / D; }
int gdn_bwd_col_slices(int D) { return D / GB_CW; }

template <int D, int SL, int BK>
static hipError_t launch_gdn_bwd_lk(const GdnBwdParams& p, hipStream_t stream) {
    const unsigned bh = (unsigned)(p.f.B * p.f.H), ns = (unsigned)p.nseg;
    const dim3 grid(D / GB_CW, bh, ns);
    const dim3 bgrid(D / GB_CW, bh, (unsigned)((p.nc + p.bsegc - 1) / p.bsegc));
    hipError_t e;
    if constexpr (BK != BETA_VALUE) {
        if (ns > 1) {
            hipLaunchKernelGGL((gdn_segmap_kernel<D, SL, BK>), dim3(2 * D / GB_CW, bh, ns), dim3(64), 0, stream, p);
            hipLaunchKernelGGL((gdn_carry_kernel<D, false>), dim3(D / 16, bh), dim3(256), 0, stream, p);
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
    } else {
        if (ns != 1) return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL((gdn_ckpt_kernel<D, SL, BK>), grid, dim3(64), 0, stream, p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if constexpr (BK != BETA_VALUE) {
        if (ns > 1) {
            hipLaunchKernelGGL((gdn_dloc_kernel<D, SL, BK>), dim3(D / GB_CW, bh, ns - 1), dim3(64), 0, stream, p);
            hipLaunchKernelGGL((gdn_carry_kernel<D, true>), dim3(D / 16, bh), dim3(256), 0, stream, p);
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
    }
    hipLaunchKernelGGL((gdn_bwd_kernel<D, SL, BK>), bgrid, dim3(64), 0, stream, p);
    return hipGetLastError();
}

template <int D, int BK>
static hipError_t launch_gdn_bwd_dk(const GdnBwdParams& p, hipStream_t stream) {
    if (p.L == 2048 / D) return launch_gdn_bwd_lk<D, 2048 / D, BK>(p, stream);
    if (p.L == 1024 / D) return launch_gdn_bwd_lk<D, 1024 / D, BK>(p, stream);
    if (p.L == 512 / D) return launch_gdn_bwd_lk<D, 512 / D, BK>(p, stream);
    return hipErrorInvalidValue;
}

template <int D>
static hipError_t launch_gdn_bwd_d(const GdnBwdParams& p, hipStream_t stream) {
    switch (p.f.beta_kind) {
        case BETA_HEAD: return launch_gdn_bwd_dk<D, BETA_HEAD>(p, stream);
        case BETA_KEY: return launch_gdn_bwd_dk<D, BETA_KEY>(p, stream);
        case BETA_VALUE: return launch_gdn_bwd_dk<D, BETA_VALUE>(p, stream);
        default: return launch_gdn_bwd_dk<D, BETA_NONE>(p, stream);
    }
}

hipError_t launch_gdn_bwd(const GdnBwdParams& p, int D, hipStream_t stream) {
    if (D == 64) return launch_gdn_bwd_d<64>(p, stream);
    if (D == 128) return launch_gdn_bwd_d<128>(p, stream);
    return hipErrorInvalidValue;
}

hipError_t launch_gdn_slice_sum(const float* src, int nsl, int64_t stride, int64_t n, void* out, int dt,
                                hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(gdn_slice_sum_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, src, nsl, stride,
                       n, out, dt);
    return hipGetLastError();
}

}  // namespace triune
