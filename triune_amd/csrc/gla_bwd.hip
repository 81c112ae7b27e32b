// gla_bwd.hip -- gradients of the chunked GLA prefill for gfx950 (dense [B, T, H, D], Dk == Dv == D).
//
// Reference: fast_chunk_gla's training path (triune/kernels/fast_gla.py:692-778) is autograd
// through _run_gla_chunks (:569-689; g clamped with torch.clamp(max=0), :586) and
// FusedRecurrentScan (:109-203).  Its gradients are those of the token recurrence
//   S_t = diag(a_t) S_{t-1} + k_t v_t^T ,  o_t = S_t^T q_t ,  a_t = exp(g_eff_t)
// (reference check: tests/test_kernels.py:266-327).  With D_t the total gradient reaching S_t,
// D_t = q_t do_t^T + diag(a_{t+1}) D_{t+1} and D_{T-1} = dS_T + q_{T-1} do_{T-1}^T:
//   dq_t = S_t do_t ,  dk_t = D_t v_t ,  dv_t = D_t^T k_t ,  dS0 = diag(a_0) D_0 ,
//   dg_t = sum_{r >= t} (q_r . dq_r - k_r . dk_r) + sum_j dS_T[., j] S_T[., j]   (per key dim)
// The last identity holds because g_t shifts every cumulative decay from t on, and q_r carries
// exp(G_r), k_r exp(-G_r), S_T exp(G_T).  dg is zero where a clamped token had g > 0.
//
// Launch sequence: the forward's K1 and K2 (segment states, carried-in states), then
//   BK3 gla_bwd_state : per (segment, head), chunks first to last from the carried-in state:
//                       each chunk's starting state -> ws_chunk, the segment's end state ->
//                       ws_send, and the segment map R = sum_t diag(exp(G_t)) q_t do_t^T (G from
//                       the segment start, inclusive) -> ws_r
//   reverse scan      : the forward's segment scan over the segments in reverse order with maps
//                       (Gseg, R): the gradient reaching each segment's end state (in place of R)
//                       and dS0
//   BK4 gla_bwd_chunk : per (segment, head), chunks last to first from that gradient.
// Within a chunk (G inclusive from the chunk start, m = G_C / 2, Qt = q e^{G-m}, Kt = k e^{m-G},
// A = causal(Qt Kt^T), B = causal(dO V^T), dH = gradient reaching the chunk's end state):
//   dq = e^{G-m} . (B Kt + dO (e^m S)^T)        dk = e^{m-G} . (B^T Qt + V (e^m dH)^T)
//   dv = A^T dO + Kt (e^m dH)                   dH <- e^{G_C} dH + e^m (Qt^T dO)
// and dg from the in-chunk suffix sums of q.dq - k.dk plus the sum carried from the later
// chunks (started at sum_j dH S over the segment's end state).  Chunks whose decay span exceeds
// SPAN_MAX, or that hold the reference's unclamped 1-token tail, run token by token.
//
// Wave w of a workgroup (NW = D / 16 waves) owns key dims [16w, 16w+16) of dq and dk and value
// columns [16w, 16w+16) of dv and of the carried dH.  Products run on v_mfma_f32_16x16x32_bf16
// with the forward's split-precision operands.
#include "chunk_common.h"

namespace triune {

template <typename TIn, typename TG>
struct BwdIn {
    ChunkIn<TIn, TG, 4> c;  // q, k, g (4 key dims) and v (4 value columns) of tokens 4*tg + j
    Vec<TIn, 4> d[4];       // dO, same columns as v
};

struct BwdAddr {
    ChunkAddr c;
    TokAddr d;
};

template <typename TIn, typename TG>
__device__ __forceinline__ BwdAddr bwd_addr(const BwdParams& a, const Work& wk, int64_t h, int tg, int col) {
    BwdAddr r;
    r.c = chunk_addr<true, TIn, TG>(a.f, wk, h, tg, col, col);
    r.d = tok_addr<TIn>(a.dout, wk, h, tg, col);
    return r;
}

template <bool CK, typename TIn, typename TG>
__device__ __forceinline__ void bwd_load(BwdIn<TIn, TG>& x, const BwdAddr& ad, int64_t tc, bool valid) {
    chunk_load<true, CK>(x.c, ad.c, tc, valid);
    const __amdgpu_buffer_rsrc_t rd = chunk_rsrc(ad.d, tc, valid);
    rows_load<CK>(x.d, rd, ad.d, tc);
}

// Sum over the 16 lanes of each 16-lane group.
__device__ __forceinline__ float sum16(float x) { return dpp_sum16(x); }

// fp32 x added to the four floats at voff (bounded like out_store4: past the records, loads
// read zero and stores are dropped).
__device__ __forceinline__ void out_acc4(const OutRsrc& r, int voff, f32x4 x) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const f32x2 a = __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(r.lo, voff, 0, 0));
    const f32x2 b = __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(r.hi, voff + 8, 0, 0));
    x[0] += a[0]; x[1] += a[1]; x[2] += b[0]; x[3] += b[1];
    out_store4(r, voff, DT_F32, x);
}

// Four values at columns [col, col+4) of rows 4*tg + j (j < 4) of the chunk at tc: bounded
// buffer stores over the chunk's nv rows (rows past the end are dropped).  acc: added to the
// (fp32) values there.
__device__ __forceinline__ void store_rows4(const RowsOut& o, int D, int64_t tc, int nv, int tg, int col,
                                            const float (&x)[4][4], bool acc = false) {
    const int es = o.es, dt = o.dt;
    const int64_t ost = o.ost;
    char* b0 = o.base + uniform_i64(tc * ost);
    const int n = nv > 0 ? (int)((nv - 1) * ost + D * es) : 0;
    OutRsrc r;
    r.lo = __builtin_amdgcn_make_buffer_rsrc(b0, (short)0, n, 0x00020000);
    r.hi = __builtin_amdgcn_make_buffer_rsrc(b0, (short)0, dt == DT_F32 ? n : 0, 0x00020000);
    if (acc) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            out_acc4(r, (int32_t)((4 * tg + j) * ost) + col * es, f32x4{x[j][0], x[j][1], x[j][2], x[j][3]});
        return;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
        out_store4(r, (int32_t)((4 * tg + j) * ost) + col * es, dt, f32x4{x[j][0], x[j][1], x[j][2], x[j][3]});
}

// Four D-layout tiles o[tb] (lane (g4, r16): token 16*tb + r16, columns 4*g4 .. 4*g4+3 of the
// wave's 16) staged through `stage` (16 x os floats of this wave) and stored as rows.
__device__ __forceinline__ void store_tiles(char* obase, int64_t ost, int es, int dt, int nv, const f32x4 (&o)[4],
                                            float* stage, int os, bool acc = false) {
    const int lane = threadIdx.x & 63, r16 = lane & 15, g4 = lane >> 4;
    const int q = lane & 3, tq = (lane >> 4) + 4 * ((lane >> 2) & 3);
    const int32_t olane = (int32_t)(tq * ost) + 4 * q * es;
    const OutRsrc orr = out_rsrc(obase, ost, es, nv, dt == DT_F32);
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
        *reinterpret_cast<f32x4*>(stage + r16 * os + 4 * g4) = o[tb];
        const f32x4 x = *reinterpret_cast<const f32x4*>(stage + tq * os + 4 * q);
        if (acc) out_acc4(orr, (int32_t)(16 * tb * ost) + olane, x);
        else out_store4(orr, (int32_t)(16 * tb * ost) + olane, dt, x);
    }
}

__device__ __forceinline__ void store1_dt(char* p, int dt, float x) {
    if (dt == DT_F32) *reinterpret_cast<float*>(p) = x;
    else if (dt == DT_BF16) *reinterpret_cast<__bf16*>(p) = (__bf16)x;
    else *reinterpret_cast<_Float16*>(p) = (_Float16)x;
}

// =======================================================================================
// BK3: chunk starting states, segment end state, segment map R.
// =======================================================================================
template <typename TIn, int D>
struct BLayS {
    using P = Prec<TIn>;
    static constexpr int NS = P::NS, NX = P::NX, NW = D / 16;
    static constexpr int RS = D + PAD, ROWP = CHUNK * RS * 2;
    static constexpr int VS = 16, VPP = CHUNK * VS * 2;
    static constexpr int OFF_KW = 0;                       // k e^{decay after t}
    static constexpr int OFF_QW = OFF_KW + NS * ROWP;      // q e^{decay from the segment start}
    static constexpr int OFF_VP = OFF_QW + NS * ROWP;      // each wave's 16 value columns of V
    static constexpr int OFF_DP = OFF_VP + NW * NX * VPP;  // ... and of dO
    static constexpr int OFF_EG = OFF_DP + NW * NX * VPP;
    static constexpr int BYTES = OFF_EG + D * 4;
    static_assert(BYTES <= 80 * 1024, "two workgroups per CU");
};

// CK: checked row addressing; without it the loads zero rows past the chunk (see chunk_load).
template <typename TIn, typename TG, int D, bool CK>
struct BwdStateStep {
    using L = BLayS<TIn, D>;
    static constexpr int NS = L::NS, NX = L::NX, NDB = D / 16, DL = 4;

    template <typename Hook>
    __device__ static void run(const BwdParams& a, const Work& wk, int64_t tc, int nv, const BwdIn<TIn, TG>& cur,
                               f32x4 (&S)[NDB], f32x4 (&R)[NDB], float (&Gpre)[DL], float* cs, char* smem,
                               Hook&& after_inputs) {
        const int lane = threadIdx.x & 63, wave = wave_id(), r16 = lane & 15, g4 = lane >> 4;
        const int tg = lane >> 2, row = lane & 3;
        const int dl0 = 16 * wave + DL * row;
        char* sKW = smem + L::OFF_KW;
        char* sQW = smem + L::OFF_QW;
        char* sVP = smem + L::OFF_VP + wave * NX * L::VPP;
        char* sDP = smem + L::OFF_DP + wave * NX * L::VPP;
        float* sEG = reinterpret_cast<float*>(smem + L::OFF_EG);
        {
            float G[4][DL], X[4][DL], GC[DL], x[4][DL];
            chunk_float<CK>(cur.c.g, x, tg, nv);
            const bool tail_chunk = (a.f.flags & 1) && (tc + nv == wk.len);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bool unclamped = tail_chunk && (4 * tg + j == nv - 1);
#pragma unroll
                for (int i = 0; i < DL; ++i) G[j][i] = unclamped ? x[j][i] : fminf(x[j][i], 0.f);
            }
            chunk_suffix<DL>(G, X, GC, lane);  // X: decay after each token, within the chunk
            chunk_cumsum<DL>(G, GC, lane);     // G: decay from the chunk start, inclusive
            chunk_float<CK>(cur.c.k, x, tg, nv);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int i = 0; i < DL; ++i) x[j][i] *= fast_exp(X[j][i]);
                lds_put_row<NS, DL>(sKW, L::ROWP, (4 * tg + j) * L::RS + dl0, x[j]);
            }
            chunk_float<CK>(cur.c.q, x, tg, nv);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int i = 0; i < DL; ++i) x[j][i] *= fast_exp(Gpre[i] + G[j][i]);
                lds_put_row<NS, DL>(sQW, L::ROWP, (4 * tg + j) * L::RS + dl0, x[j]);
            }
#pragma unroll
            for (int i = 0; i < DL; ++i) Gpre[i] += GC[i];
            if (tg == 0) {
#pragma unroll
                for (int i = 0; i < DL; ++i) sEG[dl0 + i] = fast_exp(GC[i]);
            }
            float vx[4][4];
            chunk_float<CK>(cur.c.v, vx, tg, nv);
#pragma unroll
            for (int j = 0; j < 4; ++j) lds_put_row<NX, 4>(sVP, L::VPP, (4 * tg + j) * L::VS + 4 * row, vx[j]);
            chunk_float<CK>(cur.d, vx, tg, nv);
#pragma unroll
            for (int j = 0; j < 4; ++j) lds_put_row<NX, 4>(sDP, L::VPP, (4 * tg + j) * L::VS + 4 * row, vx[j]);
        }
        after_inputs();
        __syncthreads();
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) cs[state_off(db, i, g4, r16, wave, D)] = S[db][i];
        Split8<NX> vf[2], df[2];
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
            vf[k2] = lds_frag_tr<NX>(sVP, L::VPP, L::VS, 32 * k2, 0, g4, r16);
            df[k2] = lds_frag_tr<NX>(sDP, L::VPP, L::VS, 32 * k2, 0, g4, r16);
        }
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            f32x4 P = zero4();
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2) {
                P = mfma_split<NS, NX, NS>(lds_frag_tr<NS>(sKW, L::ROWP, L::RS, 32 * k2, 16 * db, g4, r16), vf[k2], P);
                R[db] = mfma_split<NS, NX, NS>(lds_frag_tr<NS>(sQW, L::ROWP, L::RS, 32 * k2, 16 * db, g4, r16),
                                               df[k2], R[db]);
            }
            const f32x4 eg = *reinterpret_cast<const f32x4*>(sEG + 16 * db + 4 * g4);
#pragma unroll
            for (int i = 0; i < 4; ++i) S[db][i] = eg[i] * S[db][i] + P[i];
        }
        __syncthreads();  // the next chunk rewrites LDS
    }
};

// CK: checked row addressing (T is not a multiple of 4; see chunk_load).
template <typename TIn, typename TG, int D, bool CK>
__global__ __launch_bounds__(D * 4, 2) void gla_bwd_state_kernel(BwdParams a) {
    using St = BwdStateStep<TIn, TG, D, CK>;
    using L = typename St::L;
    constexpr int NDB = D / 16, DL = 4;
    __shared__ __attribute__((aligned(16))) char smem[L::BYTES];
    const int64_t w = blockIdx.x, h = blockIdx.y;
    Work wk;
    if (!find_work(a.f, w, wk)) return;
    const int lane = threadIdx.x & 63, wave = wave_id(), r16 = lane & 15, g4 = lane >> 4;
    const int tg = lane >> 2, row = lane & 3;
    const int64_t DD = (int64_t)D * D;
    f32x4 S[NDB], R[NDB];
    float Gpre[DL];
    const float* sin = a.f.ws_state + (w * a.f.H + h) * DD;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
        R[db] = zero4();
#pragma unroll
        for (int i = 0; i < 4; ++i) S[db][i] = sin[state_off(db, i, g4, r16, wave, D)];
    }
#pragma unroll
    for (int i = 0; i < DL; ++i) Gpre[i] = 0.f;
    const BwdAddr ad = bwd_addr<TIn, TG>(a, wk, h, tg, 16 * wave + 4 * row);
    const int64_t nch = (wk.t_end - wk.t_begin + CHUNK - 1) / CHUNK;
    auto chunk_nv = [&](int64_t c) {
        const int64_t r = wk.t_end - (wk.t_begin + c * CHUNK);
        return (int)(r < CHUNK ? r : CHUNK);
    };
    auto tok = [&](int64_t c) { return wk.t_begin + c * CHUNK; };
    float* cbase = a.ws_chunk + (wk.b * a.f.H + h) * a.nchunks * DD;
    BwdIn<TIn, TG> A;
    bwd_load<CK>(A, ad, tok(0), true);
    for (int64_t c = 0; c < nch; ++c)
        St::run(a, wk, tok(c), chunk_nv(c), A, S, R, Gpre, cbase + (tok(c) / CHUNK) * DD, smem,
                [&] { bwd_load<CK>(A, ad, tok(c + 1), c + 1 < nch); });
    float* so = a.ws_send + (w * a.f.H + h) * DD;
    float* ro = a.ws_r + (w * a.f.H + h) * DD;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            so[state_off(db, i, g4, r16, wave, D)] = S[db][i];
            ro[state_off(db, i, g4, r16, wave, D)] = R[db][i];
        }
}

// =======================================================================================
// BK4: dq, dk, dv, dg, chunks last to first.
// =======================================================================================
template <typename TIn, int D>
struct BLay {
    using P = Prec<TIn>;
    static constexpr int NS = P::NS, NX = P::NX, NW = D / 16;
    static constexpr int RS = D + PAD, ROWP = CHUNK * RS * 2;  // token-major [64][RS] bf16 planes
    static constexpr int TS = CHUNK + PAD, TP = CHUNK * TS * 2;  // [64 tokens][TS] planes of A and B
    static constexpr int HS = D + PAD, HP = D * HS * 2;          // [D value][HS] plane of e^m dH
    static constexpr int FS = D + 4;                             // fp32 [64][FS] dq / dk staging
    static constexpr int OS = 20;                                // dv staging row stride (floats)
    static constexpr int OFF_QT = 0;
    static constexpr int OFF_KT = OFF_QT + NS * ROWP;
    static constexpr int OFF_V = OFF_KT + NS * ROWP;
    static constexpr int OFF_DO = OFF_V + NX * ROWP;
    static constexpr int OFF_PA = OFF_DO + NX * ROWP;
    static constexpr int OFF_PB = OFF_PA + NS * TP;
    static constexpr int OFF_PH = OFF_PB + NS * TP;
    static constexpr int OFF_EM = OFF_PH + NS * HP;
    static constexpr int OFF_EG = OFF_EM + D * 4;
    static constexpr int OFF_FLAG = OFF_EG + D * 4;
    static constexpr int OFF_C = OFF_FLAG + 16 * 4;
    static constexpr int BYTES = OFF_C + NW * D * 4;
    static constexpr int OFF_FQ = OFF_PA;  // over the A / B planes once stage 3 is done
    static constexpr int OFF_FK = OFF_PA + CHUNK * FS * 4;
    static_assert(2 * CHUNK * FS * 4 <= 2 * NS * TP, "dq / dk staging fits over the A and B planes");
    static_assert(NW * 16 * OS * 4 <= NS * HP, "dv staging fits over the dH plane");
    static_assert(BYTES <= 160 * 1024, "LDS budget");
};

// Token-by-token gradients of one chunk (large decay spans, unclamped tail).  dH (value columns
// of this wave) enters as the gradient reaching the chunk's end state and leaves as the one
// reaching its start state.  dq and dk go to the fp32 planes sFQ / sFK (zeroed by the caller)
// through LDS atomics, dv straight to memory.
template <typename TIn, typename TG, int D>
__device__ void bwd_tokenwise(const BwdParams& a, const Work& wk, int64_t h, int64_t tc, int nv,
                              f32x4 (&dH)[D / 16], float* sFQ, float* sFK, int fs) {
    constexpr int NDB = D / 16;
    const int lane = threadIdx.x & 63, wave = wave_id(), r16 = lane & 15, g4 = lane >> 4;
    const int c0 = 16 * wave;
    const int64_t DD = (int64_t)D * D;
    const float* cs = a.ws_chunk + ((wk.b * a.f.H + h) * a.nchunks + tc / CHUNK) * DD;
    f32x4 S[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) S[db][i] = cs[state_off(db, i, g4, r16, wave, D)];
    auto decay = [&](int64_t tt, int d, bool unclamped) {
        const float gg = (float)tok_row<TG>(a.f.g, wk, tt, h, d)[0];
        return expf(unclamped ? gg : fminf(gg, 0.f));
    };
    for (int t = 0; t < nv; ++t) {  // forward: S_t, dq_t = S_t do_t
        const int64_t tt = tc + t;
        const bool unclamped = (a.f.flags & 1) && (tt == wk.len - 1);
        const float vv = (float)tok_row<TIn>(a.f.v, wk, tt, h, c0)[r16];
        const float dd = (float)tok_row<TIn>(a.dout, wk, tt, h, c0)[r16];
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int d = 16 * db + 4 * g4 + i;
                const float kk = (float)tok_row<TIn>(a.f.k, wk, tt, h, d)[0];
                S[db][i] = decay(tt, d, unclamped) * S[db][i] + kk * vv;
                const float p = sum16(S[db][i] * dd);
                if (r16 == 0) atomicAdd(sFQ + t * fs + d, p);
            }
    }
    f32x4 Dm[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) Dm[db] = dH[db];
    const int es = dt_size(a.d_dt);
    for (int t = nv - 1; t >= 0; --t) {  // reverse: D_t, dk_t = D_t v_t, dv_t = D_t^T k_t
        const int64_t tt = tc + t;
        const bool unclamped = (a.f.flags & 1) && (tt == wk.len - 1);
        const float vv = (float)tok_row<TIn>(a.f.v, wk, tt, h, c0)[r16];
        const float dd = (float)tok_row<TIn>(a.dout, wk, tt, h, c0)[r16];
        float dvp = 0.f;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int d = 16 * db + 4 * g4 + i;
                const float qq = (float)tok_row<TIn>(a.f.q, wk, tt, h, d)[0];
                const float kk = (float)tok_row<TIn>(a.f.k, wk, tt, h, d)[0];
                Dm[db][i] += qq * dd;
                const float p = sum16(Dm[db][i] * vv);
                if (r16 == 0) atomicAdd(sFK + t * fs + d, p);
                dvp += Dm[db][i] * kk;
            }
        dvp += __shfl_xor(dvp, 16);
        dvp += __shfl_xor(dvp, 32);
        if (g4 == 0) {
            char* p = reinterpret_cast<char*>(a.dv) +
                      (wk.b * a.dv_sb + (wk.row0 + tt) * a.dv_st + h * a.dv_sh + c0 + r16) * es;
            if (a.acc & 2) *reinterpret_cast<float*>(p) += dvp;
            else store1_dt(p, a.d_dt, dvp);
        }
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) Dm[db][i] *= decay(tt, 16 * db + 4 * g4 + i, unclamped);
    }
#pragma unroll
    for (int db = 0; db < NDB; ++db) dH[db] = Dm[db];
}

template <typename TIn, typename TG, int D, bool CK>
struct BwdStep {
    using L = BLay<TIn, D>;
    static constexpr int NS = L::NS, NX = L::NX, NW = L::NW, NDB = D / 16, NKS = D / 32, DL = 4;
    // q, k, g, v, dO arrive as one LDS tile set (tile_dma) where it fits beside the planes: the next
    // chunk's tiles are issued once every wave has read this chunk's (after stage 1) and have
    // landed by the wait before this chunk's stores, so the next step reads them after the
    // barrier that follows those stores.
    static constexpr int RB = D * 2, TB = CHUNK * RB;
    static constexpr bool DMA = tile_dma_inputs<TIn, TG, D, D>() && L::BYTES + 5 * TB <= 160 * 1024;

    // Causal 16x16 tiles (key block sb <= query block tb) of X^T with X[t][s] = U_t . W_s over D,
    // for tiles first, first + NW, ... < 10; stored masked as rows of the plane P[t][s].
    template <int NU, int NWP>
    __device__ static void causal_tiles(const char* sU, const char* sW, int plane_bytes, char* sP, int first) {
        const int lane = threadIdx.x & 63, r16 = lane & 15, g4 = lane >> 4;
        constexpr int MT = (10 + NW - 1) / NW;
        int sb[MT], tb[MT];
        f32x4 acc[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            tile_sb_tb(min(first + t * NW, 9), sb[t], tb[t]);
            acc[t] = zero4();
        }
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
            Split8<NWP> wf[MT];
            Split8<NU> uf[MT];
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                wf[t] = lds_frag<NWP>(sW, plane_bytes, L::RS, 16 * sb[t] + r16, 32 * ks, g4);
                uf[t] = lds_frag<NU>(sU, plane_bytes, L::RS, 16 * tb[t] + r16, 32 * ks, g4);
            }
#pragma unroll
            for (int t = 0; t < MT; ++t) acc[t] = mfma_split<NWP, NU, NS>(wf[t], uf[t], acc[t]);
        }
        f32x4 diag;  // row = key 4*g4 + j, column = query r16
#pragma unroll
        for (int j = 0; j < 4; ++j) diag[j] = (4 * g4 + j > r16) ? 0.f : 1.f;
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            if (first + t * NW >= 10) continue;
            const f32x4 m = sb[t] == tb[t] ? diag : f32x4{1.f, 1.f, 1.f, 1.f};
            const float x[4] = {acc[t][0] * m[0], acc[t][1] * m[1], acc[t][2] * m[2], acc[t][3] * m[3]};
            lds_put_row<NS, 4>(sP, L::TP, (16 * tb[t] + r16) * L::TS + 16 * sb[t] + 4 * g4, x);
        }
    }

    template <typename Hook, typename TileHook>
    __device__ static void run(const BwdParams& a, const Work& wk, int64_t h, int64_t tc, int nv,
                               BwdIn<TIn, TG>& cur, f32x4 (&dH)[NDB], float (&acc)[DL], char* smem,
                               const char* tiles, const RowsOut (&go)[4], Hook&& after_inputs,
                               TileHook&& issue_tiles) {
        const int lane = threadIdx.x & 63, wave = wave_id(), r16 = lane & 15, g4 = lane >> 4;
        const int tg = lane >> 2, row = lane & 3;
        const int c0 = 16 * wave;       // key dims of dq / dk, value columns of dv / dH
        const int dl0 = c0 + DL * row;  // stage-1 key dims of this lane
        char* sQT = smem + L::OFF_QT;
        char* sKT = smem + L::OFF_KT;
        char* sV = smem + L::OFF_V;
        char* sDO = smem + L::OFF_DO;
        char* sPA = smem + L::OFF_PA;
        char* sPB = smem + L::OFF_PB;
        char* sPH = smem + L::OFF_PH;
        float* sEM = reinterpret_cast<float*>(smem + L::OFF_EM);
        float* sEG = reinterpret_cast<float*>(smem + L::OFF_EG);
        int* sFLAG = reinterpret_cast<int*>(smem + L::OFF_FLAG);
        float* sFQ = reinterpret_cast<float*>(smem + L::OFF_FQ);
        float* sFK = reinterpret_cast<float*>(smem + L::OFF_FK);
        const bool tail_chunk = (a.f.flags & 1) && (tc + nv == wk.len);

        // Rows i = c0 + r16 of the chunk's starting state (stage 3's dq term), loaded now so that
        // stages 1 and 2 cover their latency.
        f32x4 sprev[NKS][2];
        {
            const float* sp = a.ws_chunk + ((wk.b * a.f.H + h) * a.nchunks + tc / CHUNK) * (int64_t)D * D +
                              (int64_t)(c0 + r16) * D;
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
                sprev[ks][0] = *reinterpret_cast<const f32x4*>(sp + 32 * ks + 4 * g4);
                sprev[ks][1] = *reinterpret_cast<const f32x4*>(sp + 32 * ks + 16 + 4 * g4);
            }
        }
        // ---------------- stage 1: factors, split operands -> LDS ---------------------------
        if constexpr (DMA) {
            tile_rows<RB, 0>(cur.c.q, tiles, tg, dl0);
            tile_rows<RB, 0>(cur.c.k, tiles + TB, tg, dl0);
            tile_rows<RB, 0>(cur.c.g, tiles + 2 * TB, tg, dl0);
            tile_rows<RB, 0>(cur.c.v, tiles + 3 * TB, tg, c0 + 4 * row);
            tile_rows<RB, 0>(cur.d, tiles + 4 * TB, tg, c0 + 4 * row);
        }
        float qx[4][DL], kx[4][DL], fq[4][DL];
        uint32_t pass = 0;  // bit 4*j + i: token 4*tg + j, dim dl0 + i passes its gate gradient
        {
            float G[4][DL], GC[DL];
            chunk_float<CK>(cur.c.g, G, tg, nv);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bool unclamped = tail_chunk && (4 * tg + j == nv - 1);
#pragma unroll
                for (int i = 0; i < DL; ++i) {
                    const float gr = G[j][i];
                    pass |= (unclamped || !(gr > 0.f)) ? (1u << (4 * j + i)) : 0u;
                    G[j][i] = unclamped ? gr : fminf(gr, 0.f);
                }
            }
            chunk_cumsum<DL>(G, GC, lane);
            bool bad = tail_chunk;
#pragma unroll
            for (int i = 0; i < DL; ++i) bad |= !(GC[i] >= -SPAN_MAX);
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int i = 0; i < DL; ++i) fq[j][i] = fast_exp(G[j][i] - 0.5f * GC[i]);
            if (tg == 0) {
#pragma unroll
                for (int i = 0; i < DL; ++i) {
                    const float em = fast_exp(0.5f * GC[i]);
                    sEM[dl0 + i] = em;
                    sEG[dl0 + i] = em * em;
                }
            }
            const bool any_bad = __any(bad);
            if (lane == 0) sFLAG[wave] = any_bad ? 1 : 0;
            chunk_float<CK>(cur.c.q, qx, tg, nv);
            chunk_float<CK>(cur.c.k, kx, tg, nv);
            float x[DL];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int i = 0; i < DL; ++i) x[i] = qx[j][i] * fq[j][i];
                lds_put_row<NS, DL>(sQT, L::ROWP, (4 * tg + j) * L::RS + dl0, x);
#pragma unroll
                for (int i = 0; i < DL; ++i) x[i] = kx[j][i] * __builtin_amdgcn_rcpf(fq[j][i]);
                lds_put_row<NS, DL>(sKT, L::ROWP, (4 * tg + j) * L::RS + dl0, x);
            }
            float vx[4][4];
            chunk_float<CK>(cur.c.v, vx, tg, nv);
#pragma unroll
            for (int j = 0; j < 4; ++j) lds_put_row<NX, 4>(sV, L::ROWP, (4 * tg + j) * L::RS + c0 + 4 * row, vx[j]);
            chunk_float<CK>(cur.d, vx, tg, nv);
#pragma unroll
            for (int j = 0; j < 4; ++j) lds_put_row<NX, 4>(sDO, L::ROWP, (4 * tg + j) * L::RS + c0 + 4 * row, vx[j]);
        }
        after_inputs();
        block_sync<DMA>();
        if constexpr (DMA) {
            // the starting-state rows (loaded at the top, stage 1 covered their latency) are in, so
            // stage 3's use of them waits for nothing issued later; then the next chunk's tiles,
            // every wave having read this chunk's
            wait_vmem();
            issue_tiles();
        }
        bool fast = true;
#pragma unroll
        for (int w = 0; w < NW; ++w) fast = fast && (sFLAG[w] == 0);

        f32x4 dQ[4], dK[4], dV[4];
        if (fast) {
            // ---------------- stage 2: A, B tiles; this wave's e^m dH -> PH[j][i] ---------------
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
                const f32x4 em = *reinterpret_cast<const f32x4*>(sEM + 16 * db + 4 * g4);
                const float x[4] = {dH[db][0] * em[0], dH[db][1] * em[1], dH[db][2] * em[2], dH[db][3] * em[3]};
                lds_put_row<NS, 4>(sPH, L::HP, (c0 + r16) * L::HS + 16 * db + 4 * g4, x);
            }
            causal_tiles<NS, NS>(sQT, sKT, L::ROWP, sPA, wave);                         // A[t][s] = Qt_t . Kt_s
            causal_tiles<NX, NX>(sDO, sV, L::ROWP, sPB, (wave + NW - 10 % NW) % NW);   // B[t][s] = dO_t . V_s
            block_sync<DMA>();

            // ---------------- stage 3 ------------------------------------------------------
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) dQ[tb] = dK[tb] = dV[tb] = zero4();
            const bf16x8 z8 = {};
            // dQ^T[i][t] += (e^m S)[i][.] dO[t][.]: rows i = c0 + r16 of the chunk's starting state
            {
                const float emi = sEM[c0 + r16];
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) {
                    const f32x4 lo = sprev[ks][0], hi = sprev[ks][1];
                    const float x[8] = {lo[0] * emi, lo[1] * emi, lo[2] * emi, lo[3] * emi,
                                        hi[0] * emi, hi[1] * emi, hi[2] * emi, hi[3] * emi};
                    const Split8<NS> sf = split8<NS>(x);
#pragma unroll
                    for (int tb = 0; tb < 4; ++tb)
                        dQ[tb] = mfma_split<NS, NX, NS>(sf, lds_frag<NX>(sDO, L::ROWP, L::RS, 16 * tb + r16, 32 * ks, g4),
                                                        dQ[tb]);
                }
            }
            // dQ^T[i][t] += Kt^T[i][s] B[t][s], s <= t
            {
                Split8<NS> kt[2];
#pragma unroll
                for (int k2 = 0; k2 < 2; ++k2) kt[k2] = lds_frag_tr<NS>(sKT, L::ROWP, L::RS, 32 * k2, c0, g4, r16);
#pragma unroll
                for (int tb = 0; tb < 4; ++tb)
#pragma unroll
                    for (int k2 = 0; k2 <= tb / 2; ++k2) {
                        Split8<NS> pb = lds_frag<NS>(sPB, L::TP, L::TS, 16 * tb + r16, 32 * k2, g4);
                        if (2 * k2 + 1 > tb) {  // key block 2*k2+1 lies above the diagonal
#pragma unroll
                            for (int pl = 0; pl < NS; ++pl)
                                pb.p[pl] = bf16x8{pb.p[pl][0], pb.p[pl][1], pb.p[pl][2], pb.p[pl][3], z8[0], z8[1], z8[2], z8[3]};
                        }
                        dQ[tb] = mfma_split<NS, NS, NS>(kt[k2], pb, dQ[tb]);
                    }
            }
            // dK^T[i][t] += Qt^T[i][r] B[r][t], r >= t;  dV^T[j][t] += dO^T[j][r] A[r][t], r >= t
            {
                Split8<NS> qt[2];
                Split8<NX> dt[2];
#pragma unroll
                for (int k2 = 0; k2 < 2; ++k2) {
                    qt[k2] = lds_frag_tr<NS>(sQT, L::ROWP, L::RS, 32 * k2, c0, g4, r16);
                    dt[k2] = lds_frag_tr<NX>(sDO, L::ROWP, L::RS, 32 * k2, c0, g4, r16);
                }
#pragma unroll
                for (int tb = 0; tb < 4; ++tb)
#pragma unroll
                    for (int k2 = tb / 2; k2 < 2; ++k2) {
                        Split8<NS> pbt = lds_frag_tr<NS>(sPB, L::TP, L::TS, 32 * k2, 16 * tb, g4, r16);
                        Split8<NS> pat = lds_frag_tr<NS>(sPA, L::TP, L::TS, 32 * k2, 16 * tb, g4, r16);
                        if (2 * k2 < tb) {  // rows of block 2*k2 lie above the diagonal
#pragma unroll
                            for (int pl = 0; pl < NS; ++pl) {
                                pbt.p[pl] = bf16x8{z8[0], z8[1], z8[2], z8[3], pbt.p[pl][4], pbt.p[pl][5], pbt.p[pl][6], pbt.p[pl][7]};
                                pat.p[pl] = bf16x8{z8[0], z8[1], z8[2], z8[3], pat.p[pl][4], pat.p[pl][5], pat.p[pl][6], pat.p[pl][7]};
                            }
                        }
                        dK[tb] = mfma_split<NS, NS, NS>(qt[k2], pbt, dK[tb]);
                        dV[tb] = mfma_split<NX, NS, NS>(dt[k2], pat, dV[tb]);
                    }
            }
            // dK^T[i][t] += (e^m dH)[i][j] V[t][j]  (rows i of e^m dH from the PH plane)
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
                const Split8<NS> hf = lds_frag_tr<NS>(sPH, L::HP, L::HS, 32 * ks, c0, g4, r16);
#pragma unroll
                for (int tb = 0; tb < 4; ++tb)
                    dK[tb] = mfma_split<NS, NX, NS>(hf, lds_frag<NX>(sV, L::ROWP, L::RS, 16 * tb + r16, 32 * ks, g4), dK[tb]);
            }
            // dV^T[j][t] += (e^m dH)^T[j][i] Kt[t][i]  (this wave's dH columns, from registers)
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
                const f32x4 e0 = *reinterpret_cast<const f32x4*>(sEM + 32 * ks + 4 * g4);
                const f32x4 e1 = *reinterpret_cast<const f32x4*>(sEM + 32 * ks + 16 + 4 * g4);
                float x[8];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    x[i] = dH[2 * ks][i] * e0[i];
                    x[4 + i] = dH[2 * ks + 1][i] * e1[i];
                }
                const Split8<NS> hf = split8<NS>(x);
#pragma unroll
                for (int tb = 0; tb < 4; ++tb)
                    dV[tb] = mfma_split<NS, NS, NS>(hf, lds_frag<NS>(sKT, L::ROWP, L::RS, 16 * tb + r16, 32 * ks, g4), dV[tb]);
            }
            // dH <- e^{G_C} dH + e^m (Qt^T dO)
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
                f32x4 P = zero4();
#pragma unroll
                for (int k2 = 0; k2 < 2; ++k2)
                    P = mfma_split<NS, NX, NS>(lds_frag_tr<NS>(sQT, L::ROWP, L::RS, 32 * k2, 16 * db, g4, r16),
                                               lds_frag_tr<NX>(sDO, L::ROWP, L::RS, 32 * k2, c0, g4, r16), P);
                const f32x4 em = *reinterpret_cast<const f32x4*>(sEM + 16 * db + 4 * g4);
                const f32x4 eg = *reinterpret_cast<const f32x4*>(sEG + 16 * db + 4 * g4);
#pragma unroll
                for (int i = 0; i < 4; ++i) dH[db][i] = eg[i] * dH[db][i] + em[i] * P[i];
            }
        } else {
            // token by token: zero the dq / dk planes (nobody reads the A / B planes now)
            for (int e = threadIdx.x; e < 2 * CHUNK * L::FS; e += NW * 64) sFQ[e] = 0.f;  // sFK follows sFQ
            block_sync<DMA>();
            bwd_tokenwise<TIn, TG, D>(a, wk, h, tc, nv, dH, sFQ, sFK, L::FS);
        }
        block_sync<DMA>();  // stage 3 is done with every plane
        wait_vmem();  // the next chunk's inputs (registers, or tiles: read after the barrier below) are
                      // in, so this chunk's stores do not delay them
        if (fast) {
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) {
                *reinterpret_cast<f32x4*>(sFQ + (16 * tb + r16) * L::FS + c0 + 4 * g4) = dQ[tb];
                *reinterpret_cast<f32x4*>(sFK + (16 * tb + r16) * L::FS + c0 + 4 * g4) = dK[tb];
            }
            const RowsOut& ov = go[2];
            store_tiles(ov.base + uniform_i64(tc * ov.ost + c0 * ov.es), ov.ost, ov.es, ov.dt, nv, dV,
                        reinterpret_cast<float*>(sPH) + wave * 16 * L::OS, L::OS, (a.acc & 2) != 0);
        }
        block_sync<DMA>();

        // ---------------- epilogue (stage-1 layout): dq, dk, dg ------------------------------
        {
            float dq[4][DL], dk[4][DL], x[4][DL], X[4][DL], tot[DL];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const f32x4 u = *reinterpret_cast<const f32x4*>(sFQ + (4 * tg + j) * L::FS + dl0);
                const f32x4 w = *reinterpret_cast<const f32x4*>(sFK + (4 * tg + j) * L::FS + dl0);
#pragma unroll
                for (int i = 0; i < DL; ++i) {
                    const float f = fast ? fq[j][i] : 1.f;
                    const float rf = fast ? __builtin_amdgcn_rcpf(fq[j][i]) : 1.f;
                    dq[j][i] = u[i] * f;
                    dk[j][i] = w[i] * rf;
                    x[j][i] = qx[j][i] * dq[j][i] - kx[j][i] * dk[j][i];
                }
            }
            chunk_suffix<DL>(x, X, tot, lane);
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int i = 0; i < DL; ++i) {
                    const float dgv = acc[i] + X[j][i] + x[j][i];
                    X[j][i] = ((pass >> (4 * j + i)) & 1u) ? dgv : 0.f;
                }
#pragma unroll
            for (int i = 0; i < DL; ++i) acc[i] += tot[i];
            const bool acc = (a.acc & 1) != 0;
            store_rows4(go[0], D, tc, nv, tg, dl0, dq, acc);
            store_rows4(go[1], D, tc, nv, tg, dl0, dk, acc);
            store_rows4(go[3], D, tc, nv, tg, dl0, X, acc);
        }
    }
};

template <typename TIn, typename TG, int D, bool CK>
__global__ __launch_bounds__(D * 4, 1) void gla_bwd_chunk_kernel(BwdParams a) {
    using St = BwdStep<TIn, TG, D, CK>;
    using L = typename St::L;
    constexpr int NDB = D / 16, DL = 4;
    __shared__ __attribute__((aligned(16))) char smem[L::BYTES];
    __shared__ __attribute__((aligned(16))) char tiles[St::DMA ? 5 * St::TB : 16];
    const int64_t w = blockIdx.x, h = blockIdx.y;
    Work wk;
    if (!find_work(a.f, w, wk)) return;
    const int lane = threadIdx.x & 63, wave = wave_id(), r16 = lane & 15, g4 = lane >> 4;
    const int tg = lane >> 2, row = lane & 3;
    const int64_t DD = (int64_t)D * D;
    // the gradient reaching the segment's end state; the dg carry starts at sum_j dH S there
    f32x4 dH[NDB];
    const float* rp = a.ws_r + (w * a.f.H + h) * DD;
    const float* ep = a.ws_send + (w * a.f.H + h) * DD;
    float* sC = reinterpret_cast<float*>(smem + L::OFF_C);
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t off = state_off(db, i, g4, r16, wave, D);
            dH[db][i] = rp[off];
            const float p = sum16(dH[db][i] * ep[off]);
            if (r16 == 0) sC[wave * D + 16 * db + 4 * g4 + i] = p;
        }
    __syncthreads();
    float acc[DL];
#pragma unroll
    for (int i = 0; i < DL; ++i) {
        float s = 0.f;
#pragma unroll
        for (int ww = 0; ww < L::NW; ++ww) s += sC[ww * D + 16 * wave + DL * row + i];
        acc[i] = s;
    }
    const BwdAddr ad = bwd_addr<TIn, TG>(a, wk, h, tg, 16 * wave + 4 * row);
    const int64_t nch = (wk.t_end - wk.t_begin + CHUNK - 1) / CHUNK;
    auto chunk_nv = [&](int64_t c) {
        const int64_t r = wk.t_end - (wk.t_begin + c * CHUNK);
        return (int)(r < CHUNK ? r : CHUNK);
    };
    auto tok = [&](int64_t c) { return wk.t_begin + c * CHUNK; };
    const RowsOut go[4] = {rows_out(a.dq, a.dq_sb, a.dq_st, a.dq_sh, a.d_dt, wk, h),
                           rows_out(a.dk, a.dk_sb, a.dk_st, a.dk_sh, a.d_dt, wk, h),
                           rows_out(a.dv, a.dv_sb, a.dv_st, a.dv_sh, a.d_dt, wk, h),
                           rows_out(a.dg, a.dg_sb, a.dg_st, a.dg_sh, a.dg_dt, wk, h)};
    BwdIn<TIn, TG> A;
    if constexpr (St::DMA) {
        const TokAddr* const src[5] = {&ad.c.q, &ad.c.k, &ad.c.g, &ad.c.v, &ad.d};
        auto fill = [&](int64_t c1) {
            if (c1 >= 0) tiles_from<St::RB, 0>(tiles, src, tok(c1), wave, lane);
        };
        fill(nch - 1);
        wait_vmem();  // the first chunk's tiles (later ones land before each chunk's stores)
        lds_sync();
        for (int64_t c = nch - 1; c >= 0; --c)
            St::run(a, wk, h, tok(c), chunk_nv(c), A, dH, acc, smem, tiles, go, [] {}, [&] { fill(c - 1); });
        return;
    }
    bwd_load<CK>(A, ad, tok(nch - 1), true);
    for (int64_t c = nch - 1; c >= 0; --c)
        St::run(a, wk, h, tok(c), chunk_nv(c), A, dH, acc, smem, tiles, go,
                [&] { bwd_load<CK>(A, ad, tok(c - 1), c >= 1); }, [] {});
}

// ---------------------------------------------------------------------------------------
// Host launchers.
// ---------------------------------------------------------------------------------------
bool gla_bwd_supported(int D, int io_dt) { return D == 32 || (D == 64 && io_dt != DT_F32); }

template <typename TIn, typename TG, bool CK>
static hipError_t launch_bwd_ck(const BwdParams& a, int64_t n_work, bool chunk, hipStream_t stream) {
    const dim3 grid((unsigned)n_work, (unsigned)a.f.H);
    const dim3 block((unsigned)(a.f.Dk * 4));
#define TRIUNE_BWD_CASE(D_)                                                                                   \
    if (a.f.Dk == D_) {                                                                                       \
        if (chunk) hipLaunchKernelGGL((gla_bwd_chunk_kernel<TIn, TG, D_, CK>), grid, block, 0, stream, a);    \
        else hipLaunchKernelGGL((gla_bwd_state_kernel<TIn, TG, D_, CK>), grid, block, 0, stream, a);          \
        return hipGetLastError();                                                                             \
    }
    TRIUNE_BWD_CASE(32)
    if constexpr (!Prec<TIn>::F32) {
        TRIUNE_BWD_CASE(64)
    }
#undef TRIUNE_BWD_CASE
    return hipErrorInvalidValue;
}

// Unchecked row addressing only when T is a whole number of four-row groups.
template <typename TIn, typename TG>
static hipError_t launch_bwd_t(const BwdParams& a, int64_t n_work, bool chunk, hipStream_t stream) {
    if (!a.f.varlen && a.f.T % 4 == 0) return launch_bwd_ck<TIn, TG, false>(a, n_work, chunk, stream);
    return launch_bwd_ck<TIn, TG, true>(a, n_work, chunk, stream);
}

static hipError_t launch_bwd(const BwdParams& a, int64_t n_work, int io_dt, bool chunk, hipStream_t stream) {
    const bool g32 = a.f.g_dt == DT_F32;
    if (io_dt == DT_BF16) {
        if (g32) return launch_bwd_t<__bf16, float>(a, n_work, chunk, stream);
        if (a.f.g_dt == DT_BF16) return launch_bwd_t<__bf16, __bf16>(a, n_work, chunk, stream);
    } else if (io_dt == DT_F16) {
        if (g32) return launch_bwd_t<_Float16, float>(a, n_work, chunk, stream);
        if (a.f.g_dt == DT_F16) return launch_bwd_t<_Float16, _Float16>(a, n_work, chunk, stream);
    } else if (io_dt == DT_F32 && g32) {
        return launch_bwd_t<float, float>(a, n_work, chunk, stream);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_gla_bwd_state(const BwdParams& a, int64_t n_work, int io_dt, hipStream_t stream) {
    return launch_bwd(a, n_work, io_dt, false, stream);
}

hipError_t launch_gla_bwd_chunk(const BwdParams& a, int64_t n_work, int io_dt, hipStream_t stream) {
    return launch_bwd(a, n_work, io_dt, true, stream);
}

}  // namespace triune
