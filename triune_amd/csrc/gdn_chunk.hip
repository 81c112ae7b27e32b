// gdn_chunk.hip -- chunked Gated DeltaNet prefill for gfx950 (WY/UT form, LDS-staged, MFMA).
//
// Recurrence (reference: triune/kernels/fast_gla.py:781-836 fast_recurrent_gated_deltanet,
// :383-477 the Triton per-token kernel), per (sequence, head):
//   u_t = v_t - S_{t-1}^T k_t ,  S_t = D_t S_{t-1} + w_t u_t^T ,  o_t = S_t^T q_t
// with D_t = diag(exp(min(g_t, 0))) and w_t = beta_t * k_t (beta per token, per key dim, or 1;
// beta per value dim scales u_t instead, see col_solve).  Head dims Dk = Dv = D in {64, 128}: one
// wave per 16 value columns.
//
// Chunk form (C = 64 tokens, G = inclusive cumulative log-decay inside the chunk, Gp = G - g the
// exclusive one, m = G_C / 2 per key dim, S0 the state at the chunk start, S' = e^m S0):
//   Qt = q e^{G-m},  Wt = w e^{m-G},  Bt = k e^{Gp-m}          (|exponents| <= span / 2)
//   L  = strictly_lower(Bt Wt^T),  A = lower(Qt Wt^T)
//   U  = (I + L)^{-1} (V - Bt S')                                (the UT transform)
//   O  = Qt S' + A U ,   S_C = e^m (S' + Wt^T U)
// (I + L)^{-1} is applied block-wise on 16-token blocks: U_i = T_ii (R_i - sum_{j<i} L_ij U_j),
// with each 16x16 unit-lower inverse T_ii = prod_k (I + M^(2^k)), M = -L_ii, by doubling.
// The chunk map S0 -> S_C is affine with a full Dk x Dk matrix, so segments compose as
// S_in[p+1] = M_p S_in[p] + N_p:
//   K1 gdn_seg_mn   : per (segment, head) the segment map applied to [I | 0] with V replaced by 0
//                     (-> M_p) and to 0 with the real V (-> N_p), sharing the per-chunk factors,
//                     tiles and inverses
//   K2 gdn_seg_scan : per (sequence, head, 16 columns; one wave per 16 rows) the carry S_in[p]
//                     (written in place of N_p)
//   K3 gdn_seg_out  : per (segment, head) the chunk walk from S_in[p], writing o (beta per value
//                     dim: the whole sequence from s0, writing the final state too)
// Products run on v_mfma_f32_16x16x32_bf16 with operands split into bf16 parts (2 for 16-bit
// I/O, 3 for fp32) and fp32 accumulation, as in the GLA prefill.  Chunks whose decay span
// exceeds GDN_SPAN_MAX run token by token.
#include "gdn_common.h"

namespace triune {

// Largest chunk decay span (-G_C per key dim) of the factored form.  Every factor then lies in
// e^[-64, 64], where all bf16 parts of an operand (the third one, 2^-18 below it, included) are
// normal numbers; only products of non-causal pairs (up to e^128) overflow, and every one of
// those sits in a diagonal tile that a select (never a multiply) replaces with 0.  The
// reference's bf16 GLA chunk kernel allows 160 (fast_gla.py:377).
constexpr float GDN_SPAN_MAX = 128.f;

// LDS layout of one (segment, head) workgroup at head dim D (Dk = Dv = D, one wave per 16 value
// columns; stage 1 gives every wave 16 key dims).
template <typename TIn, bool OUT, int D>
struct GLay {
    using P = Prec<TIn>;
    static constexpr int DK = D, DV = D, NW = D / 16, DPW = 16, DL = 4;
    static constexpr int RS = DK + PAD, VS = 16;
    static constexpr int ROWP = CHUNK * RS * 2;
    static constexpr int VPP = CHUNK * VS * 2;
    static constexpr int TILEP = 10 * 64 * 4 * 2;  // ten 16x16 tiles (causal blocks), one bf16 part
    static constexpr int LTP = 6 * 64 * 4 * 2;     // the six off-diagonal blocks of L^T
    static constexpr int DIAGP = 4 * 64 * 4 * 2;   // four 16x16 tiles
    static constexpr int OFF_QT = 0;
    static constexpr int OFF_WT = OFF_QT + (OUT ? P::NS * ROWP : 0);
    static constexpr int OFF_BT = OFF_WT + P::NS * ROWP;
    static constexpr int OFF_AT = OFF_BT + P::NS * ROWP;
    static constexpr int OFF_LT = OFF_AT + (OUT ? P::NS * TILEP : 0);
    static constexpr int OFF_TI = OFF_LT + P::NS * LTP;
    static constexpr int OFF_VP = OFF_TI + P::NS * DIAGP;
    static constexpr int OFF_FAC = OFF_VP + NW * P::NX * VPP;
    static constexpr int OFF_FLAG = OFF_FAC + DK * 4;
    static constexpr int BYTES = OFF_FLAG + NW * 4;
    static constexpr int OS = 20;
    static_assert(16 * OS * 4 <= P::NX * VPP, "output staging fits in a wave's V planes");
    static_assert(BYTES <= 160 * 1024, "LDS budget");
};

// Inputs of a GDN chunk: the GLA chunk inputs plus, when PBK, per-key-dim beta (BETA_KEY, fp32)
// loaded a chunk ahead with them.  Without PBK (D = 128, where those 16 registers would spill)
// stage 1 reads the beta rows of its own chunk.
template <typename TIn, typename TG, bool PBK>
struct GChunkIn {
    ChunkIn<TIn, TG, 4> x;
    Vec<float, 4> bk[PBK ? 4 : 1];
};

template <bool OUT, bool CK, typename TIn, typename TG, bool PBK>
__device__ __forceinline__ void gchunk_load(GChunkIn<TIn, TG, PBK>& c, const ChunkAddr& ad, const TokAddr& kb,
                                            bool key_beta, int64_t tc, bool valid) {
    chunk_load<OUT, CK>(c.x, ad, tc, valid);
    if constexpr (PBK) {
        if (key_beta) {
            const __amdgpu_buffer_rsrc_t r = chunk_rsrc(kb, tc, valid);
            rows_load<CK>(c.bk, r, kb, tc);
        }
    }
}

// One chunk of the GDN walk for (segment, head).  OUT: outputs from the state S (K3).  Otherwise
// (K1) the segment map on two states at once: S driven with V = 0 (the M columns) and SN with
// the real V (the N columns); stages 1-2 (factors, tiles, inverses) are shared by both.
// skip_m (K1): S is left as it is (the map of a segment whose carried-in state is zero is
// never used).
// CK: checked row addressing; without it the loads zero rows past the chunk (see chunk_load).
// Per-value-column beta (BV): with y_t = beta_t (.) u_t the recurrence is S_t = D_t S + k_t y_t^T,
// so the factors are the beta-free ones (W0 = k e^{m-G}, L0 = strictly_lower(Bt W0^T),
// A0 = lower(Qt W0^T)) and, column by column,
//   y_t = beta_t (R_t - sum_{s<t} L0[t,s] y_s),   O = Qt S' + A0 Y,   S_C = e^m (S' + W0^T Y).
// Blocks of 16 tokens keep the MFMA form for every off-diagonal term; inside a diagonal block each
// column has its own triangular system (its own beta), solved here by forward substitution.
// Lane (g4, r16) holds tokens 4*g4 .. 4*g4 + 3 of column r16 (the MFMA D layout), so the block
// runs as four 4-token steps: lanes g4 == o solve their own 4x4 system in registers, the four
// results go to the column's other lanes (ds_bpermute), and every lane subtracts their
// contributions with its rows of L0.  sL: the block's L0 in fp32, [16][16] row-major with the
// four-column group of row t stored at group (group ^ (t >> 2)), so the 16 lanes of a g4 group read
// one address and the four groups four bank ranges; entries with t <= s hold 0.
__device__ __forceinline__ f32x4 col_solve(const f32x4& X0, const f32x4& bt, const float* sL, int g4, int r16) {
    f32x4 X = X0, Y = zero4();
#pragma unroll
    for (int o = 0; o < 4; ++o) {
        f32x4 Lg[4];  // L0[4*g4 + k][4*o + j]: the own diagonal block where g4 == o
#pragma unroll
        for (int k = 0; k < 4; ++k) Lg[k] = *reinterpret_cast<const f32x4*>(sL + (4 * g4 + k) * 16 + 4 * (o ^ g4));
        float y[4];
        y[0] = bt[0] * X[0];
        y[1] = bt[1] * (X[1] - Lg[1][0] * y[0]);
        y[2] = bt[2] * (X[2] - Lg[2][0] * y[0] - Lg[2][1] * y[1]);
        y[3] = bt[3] * (X[3] - Lg[3][0] * y[0] - Lg[3][1] * y[1] - Lg[3][2] * y[2]);
        const bool own = g4 == o;
#pragma unroll
        for (int j = 0; j < 4; ++j) Y[j] = own ? y[j] : Y[j];
        float yb[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) yb[j] = __shfl(y[j], 16 * o + r16);
        // rows below sub-block o (lanes g4 > o); zeros of L0 above the diagonal make it a no-op
        // for g4 < o, and lanes g4 == o no longer read X
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int j = 0; j < 4; ++j) X[k] -= Lg[k][j] * yb[j];
    }
    return Y;
}

// D: head dim (NDB = D/16 state row tiles per wave, NKS = D/32 K steps over key dims).  BV: beta
// per value column (BETA_VALUE, fp32 in `kb`).
template <typename TIn, typename TG, bool OUT, bool CK, int D, bool BV>
struct GdnStep {
    using L = GLay<TIn, OUT, D>;
    using PR = Prec<TIn>;
    static constexpr int NS = PR::NS, NX = PR::NX, DL = 4, NW = L::NW, NDB = D / 16, NKS = D / 32;
    // Stage 2 at D = 128: waves 0-3 form the A^T / L^T tiles, waves 4-7 the four diagonal
    // inverses (about as much MFMA work as four tiles each); at D = 64 every wave does both.
    static constexpr int TW = NW >= 8 ? 4 : NW, DW0 = NW >= 8 ? 4 : 0;
    static constexpr bool PBK = D == 64;
    // K1 at D = 128 holds two 128-row states: the next chunk's input registers are issued between
    // its two passes (live through one of them) rather than after stage 1, where they spilled.
    static constexpr bool LATE_LOAD = !OUT && D > 64;
    // K3 at D = 128: issued after the chunk's output stores, before its state update.
    static constexpr bool LATE_LOAD_OUT = OUT && D > 64;

    // Lane context of wave `wave` (0 .. NW - 1: its 16 value columns and stage-1 dims) in the chunk
    // region at smem.
    struct Ctx {
        int lane, wave, r16, g4, tg, row, c0, dl0;
        char *sQT, *sWT, *sBT, *sAT, *sLT, *sTI, *sVP;
        float* sEM;
        int* sFLAG;
    };
    __device__ static Ctx ctx(char* smem, int wave) {
        int lane = threadIdx.x & 63;
        // At D = 128 the planes span more than the 64 KB reach of an LDS instruction's offset, so
        // every operand read needs its own lane address; computed once per kernel they outlive
        // the register file and spill.  An opaque lane index per chunk keeps them in the step.
        if constexpr (D > 64) asm volatile("" : "+v"(lane));
        Ctx c;
        c.lane = lane;
        c.wave = wave;
        c.r16 = lane & 15;
        c.g4 = lane >> 4;
        c.tg = lane >> 2;
        c.row = lane & 3;
        c.c0 = wave * 16;
        c.dl0 = wave * 16 + DL * c.row;
        c.sQT = smem + L::OFF_QT;
        c.sWT = smem + L::OFF_WT;
        c.sBT = smem + L::OFF_BT;
        c.sAT = smem + L::OFF_AT;
        c.sLT = smem + L::OFF_LT;
        c.sTI = smem + L::OFF_TI;
        c.sVP = smem + L::OFF_VP + wave * NX * L::VPP;
        c.sEM = reinterpret_cast<float*>(smem + L::OFF_FAC);
        c.sFLAG = reinterpret_cast<int*>(smem + L::OFF_FLAG);
        return c;
    }

    // Stage 1: factors and split operands of the chunk -> LDS, and this wave's span flag.
    __device__ static void stage1(const PrefillParams& a, const Work& wk, int64_t h, int64_t tc, int nv,
                                  const GChunkIn<TIn, TG, PBK>& cur, const TokAddr& kb, const Ctx& c) {
        const int lane = c.lane, wave = c.wave, r16 = c.r16, g4 = c.g4, tg = c.tg, row = c.row, c0 = c.c0,
                  dl0 = c.dl0;
        char *sQT = c.sQT, *sWT = c.sWT, *sBT = c.sBT, *sAT = c.sAT, *sLT = c.sLT, *sTI = c.sTI, *sVP = c.sVP;
        float* sEM = c.sEM;
        int* sFLAG = c.sFLAG;
        (void)lane; (void)wave; (void)r16; (void)g4; (void)tg; (void)row; (void)c0; (void)dl0;
        (void)sQT; (void)sWT; (void)sBT; (void)sAT; (void)sLT; (void)sTI; (void)sVP; (void)sEM; (void)sFLAG;
        {
            float G[4][DL], Gc[4][DL], GC[DL], x[4][DL];
            chunk_float<CK>(cur.x.g, G, tg, nv);
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int i = 0; i < DL; ++i) {
                    G[j][i] = fminf(G[j][i], 0.f);
                    Gc[j][i] = G[j][i];
                }
            chunk_cumsum<DL>(G, GC, lane);
            bool bad = false;
#pragma unroll
            for (int i = 0; i < DL; ++i) bad |= !(GC[i] >= -GDN_SPAN_MAX);
            float fq[4][DL];
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int i = 0; i < DL; ++i) fq[j][i] = fast_exp(G[j][i] - 0.5f * GC[i]);  // exp(G - m)
            if (tg == 0) {
#pragma unroll
                for (int i = 0; i < DL; ++i) sEM[dl0 + i] = fast_exp(0.5f * GC[i]);
            }
            const bool any_bad = __any(bad);
            if (lane == 0) sFLAG[wave] = any_bad ? 1 : 0;
            if (OUT) {
                chunk_float<CK>(cur.x.q, x, tg, nv);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
#pragma unroll
                    for (int i = 0; i < DL; ++i) x[j][i] *= fq[j][i];
                    lds_put_row<NS, DL>(sQT, L::ROWP, (4 * tg + j) * L::RS + dl0, x[j]);
                }
            }
            float kx[4][DL];
            chunk_float<CK>(cur.x.k, kx, tg, nv);
            // Bt = k exp(Gp - m)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int i = 0; i < DL; ++i) x[j][i] = kx[j][i] * fast_exp(G[j][i] - Gc[j][i] - 0.5f * GC[i]);
                lds_put_row<NS, DL>(sBT, L::ROWP, (4 * tg + j) * L::RS + dl0, x[j]);
            }
            // Wt = beta k exp(m - G)
            float bt[4];
            if (a.beta_kind == BETA_HEAD) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int tl = min(4 * tg + j, nv - 1);
                    bt[j] = beta_value(a, wk, h, tc + tl);
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) bt[j] = 1.f;
            }
            float bkx[4][DL];
            if (a.beta_kind == BETA_KEY) {
                if constexpr (PBK) {
                    chunk_float<CK>(cur.bk, bkx, tg, nv);
                } else {
                    Vec<float, 4> bk[4];
                    rows_load<CK>(bk, chunk_rsrc(kb, tc, true), kb, tc);
                    chunk_float<CK>(bk, bkx, tg, nv);
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int i = 0; i < DL; ++i) bkx[j][i] = bt[j];
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int i = 0; i < DL; ++i) x[j][i] = kx[j][i] * bkx[j][i] * __builtin_amdgcn_rcpf(fq[j][i]);
                lds_put_row<NS, DL>(sWT, L::ROWP, (4 * tg + j) * L::RS + dl0, x[j]);
            }
            // V rows of this wave's columns
            float vx[4][4];
            chunk_float<CK>(cur.x.v, vx, tg, nv);
#pragma unroll
            for (int j = 0; j < 4; ++j) lds_put_row<NX, 4>(sVP, L::VPP, (4 * tg + j) * L::VS + 4 * row, vx[j]);
        }
    }

    // Whether every wave of the chunk region found its decay span in range (after stage 1's barrier).
    __device__ static bool chunk_fast(const Ctx& c) {
        bool fast = true;
#pragma unroll
        for (int w = 0; w < NW; ++w) fast = fast && (c.sFLAG[w] == 0);
        return fast;
    }

    // Stage 2: tiles -> LDS; diagonal-block inverses.
    __device__ static void stage2(const Ctx& c) {
        const int lane = c.lane, wave = c.wave, r16 = c.r16, g4 = c.g4, tg = c.tg, row = c.row, c0 = c.c0,
                  dl0 = c.dl0;
        char *sQT = c.sQT, *sWT = c.sWT, *sBT = c.sBT, *sAT = c.sAT, *sLT = c.sLT, *sTI = c.sTI, *sVP = c.sVP;
        float* sEM = c.sEM;
        int* sFLAG = c.sFLAG;
        (void)lane; (void)wave; (void)r16; (void)g4; (void)tg; (void)row; (void)c0; (void)dl0;
        (void)sQT; (void)sWT; (void)sBT; (void)sAT; (void)sLT; (void)sTI; (void)sVP; (void)sEM; (void)sFLAG;
        // ---------------- stage 2: tiles -> LDS; diagonal-block inverses -------------------
        // Tile list: the ten lower tiles of A^T = Wt Qt^T (OUT) and the six strictly lower
        // off-diagonal tiles of L^T = Wt Bt^T; tile (sb, tb) holds rows s of block sb, columns t
        // of block tb.
        {
            constexpr int NT = OUT ? 16 : 6;
            for (int n = wave; wave < TW && n < NT; n += TW) {
                const bool is_a = OUT && n < 10;
                int sb, tb, idx;
                if (is_a) {
                    idx = n;
                    tile_sb_tb(idx, sb, tb);
                } else {
                    const int m = OUT ? n - 10 : n;  // off-diagonal L tiles: (0,1) (0,2) (1,2) (0,3) (1,3) (2,3)
                    tb = m >= 3 ? 3 : (m >= 1 ? 2 : 1);
                    sb = m - (tb - 1) * tb / 2;
                    idx = m;
                }
                const char* rhs = is_a ? sQT : sBT;
                f32x4 acc = zero4();
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) {
                    const Split8<NS> wf = lds_frag<NS>(sWT, L::ROWP, L::RS, 16 * sb + r16, 32 * ks, g4);
                    const Split8<NS> rf = lds_frag<NS>(rhs, L::ROWP, L::RS, 16 * tb + r16, 32 * ks, g4);
                    acc = mfma_split<NS, NS, NS>(wf, rf, acc);
                }
                if (is_a && sb == tb) {  // row = s (4*g4 + j), column = t (r16): keep s <= t
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[j] = (4 * g4 + j > r16) ? 0.f : acc[j];
                }
                const float xv[4] = {acc[0], acc[1], acc[2], acc[3]};
                lds_put_row<NS, 4>(is_a ? sAT : sLT, is_a ? L::TILEP : L::LTP, (idx * 64 + lane) * 4, xv);
            }
            // Diagonal block wave of the UT transform: T_ww = (I + L_ww)^-1 by doubling, kept as
            // D-layout pairs (X, X^T) so every product reads its operands from registers.
            if (BV && wave >= DW0 && wave < DW0 + 4) {
                // per-value beta: the diagonal block of L0 itself, fp32, for the column solves
                const int ib = wave - DW0;
                f32x4 Lm = zero4();
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) {
                    const Split8<NS> bf = lds_frag<NS>(sBT, L::ROWP, L::RS, 16 * ib + r16, 32 * ks, g4);
                    const Split8<NS> wf = lds_frag<NS>(sWT, L::ROWP, L::RS, 16 * ib + r16, 32 * ks, g4);
                    Lm = mfma_split<NS, NS, NS>(bf, wf, Lm);  // Lm[t = 4*g4+j][s = r16]
                }
                float* sL = reinterpret_cast<float*>(sTI) + ib * 256;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int t = 4 * g4 + j;
                    sL[t * 16 + 4 * ((r16 >> 2) ^ g4) + (r16 & 3)] = t > r16 ? Lm[j] : 0.f;
                }
            } else if (!BV && wave >= DW0 && wave < DW0 + 4) {
                const int ib = wave - DW0;
                f32x4 Lm = zero4(), LmT = zero4();
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) {
                    const Split8<NS> bf = lds_frag<NS>(sBT, L::ROWP, L::RS, 16 * ib + r16, 32 * ks, g4);
                    const Split8<NS> wf = lds_frag<NS>(sWT, L::ROWP, L::RS, 16 * ib + r16, 32 * ks, g4);
                    Lm = mfma_split<NS, NS, NS>(bf, wf, Lm);    // Lm[t = 4*g4+j][s = r16]
                    LmT = mfma_split<NS, NS, NS>(wf, bf, LmT);  // LmT[s = 4*g4+j][t = r16]
                }
                f32x4 P, PT, Tm, TT;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int rr = 4 * g4 + j;
                    P[j] = rr > r16 ? -Lm[j] : 0.f;    // M = -L (strictly lower: t > s)
                    PT[j] = r16 > rr ? -LmT[j] : 0.f;  // M^T
                    Tm[j] = P[j] + (rr == r16 ? 1.f : 0.f);
                    TT[j] = PT[j] + (rr == r16 ? 1.f : 0.f);
                }
#pragma unroll
                for (int step = 0; step < 3; ++step) {
                    // A-layout of X = D-layout registers of X^T
                    const Split8<NS> pA = split_k16<NS>(PT), pB = split_k16<NS>(P);
                    const Split8<NS> ptA = split_k16<NS>(P), ptB = split_k16<NS>(PT);
                    const f32x4 Pn = mfma_split<NS, NS, NS>(pA, pB, zero4());     // P P
                    const f32x4 PTn = mfma_split<NS, NS, NS>(ptA, ptB, zero4());  // P^T P^T
                    const Split8<NS> tA = split_k16<NS>(Tm), tB = split_k16<NS>(Tm);
                    const Split8<NS> pnA = split_k16<NS>(PTn), ptnB = split_k16<NS>(PTn);
                    const f32x4 TTn = mfma_split<NS, NS, NS>(tA, ptnB, TT);  // T^T + T^T (P^T)^2
                    const f32x4 Tn = mfma_split<NS, NS, NS>(pnA, tB, Tm);    // T + P^2 T
                    Tm = Tn;
                    TT = TTn;
                    P = Pn;
                    PT = PTn;
                }
                const float xv[4] = {TT[0], TT[1], TT[2], TT[3]};  // A-layout of T_ww
                lds_put_row<NS, 4>(sTI, L::DIAGP, (ib * 64 + lane) * 4, xv);
            }
        }
    }

    // Stage 3 on one state (K3 runs it on S with V; K1 on S with V = 0 and on SN with V): residuals,
    // UT solve, outputs, state update.  mid() runs between the solve and the rest.
    template <bool WV, typename LateHook, typename Mid>
    __device__ static void pass(const PrefillParams& a, const Work& wk, int64_t h, int64_t tc, int nv,
                                f32x4 (&St)[NDB], const Ctx& c, const f32x4* bv_in, LateHook&& after_inputs,
                                Mid&& mid) {
        const int lane = c.lane, wave = c.wave, r16 = c.r16, g4 = c.g4, tg = c.tg, row = c.row, c0 = c.c0,
                  dl0 = c.dl0;
        char *sQT = c.sQT, *sWT = c.sWT, *sBT = c.sBT, *sAT = c.sAT, *sLT = c.sLT, *sTI = c.sTI, *sVP = c.sVP;
        float* sEM = c.sEM;
        int* sFLAG = c.sFLAG;
        (void)lane; (void)wave; (void)r16; (void)g4; (void)tg; (void)row; (void)c0; (void)dl0;
        (void)sQT; (void)sWT; (void)sBT; (void)sAT; (void)sLT; (void)sTI; (void)sVP; (void)sEM; (void)sFLAG;
        f32x4 Sp[NDB];
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            const f32x4 em = *reinterpret_cast<const f32x4*>(sEM + 16 * db + 4 * g4);
#pragma unroll
            for (int i = 0; i < 4; ++i) Sp[db][i] = St[db][i] * em[i];
        }
        f32x4 bv[4];  // BV: beta of rows 16i + 4*g4 + k, column c0 + r16 (rows past nv: the last row's)
        if constexpr (BV) {
            if (bv_in) {
#pragma unroll
                for (int i = 0; i < 4; ++i) bv[i] = bv_in[i];
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        bv[i][k] = tok_row<float>(a.kb, wk, tc + min(16 * i + 4 * g4 + k, nv - 1), h, c0)[r16];
            }
        }
        Split8<NS> sf[NKS];  // S' with K = key dims (A-operand of S'^T, B-operand of S')
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) sf[ks] = split_k32<NS>(Sp[2 * ks], Sp[2 * ks + 1]);
        // R_i = V_i - Bt_i S'  (D layout: rows t = 16i + 4*g4 + k, column c0 + r16)
        f32x4 R[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f32x4 p = zero4();
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
                const Split8<NS> bf = lds_frag<NS>(sBT, L::ROWP, L::RS, 16 * i + r16, 32 * ks, g4);
                p = mfma_split<NS, NS, NS>(bf, sf[ks], p);
            }
            f32x4 vv = zero4();
            if constexpr (WV) {
                const int off = (16 * i + 4 * g4 + (r16 >> 2)) * L::VS + 4 * (r16 & 3);
#pragma unroll
                for (int pl = 0; pl < NX; ++pl) {
                    const bf16x4 t4 = lds_read_tr(reinterpret_cast<const __bf16*>(sVP + pl * L::VPP) + off);
#pragma unroll
                    for (int k = 0; k < 4; ++k) vv[k] += (float)t4[k];
                }
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) R[i][k] = vv[k] - p[k];
        }
        // O^T from the carried state first (Qt S'), so that S' in split form is dead before
        // the UT solve
        f32x4 Ot[4];
        if constexpr (OUT) {
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) {
                f32x4 o = zero4();
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) {
                    const Split8<NS> qf = lds_frag<NS>(sQT, L::ROWP, L::RS, 16 * tb + r16, 32 * ks, g4);
                    o = mfma_split<NS, NS, NS>(sf[ks], qf, o);
                }
                Ot[tb] = o;
            }
        }
        // U_i = T_ii (R_i - sum_{j<i} L_ij U_j)
        f32x4 U[4];
        Split8<NS> us[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f32x4 X = R[i];
            if (i >= 1) {
                f32x4 p = zero4();
                if (i >= 2) {  // blocks 0 and 1 together (K = 32)
                    const Split8<NS> lf = tile_frag<NS>(sLT, L::LTP, lt_index(0, i), lt_index(1, i), true, lane);
                    p = mfma_split<NS, NS, NS>(lf, split_k32<NS>(U[0], U[1]), p);
                    if (i == 3) {
                        const Split8<NS> lf2 = tile_frag<NS>(sLT, L::LTP, lt_index(2, 3), 0, false, lane);
                        p = mfma_split<NS, NS, NS>(lf2, us[2], p);
                    }
                } else {
                    const Split8<NS> lf = tile_frag<NS>(sLT, L::LTP, lt_index(0, 1), 0, false, lane);
                    p = mfma_split<NS, NS, NS>(lf, us[0], p);
                }
#pragma unroll
                for (int k = 0; k < 4; ++k) X[k] -= p[k];
            }
            if constexpr (BV) {
                U[i] = col_solve(X, bv[i], reinterpret_cast<const float*>(sTI) + i * 256, g4, r16);
            } else {
                const Split8<NS> tf = tile_frag<NS>(sTI, L::DIAGP, i, 0, false, lane);
                U[i] = mfma_split<NS, NS, NS>(tf, split_k16<NS>(X), zero4());
            }
            us[i] = split_k16<NS>(U[i]);
        }
        mid();  // the two-role kernel's barrier between the solve and the rest
        // U with K = tokens 32*k2 + pi(g4, j): A-operand of U^T, B-operand of U
        Split8<NS> uf[2];
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) uf[k2] = split_k32<NS>(U[2 * k2], U[2 * k2 + 1]);

        if constexpr (OUT) {
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) {
                f32x4 o = Ot[tb];
#pragma unroll
                for (int k2 = 0; k2 < 2; ++k2) {
                    if (2 * k2 > tb) continue;
                    const bool has_hi = 2 * k2 + 1 <= tb;
                    const Split8<NS> af = tile_frag<NS>(sAT, L::TILEP, tile_index(2 * k2, tb),
                                                        has_hi ? tile_index(2 * k2 + 1, tb) : 0, has_hi, lane);
                    o = mfma_split<NS, NS, NS>(uf[k2], af, o);
                }
                Ot[tb] = o;
            }
            // lane (g4, r16) holds O[token 16*tb + r16][columns c0 + 4*g4 + 0..3]; stage
            // through this wave's V planes (read above) and store quad-coalesced rows
            float* sO = reinterpret_cast<float*>(sVP);
            const int es = dt_size(a.o_dt);
            const int64_t ost = a.o_st * es;
            char* obase = reinterpret_cast<char*>(a.o) +
                          uniform_i64((wk.b * a.o_sb + (wk.row0 + tc) * a.o_st + h * a.o_sh + c0) * es);
            const int q = lane & 3, tq = (lane >> 4) + 4 * ((lane >> 2) & 3);
            const int32_t olane = (int32_t)(tq * ost) + 4 * q * es;
            const OutRsrc orr = out_rsrc(obase, ost, es, nv, a.o_dt == DT_F32);
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) {
                *reinterpret_cast<f32x4*>(sO + r16 * L::OS + 4 * g4) = Ot[tb];
                const f32x4 xo = *reinterpret_cast<const f32x4*>(sO + tq * L::OS + 4 * q);
                out_store4(orr, (int32_t)(16 * tb * ost) + olane, a.o_dt, xo);
            }
        }
        if constexpr (LATE_LOAD_OUT) after_inputs();
        // S <- e^m (S' + Wt^T U)
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            f32x4 acc = Sp[db];
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2) {
                const Split8<NS> wf = lds_frag_tr<NS>(sWT, L::ROWP, L::RS, 32 * k2, 16 * db, g4, r16);
                acc = mfma_split<NS, NS, NS>(wf, uf[k2], acc);
            }
            const f32x4 em = *reinterpret_cast<const f32x4*>(sEM + 16 * db + 4 * g4);
#pragma unroll
            for (int i = 0; i < 4; ++i) St[db][i] = em[i] * acc[i];
        }
    }

    // bv_in (BV): this chunk's beta in stage 3's layout (rows 16i + 4*g4 + k, column c0 + r16),
    // loaded a chunk ahead by the caller; null: stage 3 loads it.
    template <typename Hook>
    __device__ static void run(const PrefillParams& a, const Work& wk, int64_t h, int64_t tc, int nv,
                               const GChunkIn<TIn, TG, PBK>& cur, const TokAddr& kb, f32x4 (&S)[NDB],
                               f32x4 (&SN)[NDB], bool skip_m, char* smem, const f32x4* bv_in, Hook&& after_inputs) {
        const Ctx c = ctx(smem, wave_id());
        // Issue priority: stage 1 at the base level, stage 2 and the passes that carry the state one
        // level up, so of the workgroups on a CU the one further along issues first (config 3 with
        // per-key-dim gates 0.166 -> 0.159 ms, same-box A/B).
        __builtin_amdgcn_s_setprio(0);
        stage1(a, wk, h, tc, nv, cur, kb, c);
        if constexpr (!LATE_LOAD && !LATE_LOAD_OUT) after_inputs();
        __syncthreads();
        __builtin_amdgcn_s_setprio(1);
        if (!chunk_fast(c)) {
            if (!skip_m) gdn_tokenwise<TIn, TG, OUT, BV>(a, wk, h, c.c0, tc, nv, c.g4, c.r16, OUT, S);
            if (!OUT) gdn_tokenwise<TIn, TG, false, BV>(a, wk, h, c.c0, tc, nv, c.g4, c.r16, true, SN);
            if constexpr (LATE_LOAD || LATE_LOAD_OUT) after_inputs();
            __syncthreads();
            return;
        }
        stage2(c);
        __syncthreads();
        auto nomid = [] {};
        if constexpr (OUT) {
            pass<true>(a, wk, h, tc, nv, S, c, bv_in, after_inputs, nomid);
        } else {
            if (!skip_m) pass<false>(a, wk, h, tc, nv, S, c, bv_in, after_inputs, nomid);
            if constexpr (LATE_LOAD) after_inputs();
            __builtin_amdgcn_sched_barrier(0);  // one pass at a time: their temporaries never overlap
            pass<true>(a, wk, h, tc, nv, SN, c, bv_in, after_inputs, nomid);
        }
        __syncthreads();  // the next chunk rewrites LDS
    }
};

template <typename TIn, typename TG, bool OUT, bool CK, int D, bool BV>
__device__ void gdn_walk(const PrefillParams& a, const Work& wk, int64_t h, f32x4 (&S)[D / 16],
                         f32x4 (&SN)[D / 16], bool skip_m, char* smem) {
    using St = GdnStep<TIn, TG, OUT, CK, D, BV>;
    const int lane = threadIdx.x & 63, wave = wave_id(), tg = lane >> 2, row = lane & 3;
    const ChunkAddr ad = chunk_addr<OUT, TIn, TG>(a, wk, h, tg, wave * 16 + 4 * row, wave * 16 + 4 * row);
    const bool key_beta = a.beta_kind == BETA_KEY;
    TokAddr kb{};
    if (key_beta) kb = tok_addr<float>(a.kb, wk, h, tg, wave * 16 + 4 * row);
    const int64_t nch = (wk.t_end - wk.t_begin + CHUNK - 1) / CHUNK;
    auto chunk_nv = [&](int64_t c) {
        const int64_t r = wk.t_end - (wk.t_begin + c * CHUNK);
        return (int)(r < CHUNK ? r : CHUNK);
    };
    auto tok = [&](int64_t c) { return wk.t_begin + c * CHUNK; };
    GChunkIn<TIn, TG, St::PBK> A;
    gchunk_load<OUT, CK>(A, ad, kb, key_beta, tok(0), true);
    // BV outputs at D = 64: the chunk's beta in stage 3's layout, loaded with the chunk's other
    // inputs (a chunk ahead) rather than inside stage 3, whose dependent chain is the walk's
    // critical path (1.154 -> 1.113 ms at config 3's shape; at D = 128 the 16 extra registers
    // spill: 1.96 -> 2.11 ms, so stage 3 loads it there)
    constexpr bool BVP = OUT && BV && D == 64;
    f32x4 bvn[BVP ? 4 : 1], bvc[BVP ? 4 : 1];
    const int g4 = lane >> 4, r16 = lane & 15, c0 = wave * 16;
    auto load_bv = [&](int64_t c) {
        if constexpr (BVP) {
            const int nvc = chunk_nv(c);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    bvn[i][k] = tok_row<float>(a.kb, wk, tok(c) + min(16 * i + 4 * g4 + k, nvc - 1), h, c0)[r16];
        }
    };
    load_bv(0);
    for (int64_t c = 0; c < nch; ++c) {
        if constexpr (BVP) {
#pragma unroll
            for (int i = 0; i < 4; ++i) bvc[i] = bvn[i];
        }
        St::run(a, wk, h, tok(c), chunk_nv(c), A, kb, S, SN, skip_m, smem, BVP ? bvc : nullptr, [&] {
            gchunk_load<OUT, CK>(A, ad, kb, key_beta, tok(c + 1), c + 1 < nch);
            if (c + 1 < nch) load_bv(c + 1);
        });
    }
}

// Waves per SIMD the chunk kernels ask for: two at D = 64 where the LDS of two workgroups fits
// (K1 at fp32 I/O keeps one for registers), two at D = 128 (one workgroup of eight waves per CU).
template <typename TIn, bool OUT, int D>
constexpr int gdn_min_waves() {
    if (D == 128) return 2;
    if (!OUT) return Prec<TIn>::F32 ? 1 : 2;
    return 2 * GLay<TIn, true, D>::BYTES <= 160 * 1024 ? 2 : 1;
}

// K1: the segment map driven from I with V = 0 (-> M_p, state M) and from 0 with the real V
// (-> N_p, state N) in one chunk walk.  A sequence's first segment without an initial state
// carries in S_in = 0, so its M is left at I (the scan's product with 0 stays 0) and only N runs.
template <typename TIn, typename TG, bool CK, int D, bool BV>
__global__ __launch_bounds__(4 * D, (gdn_min_waves<TIn, false, D>())) void gdn_seg_mn_kernel(PrefillParams a) {
    using L = GLay<TIn, false, D>;
    constexpr int NDB = D / 16;
    __shared__ __attribute__((aligned(16))) char smem[L::BYTES];
    const int64_t w = blockIdx.x, h = blockIdx.y;
    Work wk;
    if (!find_work(a, w, wk)) return;
    f32x4 M[NDB], N[NDB];
    init_seg_map(M, N);
    gdn_walk<TIn, TG, false, CK, D, BV>(a, wk, h, M, N, wk.p == 0 && a.s0 == nullptr, smem);
    store_seg_map<Prec<TIn>::NS>(a, w, h, M, N);
}

// K3: outputs of one segment from S_in[p] (in the N slot after the scan).  At D = 64 two
// workgroups per CU where two fit in LDS (bf16 I/O); fp16 and fp32 I/O hold larger planes and run
// one.  At D = 128 (16-bit I/O) one workgroup of eight waves per CU.
// gdn_whole (beta per value column, BV): each value column then has its own segment map, so there
// is one segment per sequence, walked from s0 (or zero), and the final state is written here;
// with B * H workgroups in all, each may take a whole SIMD's registers.
template <typename TIn, typename TG, bool CK, int D, bool BV>
__global__ __launch_bounds__(4 * D, (BV ? 1 : gdn_min_waves<TIn, true, D>())) void gdn_seg_out_kernel(PrefillParams a) {
    using L = GLay<TIn, true, D>;
    constexpr int NDB = D / 16;
    __shared__ __attribute__((aligned(16))) char smem[L::BYTES];
    const int64_t w = blockIdx.x, h = blockIdx.y;
    Work wk;
    if (!find_work(a, w, wk)) return;
    f32x4 S[NDB];
    const int lane = threadIdx.x & 63, c = wave_id() * 16 + (lane & 15), g4 = lane >> 4;
    const int64_t sb = (wk.seq * a.H + h) * (int64_t)D * D;  // [seq, h] of s0 / seq_final
    if (BV && a.gdn_whole) {
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) S[db][i] = a.s0 ? a.s0[sb + (16 * db + 4 * g4 + i) * D + c] : 0.f;
    } else {
        load_seg_state(a, w, h, S);
    }
    gdn_walk<TIn, TG, true, CK, D, BV>(a, wk, h, S, S, false, smem);
    if (BV && a.gdn_whole && a.seq_final) {
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) a.seq_final[sb + (16 * db + 4 * g4 + i) * D + c] = S[db][i];
    }
}

// Beta per value column at D = 64 with bf16 I/O: the whole-sequence walk of gdn_seg_out_kernel in
// two roles over two chunk regions of LDS.  The walk's critical path is stage 3 (the residuals,
// the column solves and the state update depend on the state), while stages 1 and 2 (factors,
// split operands, tiles, diagonal blocks) depend only on the chunk's inputs.  Waves 0-3 run
// stages 1 and 2 of chunk i + 1 in region (i + 1) & 1 while waves 4-7 run stage 3 of chunk i from
// region i & 1; two workgroup barriers per chunk: after stage 1 of the front waves (the back
// waves' barrier sits between their solve and the rest of stage 3), and at the end of the chunk.
// Wave w of either role owns value columns 16w .. 16w + 15, so the back waves read the V rows the
// front waves of the same index staged.
template <typename TG, bool CK>
__global__ __launch_bounds__(512, 1) void gdn_bv_pipe_kernel(PrefillParams a) {
    using TIn = __bf16;
    constexpr int D = 64;
    using St = GdnStep<TIn, TG, true, CK, D, true>;
    using L = GLay<TIn, true, D>;
    constexpr int RB = (L::BYTES + 255) / 256 * 256;
    static_assert(RB + L::BYTES <= 160 * 1024, "two chunk regions fit in LDS");
    __shared__ __attribute__((aligned(256))) char smem[RB + L::BYTES];
    const int64_t h = blockIdx.y;
    Work wk;
    if (!find_work(a, blockIdx.x, wk)) return;
    const int wave8 = wave_id(), wave = wave8 & 3;
    const bool front = wave8 < 4;
    // The stage-3 waves carry the walk's serial chain; each SIMD holds one wave of each role, so
    // they issue one priority level up and the stage-1/2 waves fill their gaps (config-3 shape
    // 0.816 -> 0.770 ms, same-box A/B).
    if (!front) __builtin_amdgcn_s_setprio(1);
    const int lane = threadIdx.x & 63, g4 = lane >> 4, r16 = lane & 15, tg = lane >> 2, row = lane & 3;
    const int c0 = wave * 16;
    const int64_t nch = (wk.t_end - wk.t_begin + CHUNK - 1) / CHUNK;
    auto chunk_nv = [&](int64_t c) {
        const int64_t r = wk.t_end - (wk.t_begin + c * CHUNK);
        return (int)(r < CHUNK ? r : CHUNK);
    };
    auto tok = [&](int64_t c) { return wk.t_begin + c * CHUNK; };
    auto region = [&](int64_t c) { return smem + (c & 1) * RB; };
    auto nohook = [] {};

    // front waves: the chunk inputs, a chunk ahead
    const ChunkAddr ad = chunk_addr<true, TIn, TG>(a, wk, h, tg, c0 + 4 * row, c0 + 4 * row);
    const TokAddr kb{};
    GChunkIn<TIn, TG, St::PBK> A;
    // back waves: the state (rows 16 db + 4 g4 + i, column c0 + r16) and beta a chunk ahead
    f32x4 S[4], bvn[4], bvc[4];
    const int64_t sb = (wk.seq * a.H + h) * (int64_t)D * D;
    auto load_bv = [&](int64_t c) {
        const int nvc = chunk_nv(c);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int k = 0; k < 4; ++k)
                bvn[i][k] = tok_row<float>(a.kb, wk, tok(c) + min(16 * i + 4 * g4 + k, nvc - 1), h, c0)[r16];
    };
    if (front) {
        gchunk_load<true, CK>(A, ad, kb, false, tok(0), nch > 0);
    } else {
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) S[db][i] = a.s0 ? a.s0[sb + (16 * db + 4 * g4 + i) * D + c0 + r16] : 0.f;
        if (nch > 0) load_bv(0);
    }
    // chunk 0's stages 1 and 2
    if (front && nch > 0) {
        St::stage1(a, wk, h, tok(0), chunk_nv(0), A, kb, St::ctx(region(0), wave));
        gchunk_load<true, CK>(A, ad, kb, false, tok(1), nch > 1);
    }
    __syncthreads();
    if (front && nch > 0) {
        const auto c = St::ctx(region(0), wave);
        if (St::chunk_fast(c)) St::stage2(c);
    }
    __syncthreads();
    for (int64_t i = 0; i < nch; ++i) {
        if (front) {
            if (i + 1 < nch) {
                St::stage1(a, wk, h, tok(i + 1), chunk_nv(i + 1), A, kb, St::ctx(region(i + 1), wave));
                gchunk_load<true, CK>(A, ad, kb, false, tok(i + 2), i + 2 < nch);
            }
            __syncthreads();
            if (i + 1 < nch) {
                const auto c = St::ctx(region(i + 1), wave);
                if (St::chunk_fast(c)) St::stage2(c);
            }
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) bvc[k] = bvn[k];
            if (i + 1 < nch) load_bv(i + 1);
            const auto c = St::ctx(region(i), wave);
            if (St::chunk_fast(c)) {
                St::template pass<true>(a, wk, h, tok(i), chunk_nv(i), S, c, bvc, nohook, [] { __syncthreads(); });
            } else {  // decay span out of the factored range: token by token from the state
                gdn_tokenwise<TIn, TG, true, true>(a, wk, h, c0, tok(i), chunk_nv(i), g4, r16, true, S);
                __syncthreads();
            }
        }
        __syncthreads();  // the next chunk rewrites the region this one read
    }
    if (!front && a.seq_final) {
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) a.seq_final[sb + (16 * db + 4 * g4 + i) * D + c0 + r16] = S[db][i];
    }
}

// K2: one workgroup per (sequence, head, 16 state columns), one wave per 16-row tile t of that
// column strip (D / 16 waves): S_in[p] = carry (written in place of N_p), then S <- M_p S + N_p on
// MFMA.  Wave t holds rows 16t + 4*g4 + i of the strip in D layout; each step it writes its tile,
// split into NS bf16 parts, as one half of a B-operand fragment in LDS (K step t >> 1, slots
// (t & 1) * 4 + i), and after one barrier every wave reads the strip's D / 32 K=32 fragments and
// forms its new tile with NS-part products.  M_p arrives pre-split in NS bf16 planes, read straight
// into A-operand layout (row 16t + r16, K slots 32kk + pi(g4, j)).  The M/N loads of a segment do
// not depend on the carry: a ring of register sets keeps them two segments ahead.  Two LDS buffers
// alternate, so a step's writes never meet the previous step's reads.
// Placement: workgroups are dispatched round-robin over the XCDs, each with its own L2, and every
// strip of a (sequence, head) reads that pair's whole segment maps, so a 1-D grid puts the D / 16
// strips of a pair on one XCD (workgroup b runs on XCD b % SCAN_XCDS; its slot b / SCAN_XCDS
// there holds strip slot % (D / 16) of pair (slot / (D / 16)) * SCAN_XCDS + b % SCAN_XCDS).
constexpr int SCAN_XCDS = 8;

template <int NS, int D>
__global__ __launch_bounds__(4 * D) void gdn_seg_scan_kernel(PrefillParams a, float* s_final) {
    constexpr int NKS = D / 32, NDB = D / 16, DD = D * D;
    __shared__ __attribute__((aligned(16))) char sbuf[2][NKS][NS][64 * 16];
    const int64_t slot = blockIdx.x / SCAN_XCDS;
    const int64_t pair = (slot / NDB) * SCAN_XCDS + blockIdx.x % SCAN_XCDS;
    if (pair >= a.n_seqs * a.H) return;  // the grid's padding to whole rounds of the XCDs
    const int64_t seq = pair / a.H, h = pair % a.H;
    const int strip = (int)(slot % NDB), cb = strip * 16;
    const int lane = threadIdx.x & 63, t = wave_id(), r16 = lane & 15, g4 = lane >> 4;
    int64_t p0, np;
    if (a.varlen) {
        p0 = a.seg_off[seq];
        np = (int64_t)a.seg_off[seq + 1] - p0;
    } else {
        const int64_t nch = (a.T + CHUNK - 1) / CHUNK;
        p0 = seq * a.nseg_dense;
        np = a.nseg_dense < nch ? a.nseg_dense : nch;
        if (a.T == 0) np = 0;
    }
    auto d_off = [&](int i) { return (16 * t + 4 * g4 + i) * D + cb + r16; };  // D-layout element
    f32x4 S;
#pragma unroll
    for (int i = 0; i < 4; ++i) S[i] = a.s0 ? a.s0[(seq * a.H + h) * DD + d_off(i)] : 0.f;
    struct MN {
        Split8<NS> m[NKS];  // [K step] of row tile t
        f32x4 n;
    };
    // Every path issues the same loads and stores (past the end: the last segment's rows again,
    // and the store goes to a spare slot), so the wait counts leave the sets in flight.
    float* spare = a.ws_spare + (seq * a.H + h) * DD;
    auto fetch = [&](MN& x, int64_t p) {
        const int64_t w = p0 + (p < np ? p : np - 1);
        const __bf16* mp = reinterpret_cast<const __bf16*>(a.ws_m) + (w * a.H + h) * mslot<D>();
        const float* np_ = a.ws_state + (w * a.H + h) * DD;
#pragma unroll
        for (int kk = 0; kk < NKS; ++kk)
#pragma unroll
            for (int pl = 0; pl < NS; ++pl)
                x.m[kk].p[pl] = *reinterpret_cast<const bf16x8*>(mp + ((pl * NDB + t) * NKS + kk) * 512 + 8 * lane);
        x.n = *reinterpret_cast<const f32x4*>(np_ + dstate_off<NDB>(strip, t, lane));
    };
    auto step = [&](const MN& x, int64_t p) {
        const bool real = p < np;
        float* dst = real ? a.ws_state + ((p0 + p) * a.H + h) * DD : spare;
        *reinterpret_cast<f32x4*>(dst + dstate_off<NDB>(strip, t, lane)) = S;  // S_in[p]
        // this tile as half (t & 1) of the strip's K-step (t >> 1) fragment
        const int buf = (int)(p & 1);
        {
            float r[4] = {S[0], S[1], S[2], S[3]};
            uint32_t w[NS][2];
            split_pairs<NS, 2>(r, w);
#pragma unroll
            for (int pl = 0; pl < NS; ++pl)
                *reinterpret_cast<uint2*>(&sbuf[buf][t >> 1][pl][lane * 16 + (t & 1) * 8]) = uint2{w[pl][0], w[pl][1]};
        }
        __syncthreads();
        f32x4 acc = x.n;
#pragma unroll
        for (int kk = 0; kk < NKS; ++kk) {
            Split8<NS> sb;
#pragma unroll
            for (int pl = 0; pl < NS; ++pl) sb.p[pl] = *reinterpret_cast<const bf16x8*>(&sbuf[buf][kk][pl][lane * 16]);
            acc = mfma_split<NS, NS, NS>(x.m[kk], sb, acc);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) S[i] = real ? acc[i] : S[i];
    };
    if (np > 0) {
        constexpr int RING = 3;  // loads run RING - 1 segments ahead of the carry
        MN x[RING];
#pragma unroll
        for (int r = 0; r < RING - 1; ++r) fetch(x[r], r);
        const int64_t nit = (np + RING - 1) / RING;
        for (int64_t it = 0; it < nit; ++it) {
#pragma unroll
            for (int r = 0; r < RING; ++r) {
                const int64_t p = RING * it + r;
                fetch(x[(r + RING - 1) % RING], p + RING - 1);
                step(x[r], p);
            }
        }
    }
    if (s_final) {
#pragma unroll
        for (int i = 0; i < 4; ++i) s_final[(seq * a.H + h) * DD + d_off(i)] = S[i];
    }
}

// ---------------------------------------------------------------------------------------
// Host launchers.
// ---------------------------------------------------------------------------------------
template <typename TIn, typename TG, bool CK, int D, bool BV>
static hipError_t launch_gdn_bv(const PrefillParams& a, int64_t n_work, int which, hipStream_t stream) {
    if (which == 0) {
        hipLaunchKernelGGL((gdn_seg_mn_kernel<TIn, TG, CK, D, BV>), dim3((unsigned)n_work, (unsigned)a.H), dim3(4 * D),
                           0, stream, a);
    } else if constexpr (BV && D == 64 && std::is_same<TIn, __bf16>::value) {
        if (a.gdn_whole)
            hipLaunchKernelGGL((gdn_bv_pipe_kernel<TG, CK>), dim3((unsigned)n_work, (unsigned)a.H), dim3(512), 0, stream, a);
        else
            hipLaunchKernelGGL((gdn_seg_out_kernel<TIn, TG, CK, D, BV>), dim3((unsigned)n_work, (unsigned)a.H),
                               dim3(4 * D), 0, stream, a);
    } else {
        hipLaunchKernelGGL((gdn_seg_out_kernel<TIn, TG, CK, D, BV>), dim3((unsigned)n_work, (unsigned)a.H), dim3(4 * D),
                           0, stream, a);
    }
    return hipGetLastError();
}

// Per-value-column beta runs its own instances (the column solves), so the other beta kinds keep
// their register allocation.
template <typename TIn, typename TG, bool CK, int D>
static hipError_t launch_gdn_ck(const PrefillParams& a, int64_t n_work, int which, hipStream_t stream) {
    if (a.beta_kind == BETA_VALUE) return launch_gdn_bv<TIn, TG, CK, D, true>(a, n_work, which, stream);
    return launch_gdn_bv<TIn, TG, CK, D, false>(a, n_work, which, stream);
}

// Unchecked row addressing only when T is a whole number of four-row groups.  Head dim 128 takes
// 16-bit I/O only (fp32 planes do not fit in LDS).
template <typename TIn, typename TG>
static hipError_t launch_gdn_t(const PrefillParams& a, int64_t n_work, int which, hipStream_t stream) {
    if (a.Dk == 128) {
        if constexpr (Prec<TIn>::F32) {
            return hipErrorInvalidValue;
        } else {
            if (a.T % 4 == 0) return launch_gdn_ck<TIn, TG, false, 128>(a, n_work, which, stream);
            return launch_gdn_ck<TIn, TG, true, 128>(a, n_work, which, stream);
        }
    }
    if (a.T % 4 == 0) return launch_gdn_ck<TIn, TG, false, 64>(a, n_work, which, stream);
    return launch_gdn_ck<TIn, TG, true, 64>(a, n_work, which, stream);
}

static hipError_t launch_gdn(const PrefillParams& a, int64_t n_work, int io_dt, int which, hipStream_t stream) {
    const bool g32 = a.g_dt == DT_F32;
    if (io_dt == DT_BF16) {
        if (g32) return launch_gdn_t<__bf16, float>(a, n_work, which, stream);
        if (a.g_dt == DT_BF16) return launch_gdn_t<__bf16, __bf16>(a, n_work, which, stream);
    } else if (io_dt == DT_F16) {
        if (g32) return launch_gdn_t<_Float16, float>(a, n_work, which, stream);
        if (a.g_dt == DT_F16) return launch_gdn_t<_Float16, _Float16>(a, n_work, which, stream);
    } else if (io_dt == DT_F32 && g32) {
        return launch_gdn_t<float, float>(a, n_work, which, stream);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_gdn_seg_mn(const PrefillParams& a, int64_t n_work, int io_dt, hipStream_t stream) {
    return launch_gdn(a, n_work, io_dt, 0, stream);
}

hipError_t launch_gdn_seg_out(const PrefillParams& a, int64_t n_work, int io_dt, hipStream_t stream) {
    return launch_gdn(a, n_work, io_dt, 1, stream);
}

hipError_t launch_gdn_seg_scan(const PrefillParams& a, float* s_final, int io_dt, hipStream_t stream) {
    const int D = a.Dk;
    const int64_t pairs = a.n_seqs * a.H;
    const dim3 grid((unsigned)((pairs + SCAN_XCDS - 1) / SCAN_XCDS * SCAN_XCDS * (D / 16)));
    if (D == 128) {
        if (io_dt == DT_F32) return hipErrorInvalidValue;
        hipLaunchKernelGGL((gdn_seg_scan_kernel<2, 128>), grid, dim3(4 * D), 0, stream, a, s_final);
    } else if (io_dt == DT_F32) {
        hipLaunchKernelGGL((gdn_seg_scan_kernel<3, 64>), grid, dim3(4 * D), 0, stream, a, s_final);
    } else {
        hipLaunchKernelGGL((gdn_seg_scan_kernel<2, 64>), grid, dim3(4 * D), 0, stream, a, s_final);
    }
    return hipGetLastError();
}

// Resident output-kernel workgroups per CU for I/O dtype io_dt and head dim D, on the instance
// that runs (ck: checked row addressing, launched unless T % 4 == 0; the gate dtype does not change
// the kernel's LDS or register use).
template <int D>
static const void* gdn_out_kernel_ptr(int io_dt, bool ck) {
    if (io_dt == DT_F16)
        return ck ? reinterpret_cast<const void*>(gdn_seg_out_kernel<_Float16, _Float16, true, D, false>)
                  : reinterpret_cast<const void*>(gdn_seg_out_kernel<_Float16, _Float16, false, D, false>);
    if constexpr (D == 64) {
        if (io_dt == DT_F32)
            return ck ? reinterpret_cast<const void*>(gdn_seg_out_kernel<float, float, true, D, false>)
                      : reinterpret_cast<const void*>(gdn_seg_out_kernel<float, float, false, D, false>);
    }
    return ck ? reinterpret_cast<const void*>(gdn_seg_out_kernel<__bf16, __bf16, true, D, false>)
              : reinterpret_cast<const void*>(gdn_seg_out_kernel<__bf16, __bf16, false, D, false>);
}

int gdn_seg_out_blocks_per_cu(int io_dt, bool ck, int D) {
    const void* k = D == 128 ? gdn_out_kernel_ptr<128>(io_dt, ck) : gdn_out_kernel_ptr<64>(io_dt, ck);
    int nb = 0;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k, 4 * D, 0);
    return (e == hipSuccess && nb > 0) ? nb : 1;
}

}  // namespace triune
