// gdn_scalar.hip -- chunked Gated DeltaNet prefill for a gate that is one value per (token, head).
//
// Recurrence (reference: triune/kernels/fast_gla.py:781-836 fast_recurrent_gated_deltanet,
// :383-477 the Triton per-token kernel, which loads g with its own head-dim stride, so a gate
// broadcast over the head dim -- the scalar-decay form -- reaches it as a stride-0 view):
//   u_t = v_t - S_{t-1}^T k_t ,  S_t = a_t S_{t-1} + beta_t k_t u_t^T ,  o_t = S_t^T q_t
// with one decay a_t = exp(min(g_t, 0)) for every key dim.
//
// Chunk form (C = 64 tokens; gam_t = sum_{s<=t} min(g_s, 0), gamp_t = gam_{t-1}, Gam = gam_63;
// S0 the state at the chunk start):
//   L[t][s] = beta_s e^{gamp_t - gam_s} (k_t . k_s)   (s < t)
//   A[t][s] = beta_s e^{gam_t - gam_s} (q_t . k_s)     (s <= t)
//   U   = (I + L)^{-1} (V - diag(e^{gamp}) K S0)
//   O   = diag(e^{gam}) Q S0 + A U ,   S_C = e^{Gam} S0 + K^T diag(beta e^{Gam - gam}) U
// Every exponent is a sum of clamped gates over a token range, so every factor lies in [0, 1]:
// q, k and v enter the MFMA products as loaded (one bf16 part for bf16 I/O, two for fp16, three
// for fp32), the decays scale the 16x16 product tiles afterwards, and only the state, the tiles
// and U are split into bf16 parts.  (I + L)^{-1} is applied block-wise on 16-token blocks,
// U_i = T_ii (R_i - sum_{j<i} L_ij U_j); each T_ii comes from an fp32 back substitution on
// T_ii^T = (I + L_ii^T)^{-1}, one wave per block.  Chunks whose total log-decay exceeds SPAN_MAX
// (or is not finite) run token by token: the exponent differences come from prefix sums, whose
// rounding grows with the chunk total.
// The segment decomposition is the one of gdn_chunk.hip and shares its workspace layout and scan:
//   K1 gdn_sg_seg_mn  : per (segment, head) the segment map from [I | 0] with V = 0 (-> M_p) and
//                       from 0 with the real V (-> N_p) in one chunk walk
//   K2 gdn_seg_scan   : the carry S_in[p] (gdn_chunk.hip)
//   K3 gdn_sg_seg_out : per (segment, head) the chunk walk from S_in[p], writing o
#include "gdn_common.h"

namespace triune {

template <typename TIn, bool OUT>
struct SLay {
    using P = Prec<TIn>;
    static constexpr int NX = P::NX, NS = P::NS;
    static constexpr int RS = 64 + PAD;
    static constexpr int ROWP = CHUNK * RS * 2;  // one bf16 plane of a token-major [64][64] operand
    static constexpr int TILE = 64 * 4 * 2;      // one 16x16 tile in lane order, one bf16 part
    static constexpr int ATP = 10 * TILE;        // the ten causal tiles of A^T
    static constexpr int LTP = 6 * TILE;         // the six off-diagonal tiles of L^T
    static constexpr int TIP = 4 * TILE;         // the four diagonal inverses (A-operand layout)
    static constexpr int OS = 20;                // output staging row stride (floats)
    static constexpr int WSB = 16 * OS * 4;      // per wave: fp32 L_ii (stage 2) / output staging
    static constexpr int OFF_Q = 0;
    static constexpr int OFF_K = OFF_Q + (OUT ? NX * ROWP : 0);
    static constexpr int OFF_V = OFF_K + NX * ROWP;
    static constexpr int OFF_AT = OFF_V + NX * ROWP;
    static constexpr int OFF_LT = OFF_AT + (OUT ? NS * ATP : 0);
    static constexpr int OFF_TI = OFF_LT + NS * LTP;
    static constexpr int OFF_WS = OFF_TI + NS * TIP;
    static constexpr int OFF_F = OFF_WS + 4 * WSB;
    // per-token factor arrays (64 floats each); log-decays in log2 units
    static constexpr int F_G2 = 0, F_GP2 = 64, F_EG = 128, F_EGP = 192, F_W = 256, F_B = 320, F_MISC = 384;
    static constexpr int BYTES = OFF_F + (F_MISC + 4) * 4;
    static_assert(16 * 16 * 4 <= WSB, "L_ii fits in a wave's staging area");
    static_assert(BYTES <= 160 * 1024, "LDS budget");
};

// Inputs of one chunk: q, k, v under the stage-1 lane mapping of chunk_common.h (lane 4*tg + row
// of wave w holds tokens 4*tg + j, columns 16w + 4*row + [0, 4)), and the gate and beta of token
// `lane` (every wave loads them; wave 0 turns them into the factor arrays).
template <typename TIn>
struct SIn {
    Vec<TIn, 4> q[4], k[4], v[4];
    float g, b;
};

struct SAddr {
    TokAddr q, k, v;
};

template <bool OUT, bool CK, typename TIn>
__device__ __forceinline__ void sg_load(SIn<TIn>& c, const SAddr& ad, const PrefillParams& a, const Work& wk,
                                        int64_t h, int64_t tc, int nv, bool valid) {
    if (OUT) rows_load<CK>(c.q, chunk_rsrc(ad.q, tc, valid), ad.q, tc);
    rows_load<CK>(c.k, chunk_rsrc(ad.k, tc, valid), ad.k, tc);
    rows_load<CK>(c.v, chunk_rsrc(ad.v, tc, valid), ad.v, tc);
    const int lane = threadIdx.x & 63;
    const bool ok = valid && lane < nv;
    c.g = ok ? scalar_gate(a, wk, h, tc + lane) : 0.f;
    c.b = (ok && a.beta_kind == BETA_HEAD) ? beta_value(a, wk, h, tc + lane) : 1.f;
}

// The value of x held by row group G (lanes 16G..16G+15) of the same r16, in every lane: two
// whole-row swaps (VALU, no LDS).
template <int G>
__device__ __forceinline__ float group_bcast(float x) {
    const RowPair p = swap16(x);  // lo = [x0, x0, x2, x2], hi = [x1, x1, x3, x3]
    const RowPair q = swap32((G & 1) ? p.hi : p.lo);
    return (G & 2) ? q.hi : q.lo;
}

// Two K=16 fragments (slots 0..3 each) joined into one K=32 fragment.
template <int NP>
__device__ __forceinline__ Split8<NP> join_k32(const Split8<NP>& lo, const Split8<NP>& hi) {
    Split8<NP> f;
#pragma unroll
    for (int pl = 0; pl < NP; ++pl)
        f.p[pl] = bf16x8{lo.p[pl][0], lo.p[pl][1], lo.p[pl][2], lo.p[pl][3],
                         hi.p[pl][0], hi.p[pl][1], hi.p[pl][2], hi.p[pl][3]};
    return f;
}

// One chunk of the walk for (segment, head).  OUT: outputs from the state S (K3).  Otherwise (K1)
// the segment map on two states at once: S driven with V = 0 (the M columns) and SN with the
// real V (the N columns), sharing stages 1-2.
template <typename TIn, bool OUT, bool CK>
struct SgStep {
    using L = SLay<TIn, OUT>;
    static constexpr int NS = L::NS, NX = L::NX;

    template <typename Hook>
    __device__ static void run(const PrefillParams& a, const Work& wk, int64_t h, int64_t tc, int nv,
                               const SIn<TIn>& cur, f32x4 (&S)[4], f32x4 (&SN)[4], char* smem, Hook&& after_inputs) {
        const int lane = threadIdx.x & 63, wave = wave_id(), r16 = lane & 15, g4 = lane >> 4;
        const int tg = lane >> 2, row = lane & 3;
        const int c0 = wave * 16;
        char* sQ = smem + L::OFF_Q;
        char* sK = smem + L::OFF_K;
        char* sV = smem + L::OFF_V;
        char* sAT = smem + L::OFF_AT;
        char* sLT = smem + L::OFF_LT;
        char* sTI = smem + L::OFF_TI;
        float* sWS = reinterpret_cast<float*>(smem + L::OFF_WS + wave * L::WSB);
        float* sF = reinterpret_cast<float*>(smem + L::OFF_F);

        // ---------------- stage 1: operands as loaded -> LDS; per-token factors ------------
        {
            const int col = c0 + 4 * row;
            if (OUT) lds_put_v_rows<TIn, NX, CK>(sQ, L::ROWP, L::RS, col, cur.q, tg, nv);
            lds_put_v_rows<TIn, NX, CK>(sK, L::ROWP, L::RS, col, cur.k, tg, nv);
            lds_put_v_rows<TIn, NX, CK>(sV, L::ROWP, L::RS, col, cur.v, tg, nv);
            if (wave == 0) {
                // lane = token; tokens past nv carry g = 0 (their k, v, q rows are zero)
                const float gv = min0(cur.g) * LOG2E;
                const int rr = lane >> 4;
                // inclusive prefix: within each 16-lane row, then the earlier rows' totals
                float x = row_inclusive_scan(gv);
                const float t0 = lane_value(x, 15), t1 = lane_value(x, 31), t2 = lane_value(x, 47);
                x += (rr >= 1 ? t0 : 0.f) + (rr >= 2 ? t1 : 0.f) + (rr >= 3 ? t2 : 0.f);
                // exclusive prefix: the previous token's inclusive one (exactly)
                const float xl = lane_bcast(x, (lane + 63) & 63);
                const float xp = lane == 0 ? 0.f : xl;
                // exclusive suffix (sum over the later tokens), summed from the later tokens only
                float y = gv;
                y += row_shl<1>(y);
                y += row_shl<2>(y);
                y += row_shl<4>(y);
                y += row_shl<8>(y);
                const float u1 = lane_value(y, 16), u2 = lane_value(y, 32), u3 = lane_value(y, 48);
                y += (rr < 1 ? u1 : 0.f) + (rr < 2 ? u2 : 0.f) + (rr < 3 ? u3 : 0.f);
                const float yl = lane_bcast(y, (lane + 1) & 63);
                const float ys = lane == 63 ? 0.f : yl;
                const float tot = lane_value(x, 63);
                sF[L::F_G2 + lane] = x;
                sF[L::F_GP2 + lane] = xp;
                sF[L::F_EG + lane] = __builtin_amdgcn_exp2f(x);
                sF[L::F_EGP + lane] = __builtin_amdgcn_exp2f(xp);
                sF[L::F_W + lane] = cur.b * __builtin_amdgcn_exp2f(ys);
                sF[L::F_B + lane] = cur.b;
                if (lane == 0) {
                    sF[L::F_MISC] = __builtin_amdgcn_exp2f(tot);
                    sF[L::F_MISC + 1] = (tot >= -SPAN_MAX * LOG2E) ? 0.f : 1.f;  // false for NaN too
                }
            }
        }
        after_inputs();
        __syncthreads();
        if (__builtin_amdgcn_readfirstlane(__float_as_int(sF[L::F_MISC + 1])) != 0) {
            gdn_tokenwise<TIn, TIn, OUT, true>(a, wk, h, c0, tc, nv, g4, r16, OUT, S);
            if (!OUT) gdn_tokenwise<TIn, TIn, false, true>(a, wk, h, c0, tc, nv, g4, r16, true, SN);
            __syncthreads();
            return;
        }

        // ---------------- stage 2: decayed product tiles; diagonal-block inverses ----------
        {
            // Tiles (sb, tb) hold rows s of block sb and columns t of block tb: the ten causal
            // tiles of A^T = diag(beta) K Q^T (decayed) and the six off-diagonal tiles of L^T.
            constexpr int NT = OUT ? 16 : 6;
            for (int n = wave; n < NT; n += 4) {
                const bool is_a = OUT && n < 10;
                int sb, tb, idx;
                if (is_a) {
                    idx = n;
                    tile_sb_tb(idx, sb, tb);
                } else {
                    const int m = OUT ? n - 10 : n;  // (0,1) (0,2) (1,2) (0,3) (1,3) (2,3)
                    tb = m >= 3 ? 3 : (m >= 1 ? 2 : 1);
                    sb = m - (tb - 1) * tb / 2;
                    idx = m;
                }
                f32x4 acc = zero4();
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    const Split8<NX> kf = lds_frag<NX>(sK, L::ROWP, L::RS, 16 * sb + r16, 32 * ks, g4);
                    const Split8<NX> rf = lds_frag<NX>(is_a ? sQ : sK, L::ROWP, L::RS, 16 * tb + r16, 32 * ks, g4);
                    acc = mfma_split<NX, NX, NX>(kf, rf, acc);
                }
                const f32x4 gs = *reinterpret_cast<const f32x4*>(sF + L::F_G2 + 16 * sb + 4 * g4);
                const f32x4 bs = *reinterpret_cast<const f32x4*>(sF + L::F_B + 16 * sb + 4 * g4);
                const float gt = sF[(is_a ? L::F_G2 : L::F_GP2) + 16 * tb + r16];
                float xv[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const bool keep = !(is_a && sb == tb) || 4 * g4 + j <= r16;
                    const float f = bs[j] * __builtin_amdgcn_exp2f(gt - gs[j]);
                    xv[j] = keep ? acc[j] * f : 0.f;
                }
                lds_put_row<NS, 4>(is_a ? sAT : sLT, is_a ? L::ATP : L::LTP, (idx * 64 + lane) * 4, xv);
            }
            // Diagonal block `wave`: L_ii from its Gram tile (symmetric, so the lane that holds
            // G[s][t] also holds G[t][s]), stored row-major in fp32 for the substitution.
            {
                const int ib = wave;
                f32x4 G = zero4();
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    const Split8<NX> kf = lds_frag<NX>(sK, L::ROWP, L::RS, 16 * ib + r16, 32 * ks, g4);
                    G = mfma_split<NX, NX, NX>(kf, kf, G);  // G[4*g4 + j][r16]
                }
                const f32x4 gs = *reinterpret_cast<const f32x4*>(sF + L::F_G2 + 16 * ib + 4 * g4);
                const f32x4 bs = *reinterpret_cast<const f32x4*>(sF + L::F_B + 16 * ib + 4 * g4);
                const float gpt = sF[L::F_GP2 + 16 * ib + r16];
                f32x4 lr;  // L[t = r16][s = 4*g4 + j]
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float f = bs[j] * __builtin_amdgcn_exp2f(gpt - gs[j]);
                    lr[j] = (r16 > 4 * g4 + j) ? G[j] * f : 0.f;
                }
                *reinterpret_cast<f32x4*>(sWS + 16 * r16 + 4 * g4) = lr;
                __builtin_amdgcn_wave_barrier();
                // Y = T_ii^T = (I + L_ii^T)^{-1}: row a of Y is e_a - sum_{b > a} L[b][a] Y[b], so
                // rows are final from the last one down; lane (g4, r16) holds Y[4*g4 + j][r16].
                f32x4 Y;
#pragma unroll
                for (int j = 0; j < 4; ++j) Y[j] = (4 * g4 + j == r16) ? 1.f : 0.f;
#pragma unroll
                for (int b = 15; b >= 1; --b) {
                    const f32x4 lb = *reinterpret_cast<const f32x4*>(sWS + 16 * b + 4 * g4);  // L[b][4*g4 + j]
                    float yb;
                    switch (b >> 2) {
                        case 0: yb = group_bcast<0>(Y[b & 3]); break;
                        case 1: yb = group_bcast<1>(Y[b & 3]); break;
                        case 2: yb = group_bcast<2>(Y[b & 3]); break;
                        default: yb = group_bcast<3>(Y[b & 3]); break;
                    }
#pragma unroll
                    for (int j = 0; j < 4; ++j) Y[j] -= lb[j] * yb;
                }
                const float xv[4] = {Y[0], Y[1], Y[2], Y[3]};  // A-operand layout of T_ii
                lds_put_row<NS, 4>(sTI, L::TIP, (ib * 64 + lane) * 4, xv);
            }
        }
        __syncthreads();

        // ---------------- stage 3: residuals, UT solve, outputs, state ----------------------
        const float eG = sF[L::F_MISC];
        auto pass = [&](auto with_v, f32x4 (&St)[4]) {
            constexpr bool WV = decltype(with_v)::value;
            Split8<NS> sf[2];  // S0 with K = key dims (B operand of S0, A operand of S0^T)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) sf[ks] = split_k32<NS>(St[2 * ks], St[2 * ks + 1]);
            // R_i = V_i - e^{gamp} (K S0)_i  (D layout: rows t = 16i + 4*g4 + k, column c0 + r16)
            f32x4 R[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                f32x4 p = zero4();
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    const Split8<NX> kf = lds_frag<NX>(sK, L::ROWP, L::RS, 16 * i + r16, 32 * ks, g4);
                    p = mfma_split<NX, NS, NS>(kf, sf[ks], p);
                }
                const f32x4 ep = *reinterpret_cast<const f32x4*>(sF + L::F_EGP + 16 * i + 4 * g4);
                f32x4 vv = zero4();
                if constexpr (WV) {
                    const int off = (16 * i + 4 * g4 + (r16 >> 2)) * L::RS + c0 + 4 * (r16 & 3);
#pragma unroll
                    for (int pl = 0; pl < NX; ++pl) {
                        const bf16x4 t4 = lds_read_tr(reinterpret_cast<const __bf16*>(sV + pl * L::ROWP) + off);
#pragma unroll
                        for (int k = 0; k < 4; ++k) vv[k] += (float)t4[k];
                    }
                }
#pragma unroll
                for (int k = 0; k < 4; ++k) R[i][k] = vv[k] - ep[k] * p[k];
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
                        p = mfma_split<NS, NS, NS>(lf, join_k32<NS>(us[0], us[1]), p);
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
                const Split8<NS> tf = tile_frag<NS>(sTI, L::TIP, i, 0, false, lane);
                U[i] = mfma_split<NS, NS, NS>(tf, split_k16<NS>(X), zero4());
                us[i] = split_k16<NS>(U[i]);
            }

            if constexpr (OUT) {
                // O^T tiles: lane (g4, r16) holds O[token 16*tb + r16][columns c0 + 4*g4 + 0..3]
                f32x4 Ot[4];
#pragma unroll
                for (int tb = 0; tb < 4; ++tb) {
                    f32x4 o = zero4();
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) {
                        const Split8<NX> qf = lds_frag<NX>(sQ, L::ROWP, L::RS, 16 * tb + r16, 32 * ks, g4);
                        o = mfma_split<NS, NX, NS>(sf[ks], qf, o);
                    }
                    const float eg = sF[L::F_EG + 16 * tb + r16];
#pragma unroll
                    for (int k = 0; k < 4; ++k) o[k] *= eg;
#pragma unroll
                    for (int k2 = 0; k2 < 2; ++k2) {
                        if (2 * k2 > tb) continue;
                        const bool has_hi = 2 * k2 + 1 <= tb;
                        const Split8<NS> af = tile_frag<NS>(sAT, L::ATP, tile_index(2 * k2, tb),
                                                            has_hi ? tile_index(2 * k2 + 1, tb) : 0, has_hi, lane);
                        o = mfma_split<NS, NS, NS>(join_k32<NS>(us[2 * k2], us[2 * k2 + 1]), af, o);
                    }
                    Ot[tb] = o;
                }
                // stage through this wave's area and store quad-coalesced rows
                const int es = dt_size(a.o_dt);
                const int64_t ost = a.o_st * es;
                char* obase = reinterpret_cast<char*>(a.o) +
                              uniform_i64((wk.b * a.o_sb + (wk.row0 + tc) * a.o_st + h * a.o_sh + c0) * es);
                const int q = lane & 3, tq = (lane >> 4) + 4 * ((lane >> 2) & 3);
                const int32_t olane = (int32_t)(tq * ost) + 4 * q * es;
                const OutRsrc orr = out_rsrc(obase, ost, es, nv, a.o_dt == DT_F32);
                wait_vmem();  // the next chunk's loads have landed: later waits skip these stores
#pragma unroll
                for (int tb = 0; tb < 4; ++tb) {
                    *reinterpret_cast<f32x4*>(sWS + r16 * L::OS + 4 * g4) = Ot[tb];
                    const f32x4 xo = *reinterpret_cast<const f32x4*>(sWS + tq * L::OS + 4 * q);
                    out_store4(orr, (int32_t)(16 * tb * ost) + olane, a.o_dt, xo);
                }
            }
            // S <- e^{Gam} S0 + K^T diag(w) U,  w = beta e^{Gam - gam}
            Split8<NS> uw[2];
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2) {
                const f32x4 wl = *reinterpret_cast<const f32x4*>(sF + L::F_W + 32 * k2 + 4 * g4);
                const f32x4 wh = *reinterpret_cast<const f32x4*>(sF + L::F_W + 32 * k2 + 16 + 4 * g4);
                f32x4 lo, hi;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    lo[k] = U[2 * k2][k] * wl[k];
                    hi[k] = U[2 * k2 + 1][k] * wh[k];
                }
                uw[k2] = split_k32<NS>(lo, hi);
            }
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                f32x4 acc;
#pragma unroll
                for (int k = 0; k < 4; ++k) acc[k] = eG * St[db][k];
#pragma unroll
                for (int k2 = 0; k2 < 2; ++k2) {
                    const Split8<NX> kf = lds_frag_tr<NX>(sK, L::ROWP, L::RS, 32 * k2, 16 * db, g4, r16);
                    acc = mfma_split<NX, NS, NS>(kf, uw[k2], acc);
                }
                St[db] = acc;
            }
        };
        if constexpr (OUT) {
            pass(std::true_type{}, S);
        } else {
            pass(std::false_type{}, S);
            __builtin_amdgcn_sched_barrier(0);  // one pass at a time: their temporaries never overlap
            pass(std::true_type{}, SN);
        }
        __syncthreads();  // the next chunk rewrites LDS
    }
};

template <typename TIn, bool OUT, bool CK>
__device__ void sg_walk(const PrefillParams& a, const Work& wk, int64_t h, f32x4 (&S)[4], f32x4 (&SN)[4], char* smem) {
    using St = SgStep<TIn, OUT, CK>;
    const int lane = threadIdx.x & 63, wave = wave_id(), tg = lane >> 2, row = lane & 3;
    const int col = wave * 16 + 4 * row;
    SAddr ad;
    if (OUT) ad.q = tok_addr<TIn>(a.q, wk, h, tg, col);
    ad.k = tok_addr<TIn>(a.k, wk, h, tg, col);
    ad.v = tok_addr<TIn>(a.v, wk, h, tg, col);
    const int64_t nch = (wk.t_end - wk.t_begin + CHUNK - 1) / CHUNK;
    auto chunk_nv = [&](int64_t c) {
        const int64_t r = wk.t_end - (wk.t_begin + c * CHUNK);
        return (int)(r < CHUNK ? r : CHUNK);
    };
    auto tok = [&](int64_t c) { return wk.t_begin + c * CHUNK; };
    SIn<TIn> A;
    sg_load<OUT, CK>(A, ad, a, wk, h, tok(0), chunk_nv(0), true);
    for (int64_t c = 0; c < nch; ++c)
        St::run(a, wk, h, tok(c), chunk_nv(c), A, S, SN, smem, [&] {
            const bool more = c + 1 < nch;
            sg_load<OUT, CK>(A, ad, a, wk, h, tok(c + 1), more ? chunk_nv(c + 1) : 0, more);
        });
}

// K1: the segment map driven from [I | 0] with V = 0 (-> M_p) and from 0 with the real V (-> N_p).
template <typename TIn, bool CK>
__global__ __launch_bounds__(256, Prec<TIn>::F32 ? 1 : 2) void gdn_sg_seg_mn_kernel(PrefillParams a) {
    using L = SLay<TIn, false>;
    __shared__ __attribute__((aligned(16))) char smem[L::BYTES];
    const int64_t w = blockIdx.x, h = blockIdx.y;
    Work wk;
    if (!find_work(a, w, wk)) return;
    f32x4 M[4], N[4];
    init_seg_map(M, N);
    sg_walk<TIn, false, CK>(a, wk, h, M, N, smem);
    store_seg_map<Prec<TIn>::NS>(a, w, h, M, N);
}

// K3: outputs of one segment from S_in[p] (in the N slot after the scan).
template <typename TIn, bool CK>
__global__ __launch_bounds__(256, ((2 * SLay<TIn, true>::BYTES <= 160 * 1024) ? 2 : 1)) void gdn_sg_seg_out_kernel(
    PrefillParams a) {
    using L = SLay<TIn, true>;
    __shared__ __attribute__((aligned(16))) char smem[L::BYTES];
    const int64_t w = blockIdx.x, h = blockIdx.y;
    Work wk;
    if (!find_work(a, w, wk)) return;
    f32x4 S[4];
    load_seg_state(a, w, h, S);
    sg_walk<TIn, true, CK>(a, wk, h, S, S, smem);
}

// ---------------------------------------------------------------------------------------
// Host launchers.
// ---------------------------------------------------------------------------------------
template <typename TIn, bool CK>
static hipError_t launch_sg_ck(const PrefillParams& a, int64_t n_work, int which, hipStream_t stream) {
    const dim3 grid((unsigned)n_work, (unsigned)a.H);
    if (which == 0) hipLaunchKernelGGL((gdn_sg_seg_mn_kernel<TIn, CK>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((gdn_sg_seg_out_kernel<TIn, CK>), grid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

// Unchecked row addressing only when T is a whole number of four-row groups.
template <typename TIn>
static hipError_t launch_sg_t(const PrefillParams& a, int64_t n_work, int which, hipStream_t stream) {
    if (a.T % 4 == 0) return launch_sg_ck<TIn, false>(a, n_work, which, stream);
    return launch_sg_ck<TIn, true>(a, n_work, which, stream);
}

static hipError_t launch_sg(const PrefillParams& a, int64_t n_work, int io_dt, int which, hipStream_t stream) {
    if (io_dt == DT_BF16) return launch_sg_t<__bf16>(a, n_work, which, stream);
    if (io_dt == DT_F16) return launch_sg_t<_Float16>(a, n_work, which, stream);
    if (io_dt == DT_F32) return launch_sg_t<float>(a, n_work, which, stream);
    return hipErrorInvalidValue;
}

hipError_t launch_gdn_sg_seg_mn(const PrefillParams& a, int64_t n_work, int io_dt, hipStream_t stream) {
    return launch_sg(a, n_work, io_dt, 0, stream);
}

hipError_t launch_gdn_sg_seg_out(const PrefillParams& a, int64_t n_work, int io_dt, hipStream_t stream) {
    return launch_sg(a, n_work, io_dt, 1, stream);
}

// Resident output-kernel workgroups per CU for I/O dtype io_dt on the instance that runs (ck:
// checked row addressing, launched unless T % 4 == 0).
int gdn_sg_seg_out_blocks_per_cu(int io_dt, bool ck) {
    const void* k =
        io_dt == DT_F16 ? (ck ? reinterpret_cast<const void*>(gdn_sg_seg_out_kernel<_Float16, true>)
                              : reinterpret_cast<const void*>(gdn_sg_seg_out_kernel<_Float16, false>))
        : io_dt == DT_F32 ? (ck ? reinterpret_cast<const void*>(gdn_sg_seg_out_kernel<float, true>)
                                : reinterpret_cast<const void*>(gdn_sg_seg_out_kernel<float, false>))
                          : (ck ? reinterpret_cast<const void*>(gdn_sg_seg_out_kernel<__bf16, true>)
                                : reinterpret_cast<const void*>(gdn_sg_seg_out_kernel<__bf16, false>));
    int nb = 0;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k, 256, 0);
    return (e == hipSuccess && nb > 0) ? nb : 1;
}

}  // namespace triune
