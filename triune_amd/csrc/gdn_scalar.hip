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
// U_i = T_ii (R_i - sum_{j<i} L_ij U_j), with the state-independent products T_ii L_ij and
// T_ii diag(e^{gamp}) K_i formed once per chunk; each T_ii comes from an fp32 back substitution
// on T_ii^T = (I + L_ii^T)^{-1}, one wave per block.  Chunks whose total log-decay exceeds SPAN_MAX
// (or is not finite) run token by token: the exponent differences come from prefix sums, whose
// rounding grows with the chunk total.
// The segment decomposition is the one of gdn_chunk.hip and shares its workspace layout and scan:
//   K1 gdn_sg_seg_mn  : per (segment, head) the segment map from [I | 0] with V = 0 (-> M_p) and
//                       from 0 with the real V (-> N_p) in one chunk walk
//   K2 gdn_seg_scan   : the carry S_in[p] (gdn_chunk.hip)
//   K3 gdn_sg_seg_out : per (segment, head) the chunk walk from S_in[p], writing o
#include "gdn_common.h"

namespace triune {

// ---- K=16 operands ---------------------------------------------------------------------------
// Lane (g4, r16) holds row (A) or column (B) r16 and the K slots (g4, j), j < 4: the lower half of
// a K=32 fragment.  Products whose contraction is one 16-token block keep their operands in this
// form and run as K=32 products with the upper slots zero.  (The 16x16x16 bf16 instruction issues
// no faster than the 16x16x32 one on gfx950, and gave wrong results in this kernel.)
template <int N>
struct Split4 {
    bf16x4 p[N];
};

__device__ __forceinline__ f32x4 mfma16(const bf16x4& a, const bf16x4& b, const f32x4& c) {
    const __bf16 z = (__bf16)0.f;
    return mfma(bf16x8{a[0], a[1], a[2], a[3], z, z, z, z}, bf16x8{b[0], b[1], b[2], b[3], z, z, z, z}, c);
}

template <int NA, int NB, int NS>
__device__ __forceinline__ f32x4 mfma16_split(const Split4<NA>& a, const Split4<NB>& b, f32x4 c) {
#pragma unroll
    for (int ia = 0; ia < NA; ++ia)
#pragma unroll
        for (int ib = 0; ib < NB; ++ib)
            if (ia + ib < NS) c = mfma16(a.p[ia], b.p[ib], c);
    return c;
}

template <int NP>
__device__ __forceinline__ Split4<NP> split4(const f32x4& v) {
    float r[4] = {v[0], v[1], v[2], v[3]};
    uint32_t w[NP][2];
    split_pairs<NP, 2>(r, w);
    Split4<NP> f;
#pragma unroll
    for (int pl = 0; pl < NP; ++pl) f.p[pl] = __builtin_bit_cast(bf16x4, uint2{w[pl][0], w[pl][1]});
    return f;
}

// Two K=16 fragments as one K=32 fragment (slots 0..3 from lo, 4..7 from hi).
template <int NP>
__device__ __forceinline__ Split8<NP> join4(const Split4<NP>& lo, const Split4<NP>& hi) {
    Split8<NP> f;
#pragma unroll
    for (int pl = 0; pl < NP; ++pl)
        f.p[pl] = bf16x8{lo.p[pl][0], lo.p[pl][1], lo.p[pl][2], lo.p[pl][3], hi.p[pl][0], hi.p[pl][1], hi.p[pl][2],
                         hi.p[pl][3]};
    return f;
}

// ---- fragment planes --------------------------------------------------------------------------
// A fragment is one MFMA operand per lane: a pair (K=32, two 16x16 tiles, 16 bytes per lane) or a
// single (K=16, one tile, 8 bytes per lane), stored lane-major so that every lane reads its operand
// with one access.  A plane lists its fragments back to back; FragAt gives where fragment f starts.
// A tile is written as one half of a pair fragment, or as a single one.
struct FragAt {
    int off;  // byte offset of the fragment within the plane
    bool pair;
};

template <int NP>
__device__ __forceinline__ void frag_put(char* base, int plane_bytes, FragAt f, int half, int lane,
                                         const float (&x)[4]) {
    float r[4] = {x[0], x[1], x[2], x[3]};
    uint32_t w[NP][2];
    split_pairs<NP, 2>(r, w);
    const int o = f.off + (f.pair ? lane * 16 + half * 8 : lane * 8);
#pragma unroll
    for (int pl = 0; pl < NP; ++pl) *reinterpret_cast<uint2*>(base + pl * plane_bytes + o) = uint2{w[pl][0], w[pl][1]};
}

template <int NP>
__device__ __forceinline__ Split8<NP> frag_get8(const char* base, int plane_bytes, FragAt f, int lane) {
    Split8<NP> r;
#pragma unroll
    for (int pl = 0; pl < NP; ++pl) r.p[pl] = *reinterpret_cast<const bf16x8*>(base + pl * plane_bytes + f.off + lane * 16);
    return r;
}

template <int NP>
__device__ __forceinline__ Split4<NP> frag_get4(const char* base, int plane_bytes, FragAt f, int lane) {
    Split4<NP> r;
#pragma unroll
    for (int pl = 0; pl < NP; ++pl) r.p[pl] = *reinterpret_cast<const bf16x4*>(base + pl * plane_bytes + f.off + lane * 8);
    return r;
}

constexpr int SINGLE_B = 64 * 8, PAIR_B = 64 * 16;

// Fragments of A^T (tiles (sb, tb), sb <= tb): fragment (k2, tb) holds tiles (2*k2, tb) and
// (2*k2 + 1, tb), a single where 2*k2 == tb.  Order: (0,0) (0,1) (0,2) (0,3) (1,2) (1,3).
__device__ __forceinline__ FragAt afrag(int k2, int tb) {
    if (k2 == 0) return tb == 0 ? FragAt{0, false} : FragAt{SINGLE_B + (tb - 1) * PAIR_B, true};
    return tb == 2 ? FragAt{SINGLE_B + 3 * PAIR_B, false} : FragAt{2 * SINGLE_B + 3 * PAIR_B, true};
}
constexpr int AF_BYTES = 2 * SINGLE_B + 4 * PAIR_B;
// Fragments of the off-diagonal solve tiles X_ij (j < i; -L_ij or -P_ij): [X_10] [X_20 X_21]
// [X_30 X_31] [X_32]; half = j for the pairs.
__device__ __forceinline__ FragAt xfrag(int j, int i) {
    if (i == 1) return FragAt{0, false};
    if (j < 2) return FragAt{SINGLE_B + (i - 2) * PAIR_B, true};
    return FragAt{SINGLE_B + 2 * PAIR_B, false};
}
constexpr int XF_BYTES = 2 * SINGLE_B + 2 * PAIR_B;
// The diagonal inverses T_ii: four singles.
__device__ __forceinline__ FragAt tfrag(int i) { return FragAt{i * SINGLE_B, false}; }
constexpr int TF_BYTES = 4 * SINGLE_B;

// Four V (or K) elements of one 16-token block down one column, through the transposed LDS read:
// rows row0 + 4*g4 + [0, 4), column col, as a K=16 operand (one bf16 part per plane).
template <int NP>
__device__ __forceinline__ Split4<NP> col_frag4(const char* base, int plane_bytes, int rs, int row0, int col, int g4,
                                                int r16) {
    Split4<NP> f;
    const int off = (row0 + 4 * g4 + (r16 >> 2)) * rs + col + 4 * (r16 & 3);
#pragma unroll
    for (int pl = 0; pl < NP; ++pl) f.p[pl] = lds_read_tr(reinterpret_cast<const __bf16*>(base + pl * plane_bytes) + off);
    return f;
}

// LDS of one chunk step.  PRE: the solve uses the precomputed products (-Bk planes, -P tiles);
// otherwise the residual form (-L tiles).
template <typename TIn, bool OUT, bool PRE>
struct SLay {
    using P = Prec<TIn>;
    static constexpr int NX = P::NX, NS = P::NS;
    static constexpr int RS = 64 + PAD;
    static constexpr int ROWP = CHUNK * RS * 2;  // one bf16 plane of a token-major [64][64] operand
    static constexpr int OS = 16;                // output staging row stride (floats)
    static constexpr int WSB = 16 * OS * 4;      // per wave: fp32 L_ii (stage 2) / output staging
    static constexpr int OFF_Q = 0;
    static constexpr int OFF_K = OFF_Q + (OUT ? NX * ROWP : 0);
    static constexpr int OFF_V = OFF_K + NX * ROWP;
    static constexpr int OFF_BK = OFF_V + NX * ROWP;  // -Bk = -T diag(e^{gamp}) K, token-major (PRE)
    static constexpr int OFF_AF = OFF_BK + (PRE ? NS * ROWP : 0);
    static constexpr int OFF_XF = OFF_AF + (OUT ? NS * AF_BYTES : 0);
    static constexpr int OFF_TF = OFF_XF + NS * XF_BYTES;
    static constexpr int OFF_WS = OFF_TF + NS * TF_BYTES;
    static constexpr int OFF_F = OFF_WS + 4 * WSB;
    // per-token factor arrays (64 floats each; log-decays in log2 units):
    //   G2 gam, GP2 gamp, EG e^{gam}, EGP e^{gamp}, W beta e^{Gam - gam}, B beta,
    //   BSB beta e^{gam_e(blk) - gam} (gam_e(b): gam at the last token of 16-token block b),
    //   CF[j] e^{gamp - gam_e(j)} and CFA[j] e^{gam - gam_e(j)} for blocks j = 0..2 (used for
    //   tokens of later blocks, where both exponents are <= 0)
    static constexpr int F_G2 = 0, F_GP2 = 64, F_EG = 128, F_EGP = 192, F_W = 256, F_B = 320, F_BSB = 384,
                         F_CF = 448, F_CFA = 640, F_MISC = 832;
    static constexpr int BYTES = OFF_F + (F_MISC + 4) * 4;
    static_assert(16 * 16 * 4 <= WSB, "L_ii fits in a wave's staging area");
    static_assert(BYTES <= 160 * 1024, "LDS budget");
};

// What the chunk walk of one (segment, head) reads and writes, made once per workgroup: q, k, v
// under the stage-1 lane mapping of chunk_common.h (lane 4*tg + row of wave w holds tokens
// 4*tg + j, columns 16w + 4*row + [0, 4)), and the gate, beta and output of token 0 of the
// sequence with their token strides in bytes.  The chunk loop and its token-by-token fallback
// use nothing else of the kernel arguments.
struct SgCtx {
    TokAddr q, k, v;
    const char* gp;
    const char* bp;  // null without per-token beta
    char* op;
    int64_t gst, bst, ost;
    int g_dt, b_dt, o_dt;
};

template <bool OUT, typename TIn>
__device__ __forceinline__ SgCtx sg_ctx(const PrefillParams& a, const Work& wk, int64_t h, int tg, int col) {
    SgCtx x;
    if (OUT) x.q = tok_addr<TIn>(a.q, wk, h, tg, col);
    x.k = tok_addr<TIn>(a.k, wk, h, tg, col);
    x.v = tok_addr<TIn>(a.v, wk, h, tg, col);
    const int64_t ges = dt_size(a.g_dt);
    x.gp = reinterpret_cast<const char*>(a.g.p) + uniform_i64((wk.b * a.g.sb + wk.row0 * a.g.st + h * a.g.sh) * ges);
    x.gst = uniform_i64(a.g.st * ges);
    x.g_dt = a.g_dt;
    const bool hb = a.beta_kind == BETA_HEAD;
    const int64_t bes = dt_size(a.beta_dt);
    x.bp = hb ? reinterpret_cast<const char*>(a.beta) + uniform_i64((wk.b * a.b_sb + wk.row0 * a.b_st + h * a.b_sh) * bes)
              : nullptr;
    x.bst = hb ? uniform_i64(a.b_st * bes) : 0;
    x.b_dt = a.beta_dt;
    const int64_t oes = dt_size(a.o_dt);
    x.op = reinterpret_cast<char*>(a.o) + uniform_i64((wk.b * a.o_sb + wk.row0 * a.o_st + h * a.o_sh) * oes);
    x.ost = uniform_i64(a.o_st * oes);
    x.o_dt = a.o_dt;
    return x;
}

__device__ __forceinline__ float load_scalar(const char* p, int dt) {
    if (dt == DT_F32) return *reinterpret_cast<const float*>(p);
    if (dt == DT_BF16) return (float)*reinterpret_cast<const __bf16*>(p);
    return (float)*reinterpret_cast<const _Float16*>(p);
}

// Inputs of one chunk: q, k, v under the stage-1 mapping, and the gate and beta of token `lane`
// (every wave loads them; wave 0 turns them into the factor arrays).
template <typename TIn>
struct SIn {
    Vec<TIn, 4> q[4], k[4], v[4];
    float g, b;
};

template <bool OUT, bool CK, typename TIn>
__device__ __forceinline__ void sg_load(SIn<TIn>& c, const SgCtx& x, int64_t tc, int nv, bool valid) {
    if (OUT) rows_load<CK>(c.q, chunk_rsrc(x.q, tc, valid), x.q, tc);
    rows_load<CK>(c.k, chunk_rsrc(x.k, tc, valid), x.k, tc);
    rows_load<CK>(c.v, chunk_rsrc(x.v, tc, valid), x.v, tc);
    const int lane = threadIdx.x & 63;
    const bool ok = valid && lane < nv;
    c.g = ok ? load_scalar(x.gp + (tc + lane) * x.gst, x.g_dt) : 0.f;
    c.b = (ok && x.bp) ? load_scalar(x.bp + (tc + lane) * x.bst, x.b_dt) : 1.f;
}

// Token-by-token update of one wave's 16 state columns (chunks whose total log-decay is below
// -SPAN_MAX or not finite).  S tile db holds S[16*db + 4*g4 + i][c0 + r16]; with_v false reads V
// as zero.  Rows come from the context's token-0 addresses.
template <typename TIn, bool OUT>
__device__ void sg_tokenwise(const SgCtx& x, int c0, int64_t tc, int nv, int g4, int r16, bool with_v,
                             f32x4 (&S)[4]) {
    const int oes = dt_size(x.o_dt);
    for (int t = 0; t < nv; ++t) {
        const int64_t tt = tc + t;
        const float dcy = expf(fminf(load_scalar(x.gp + tt * x.gst, x.g_dt), 0.f));
        const float bt = x.bp ? load_scalar(x.bp + tt * x.bst, x.b_dt) : 1.f;
        const TIn* kr = reinterpret_cast<const TIn*>(x.k.p0 + tt * x.k.st);
        const TIn* qr = OUT ? reinterpret_cast<const TIn*>(x.q.p0 + tt * x.q.st) : nullptr;
        float kk[4][4], qq[4][4];
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                kk[db][i] = (float)kr[16 * db + 4 * g4 + i];
                qq[db][i] = OUT ? (float)qr[16 * db + 4 * g4 + i] : 0.f;
            }
        float pred = 0.f;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) pred += kk[db][i] * S[db][i];
        pred += __shfl_xor(pred, 16);
        pred += __shfl_xor(pred, 32);
        const float vv = with_v ? (float)reinterpret_cast<const TIn*>(x.v.p0 + tt * x.v.st)[c0 + r16] : 0.f;
        const float u = bt * (vv - pred);
        float part = 0.f;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float sv = dcy * S[db][i] + kk[db][i] * u;
                S[db][i] = sv;
                part += qq[db][i] * sv;
            }
        if (OUT) {
            part += __shfl_xor(part, 16);
            part += __shfl_xor(part, 32);
            if (g4 == 0) {
                char* op = x.op + tt * x.ost + (int64_t)(c0 + r16) * oes;
                if (x.o_dt == DT_F32) *reinterpret_cast<float*>(op) = part;
                else if (x.o_dt == DT_BF16) *reinterpret_cast<__bf16*>(op) = (__bf16)part;
                else *reinterpret_cast<_Float16*>(op) = (_Float16)part;
            }
        }
    }
}

// The value of x held by row group G (lanes 16G..16G+15) of the same r16, in every lane: two
// whole-row swaps (VALU, no LDS).
template <int G>
__device__ __forceinline__ float group_bcast(float x) {
    const RowPair p = swap16(x);  // lo = [x0, x0, x2, x2], hi = [x1, x1, x3, x3]
    const RowPair q = swap32((G & 1) ? p.hi : p.lo);
    return (G & 2) ? q.hi : q.lo;
}

// One chunk of the walk for (segment, head).  OUT: outputs from the state S (K3); OBF: the output
// is bf16 (stores of one encoding).  Otherwise (K1) the segment map on two states at once: S
// driven with V = 0 (the M columns) and SN with the real V (the N columns), sharing stages 1-2.
//
// Solve: U_i = T_ii (R_i - sum_{j<i} L_ij U_j), R = V - diag(e^{gamp}) K S0, T_ii = (I + L_ii)^{-1}.
// PRE (two passes per chunk, K1) forms the state-independent products once per chunk,
// P_ij = T_ii L_ij and Bk_i = T_ii diag(e^{gamp}) K_i, so that
//   U_i = T_ii V_i - Bk_i S0 - sum_{j<i} P_ij U_j
// and a pass splits only S0 and U into bf16 parts; without PRE (one pass, K3) the pass forms R
// and applies T_ii to each block, which needs no Bk planes in LDS.  Wave i forms everything of
// key block i in stage 2 (its Gram block and T_ii, the tiles of row block i of L (or P), Bk_i, and
// the A^T tiles of key block i) from the key block it holds in registers.
template <typename TIn, bool OUT, bool CK, bool OBF, bool PRE>
struct SgStep {
    using L = SLay<TIn, OUT, PRE>;
    static constexpr int NS = L::NS, NX = L::NX;

    // skip_m (K1): S is left as it is (the map of a segment whose carried-in state is zero is
    // never used).
    template <typename Hook>
    __device__ static void run(const SgCtx& x, int64_t tc, int nv, const SIn<TIn>& cur, f32x4 (&S)[4],
                               f32x4 (&SN)[4], bool skip_m, char* smem, Hook&& after_inputs) {
        const int lane = threadIdx.x & 63, wave = wave_id(), r16 = lane & 15, g4 = lane >> 4;
        const int tg = lane >> 2, row = lane & 3;
        const int c0 = wave * 16;
        char* sQ = smem + L::OFF_Q;
        char* sK = smem + L::OFF_K;
        char* sV = smem + L::OFF_V;
        char* sBK = smem + L::OFF_BK;
        char* sAF = smem + L::OFF_AF;
        char* sXF = smem + L::OFF_XF;
        char* sTF = smem + L::OFF_TF;
        float* sWS = reinterpret_cast<float*>(smem + L::OFF_WS + wave * L::WSB);
        float* sF = reinterpret_cast<float*>(smem + L::OFF_F);

        // Issue priority: stage 1 at the base level, stages 2-3 (the solve and the state chain) one
        // level up, so of the two workgroups on a CU the one further along issues first.
        __builtin_amdgcn_s_setprio(0);
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
                float xi = row_inclusive_scan(gv);
                const float t0 = lane_value(xi, 15), t1 = lane_value(xi, 31), t2 = lane_value(xi, 47);
                xi += (rr >= 1 ? t0 : 0.f) + (rr >= 2 ? t1 : 0.f) + (rr >= 3 ? t2 : 0.f);
                // exclusive prefix: the previous token's inclusive one (exactly)
                const float xl = lane_bcast(xi, (lane + 63) & 63);
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
                // gam at the last token of each 16-token block
                const float e0 = lane_value(xi, 15), e1 = lane_value(xi, 31), e2 = lane_value(xi, 47),
                            e3 = lane_value(xi, 63);
                const float eb = rr == 0 ? e0 : (rr == 1 ? e1 : (rr == 2 ? e2 : e3));
                const float b = cur.b;
                sF[L::F_G2 + lane] = xi;
                sF[L::F_GP2 + lane] = xp;
                sF[L::F_EG + lane] = __builtin_amdgcn_exp2f(xi);
                sF[L::F_EGP + lane] = __builtin_amdgcn_exp2f(xp);
                sF[L::F_W + lane] = b * __builtin_amdgcn_exp2f(ys);
                sF[L::F_B + lane] = b;
                sF[L::F_BSB + lane] = b * __builtin_amdgcn_exp2f(min0(eb - xi));
                const float ej[3] = {e0, e1, e2};
#pragma unroll
                for (int j = 0; j < 3; ++j) {
                    sF[L::F_CF + 64 * j + lane] = __builtin_amdgcn_exp2f(min0(xp - ej[j]));
                    sF[L::F_CFA + 64 * j + lane] = __builtin_amdgcn_exp2f(min0(xi - ej[j]));
                }
                if (lane == 0) {
                    sF[L::F_MISC] = __builtin_amdgcn_exp2f(e3);
                    sF[L::F_MISC + 1] = (e3 >= -SPAN_MAX * LOG2E) ? 0.f : 1.f;  // false for NaN too
                }
            }
        }
        after_inputs();
        __syncthreads();
        if (__builtin_amdgcn_readfirstlane(__float_as_int(sF[L::F_MISC + 1])) != 0) {
            if (!skip_m) sg_tokenwise<TIn, OUT>(x, c0, tc, nv, g4, r16, OUT, S);
            if (!OUT) sg_tokenwise<TIn, false>(x, c0, tc, nv, g4, r16, true, SN);
            __syncthreads();
            return;
        }

        __builtin_amdgcn_s_setprio(1);
        // ---------------- stage 2: everything of key block i = wave --------------------------
        {
            const int ib = wave;
            Split8<NX> kf[2];  // K rows of block ib (A operand, K = key dims)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) kf[ks] = lds_frag<NX>(sK, L::ROWP, L::RS, 16 * ib + r16, 32 * ks, g4);
            // T_ii^T = (I + L_ii^T)^{-1} by back substitution.  L_ii from the block's Gram tile
            // (symmetric, so the lane that holds G[s][t] also holds G[t][s]), stored row-major in
            // fp32; lane (g4, r16) ends with Y[4*g4 + j][r16] = T_ii[r16][4*g4 + j], the A-operand
            // layout of T_ii.
            f32x4 Y;
            {
                f32x4 G = zero4();
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) G = mfma_split<NX, NX, NX>(kf[ks], kf[ks], G);  // G[4*g4 + j][r16]
                const f32x4 gs = *reinterpret_cast<const f32x4*>(sF + L::F_G2 + 16 * ib + 4 * g4);
                const f32x4 bs = *reinterpret_cast<const f32x4*>(sF + L::F_B + 16 * ib + 4 * g4);
                const float gpt = sF[L::F_GP2 + 16 * ib + r16];
                f32x4 lr;  // L[t = r16][s = 4*g4 + j]
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float f = bs[j] * __builtin_amdgcn_exp2f(min0(gpt - gs[j]));
                    lr[j] = (r16 > 4 * g4 + j) ? G[j] * f : 0.f;
                }
                *reinterpret_cast<f32x4*>(sWS + 16 * r16 + 4 * g4) = lr;
                __builtin_amdgcn_wave_barrier();
                // row a of Y is e_a - sum_{b > a} L[b][a] Y[b]: rows are final from the last one down
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
                const float xv[4] = {Y[0], Y[1], Y[2], Y[3]};
                frag_put<NS>(sTF, TF_BYTES, tfrag(ib), 0, lane, xv);
            }
            if constexpr (PRE) {
                // -P_ij = -T_ii L_ij for j < ib.  L_ij as D[t][s] (rows t of block ib, columns s of
                // block j): its D layout is the A operand of L_ij^T with K = t, and the A layout of
                // T_ii is the B operand of T_ii^T, so one product gives P_ij^T in D layout, which is
                // the A-operand layout of P_ij.
                const Split4<NS> ysp = split4<NS>(Y);
                for (int j = 0; j < ib; ++j) {
                    f32x4 lt = zero4();
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) {
                        const Split8<NX> kj = lds_frag<NX>(sK, L::ROWP, L::RS, 16 * j + r16, 32 * ks, g4);
                        lt = mfma_split<NX, NX, NX>(kf[ks], kj, lt);
                    }
                    // beta_s e^{gamp_t - gam_s} = e^{gamp_t - gam_e(j)} * beta_s e^{gam_e(j) - gam_s}, negated
                    const f32x4 cf = *reinterpret_cast<const f32x4*>(sF + L::F_CF + 64 * j + 16 * ib + 4 * g4);
                    const float nbsb = -sF[L::F_BSB + 16 * j + r16];
#pragma unroll
                    for (int k = 0; k < 4; ++k) lt[k] *= cf[k] * nbsb;
                    const f32x4 pt = mfma16_split<NS, NS, NS>(split4<NS>(lt), ysp, zero4());
                    const float xv[4] = {pt[0], pt[1], pt[2], pt[3]};
                    frag_put<NS>(sXF, XF_BYTES, xfrag(j, ib), j & 1, lane, xv);
                }
                // -Bk_i = -T_ii diag(e^{gamp}) K_i as Bk^T tiles: A = K_i^T (transposed reads, K =
                // the block's tokens), B = (-T_ii diag(e^{gamp}))^T, whose B layout is the A layout
                // of T_ii with column s scaled.  Lane (g4, r16) gets -Bk[16*ib + r16][16*db + 4*g4 + j].
                const f32x4 ep = *reinterpret_cast<const f32x4*>(sF + L::F_EGP + 16 * ib + 4 * g4);
                const f32x4 te = {-Y[0] * ep[0], -Y[1] * ep[1], -Y[2] * ep[2], -Y[3] * ep[3]};
                const Split4<NS> tsp = split4<NS>(te);
#pragma unroll
                for (int db = 0; db < 4; ++db) {
                    const Split4<NX> kt = col_frag4<NX>(sK, L::ROWP, L::RS, 16 * ib, 16 * db, g4, r16);
                    const f32x4 bk = mfma16_split<NX, NS, NS>(kt, tsp, zero4());
                    const float xv[4] = {bk[0], bk[1], bk[2], bk[3]};
                    lds_put_row<NS, 4>(sBK, L::ROWP, (16 * ib + r16) * L::RS + 16 * db + 4 * g4, xv);
                }
            } else {
                // -L_ij for j < ib as D[s][t] (rows s of block j, columns t of block ib): its D layout
                // is the A-operand layout of L_ij (row t, K = s).
                for (int j = 0; j < ib; ++j) {
                    f32x4 lt = zero4();
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) {
                        const Split8<NX> kj = lds_frag<NX>(sK, L::ROWP, L::RS, 16 * j + r16, 32 * ks, g4);
                        lt = mfma_split<NX, NX, NX>(kj, kf[ks], lt);
                    }
                    const f32x4 bsb = *reinterpret_cast<const f32x4*>(sF + L::F_BSB + 16 * j + 4 * g4);
                    const float ncf = -sF[L::F_CF + 64 * j + 16 * ib + r16];
                    const float xv[4] = {lt[0] * (bsb[0] * ncf), lt[1] * (bsb[1] * ncf), lt[2] * (bsb[2] * ncf),
                                         lt[3] * (bsb[3] * ncf)};
                    frag_put<NS>(sXF, XF_BYTES, xfrag(j, ib), j & 1, lane, xv);
                }
            }
            // A^T tiles (sb = ib, tb >= ib): rows s of key block ib, columns t of query block tb,
            // beta_s e^{gam_t - gam_s}(q_t . k_s), kept for s <= t
            if constexpr (OUT) {
                const f32x4 gs = *reinterpret_cast<const f32x4*>(sF + L::F_G2 + 16 * ib + 4 * g4);
                const f32x4 bs = *reinterpret_cast<const f32x4*>(sF + L::F_B + 16 * ib + 4 * g4);
                const f32x4 bsb = *reinterpret_cast<const f32x4*>(sF + L::F_BSB + 16 * ib + 4 * g4);
                for (int tb = ib; tb < 4; ++tb) {
                    f32x4 acc = zero4();
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) {
                        const Split8<NX> qf = lds_frag<NX>(sQ, L::ROWP, L::RS, 16 * tb + r16, 32 * ks, g4);
                        acc = mfma_split<NX, NX, NX>(kf[ks], qf, acc);
                    }
                    float xv[4];
                    if (tb == ib) {
                        const float gt = sF[L::F_G2 + 16 * tb + r16];
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const float f = bs[j] * __builtin_amdgcn_exp2f(min0(gt - gs[j]));
                            xv[j] = (4 * g4 + j <= r16) ? acc[j] * f : 0.f;
                        }
                    } else {
                        const float cfa = sF[L::F_CFA + 64 * ib + 16 * tb + r16];
#pragma unroll
                        for (int j = 0; j < 4; ++j) xv[j] = acc[j] * (bsb[j] * cfa);
                    }
                    frag_put<NS>(sAF, AF_BYTES, afrag(ib >> 1, tb), ib & 1, lane, xv);
                }
            }
        }
        __syncthreads();

        // ---------------- stage 3: UT solve, outputs, state ----------------------------------
        const float eG = sF[L::F_MISC];
        auto pass = [&](auto with_v, f32x4 (&St)[4]) {
            constexpr bool WV = decltype(with_v)::value;
            Split8<NS> sf[2];  // S0 with K = key dims (B operand of S0, A operand of S0^T)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) sf[ks] = split_k32<NS>(St[2 * ks], St[2 * ks + 1]);
            // U_i in D layout: rows 16i + 4*g4 + k, column c0 + r16
            f32x4 U[4];
            Split4<NS> us[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                f32x4 acc = zero4();
                if constexpr (PRE) {
                    // T_ii V_i - Bk_i S0
                    if constexpr (WV)
                        acc = mfma16_split<NS, NX, NS>(frag_get4<NS>(sTF, TF_BYTES, tfrag(i), lane),
                                                       col_frag4<NX>(sV, L::ROWP, L::RS, 16 * i, c0, g4, r16), acc);
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks)
                        acc = mfma_split<NS, NS, NS>(lds_frag<NS>(sBK, L::ROWP, L::RS, 16 * i + r16, 32 * ks, g4),
                                                     sf[ks], acc);
                } else {
                    // R_i = V_i - e^{gamp} (K S0)_i
                    f32x4 p = zero4();
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks)
                        p = mfma_split<NX, NS, NS>(lds_frag<NX>(sK, L::ROWP, L::RS, 16 * i + r16, 32 * ks, g4), sf[ks],
                                                   p);
                    const f32x4 ep = *reinterpret_cast<const f32x4*>(sF + L::F_EGP + 16 * i + 4 * g4);
                    f32x4 vv = zero4();
                    if constexpr (WV) {
                        const Split4<NX> vf = col_frag4<NX>(sV, L::ROWP, L::RS, 16 * i, c0, g4, r16);
#pragma unroll
                        for (int pl = 0; pl < NX; ++pl)
#pragma unroll
                            for (int k = 0; k < 4; ++k) vv[k] += (float)vf.p[pl][k];
                    }
#pragma unroll
                    for (int k = 0; k < 4; ++k) acc[k] = vv[k] - ep[k] * p[k];
                }
                // - sum_{j<i} X_ij U_j (X = P with PRE, else L; stored negated)
                if (i == 1) {
                    acc = mfma16_split<NS, NS, NS>(frag_get4<NS>(sXF, XF_BYTES, xfrag(0, 1), lane), us[0], acc);
                } else if (i >= 2) {  // blocks 0 and 1 together (K = 32)
                    acc = mfma_split<NS, NS, NS>(frag_get8<NS>(sXF, XF_BYTES, xfrag(0, i), lane), join4<NS>(us[0], us[1]),
                                                 acc);
                    if (i == 3)
                        acc = mfma16_split<NS, NS, NS>(frag_get4<NS>(sXF, XF_BYTES, xfrag(2, 3), lane), us[2], acc);
                }
                if constexpr (!PRE)
                    acc = mfma16_split<NS, NS, NS>(frag_get4<NS>(sTF, TF_BYTES, tfrag(i), lane), split4<NS>(acc),
                                                   zero4());
                U[i] = acc;
                us[i] = split4<NS>(acc);
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
                    if (tb == 0) {
                        o = mfma16_split<NS, NS, NS>(us[0], frag_get4<NS>(sAF, AF_BYTES, afrag(0, 0), lane), o);
                    } else {
                        o = mfma_split<NS, NS, NS>(join4<NS>(us[0], us[1]),
                                                   frag_get8<NS>(sAF, AF_BYTES, afrag(0, tb), lane), o);
                        if (tb == 2)
                            o = mfma16_split<NS, NS, NS>(us[2], frag_get4<NS>(sAF, AF_BYTES, afrag(1, 2), lane), o);
                        if (tb == 3)
                            o = mfma_split<NS, NS, NS>(join4<NS>(us[2], us[3]),
                                                       frag_get8<NS>(sAF, AF_BYTES, afrag(1, 3), lane), o);
                    }
                    Ot[tb] = o;
                }
                // stage through this wave's area and store quad-coalesced rows
                const int es = OBF ? 2 : dt_size(x.o_dt);
                char* obase = x.op + tc * x.ost + c0 * es;
                const int q = lane & 3, tq = (lane >> 4) + 4 * ((lane >> 2) & 3);
                const int32_t olane = (int32_t)(tq * x.ost) + 4 * q * es;
                const OutRsrc orr = out_rsrc(obase, x.ost, es, nv, !OBF && x.o_dt == DT_F32);
                wait_vmem();  // the next chunk's loads have landed: later waits skip these stores
#pragma unroll
                for (int tb = 0; tb < 4; ++tb) {
                    *reinterpret_cast<f32x4*>(sWS + r16 * L::OS + 4 * g4) = Ot[tb];
                    const f32x4 xo = *reinterpret_cast<const f32x4*>(sWS + tq * L::OS + 4 * q);
                    const int32_t vo = (int32_t)(16 * tb * x.ost) + olane;
                    if constexpr (OBF) {
                        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
                        const u32x2 w = {pk_bf16(xo[0], xo[1]), pk_bf16(xo[2], xo[3])};
                        __builtin_amdgcn_raw_buffer_store_b64(w, orr.lo, vo, 0, 0);
                    } else {
                        out_store4(orr, vo, x.o_dt, xo);
                    }
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
            if (!skip_m) pass(std::false_type{}, S);
            __builtin_amdgcn_sched_barrier(0);  // one pass at a time: their temporaries never overlap
            pass(std::true_type{}, SN);
        }
        __syncthreads();  // the next chunk rewrites LDS
    }
};

template <typename TIn, bool OUT, bool CK, bool OBF, bool PRE>
__device__ void sg_walk(const PrefillParams& a, const Work& wk, int64_t h, f32x4 (&S)[4], f32x4 (&SN)[4], bool skip_m,
                        char* smem) {
    using St = SgStep<TIn, OUT, CK, OBF, PRE>;
    const int lane = threadIdx.x & 63, wave = wave_id(), tg = lane >> 2, row = lane & 3;
    const SgCtx x = sg_ctx<OUT, TIn>(a, wk, h, tg, wave * 16 + 4 * row);
    const int64_t t_end = wk.t_end;
    const int64_t nch = (t_end - wk.t_begin + CHUNK - 1) / CHUNK;
    auto chunk_nv = [&](int64_t tc) {
        const int64_t r = t_end - tc;
        return (int)(r < CHUNK ? r : CHUNK);
    };
    SIn<TIn> A;
    int64_t tc = wk.t_begin;
    sg_load<OUT, CK>(A, x, tc, chunk_nv(tc), true);
    for (int64_t c = 0; c < nch; ++c, tc += CHUNK)
        St::run(x, tc, chunk_nv(tc), A, S, SN, skip_m, smem, [&] {
            const bool more = c + 1 < nch;
            sg_load<OUT, CK>(A, x, tc + CHUNK, more ? chunk_nv(tc + CHUNK) : 0, more);
        });
}

// Workgroups per CU the launch bounds ask for: two where the LDS allows, else one.  The 16-bit
// kernels' LDS would fit three, but at two the registers grow to 169-182 with no spill, the plan
// takes 21 segments of 6-7 chunks per config-3 sequence instead of 32 of 4, and with the stage
// priorities of SgStep::run the two workgroups of a CU interleave their phases: config 3 0.1258 ->
// 0.1214 ms per pass, same-box A/B (at three per CU the priorities gained nothing).
template <typename Lay>
constexpr int sg_occupancy() {
    return 2 * Lay::BYTES <= 160 * 1024 ? 2 : 1;
}

// K1: the segment map driven from [I | 0] with V = 0 (-> M_p) and from 0 with the real V (-> N_p).
// A sequence's first segment without an initial state carries in zero: its M stays I and only N
// runs.
template <typename TIn, bool CK>
__global__ __launch_bounds__(256, (sg_occupancy<SLay<TIn, false, true>>())) void gdn_sg_seg_mn_kernel(PrefillParams a) {
    using L = SLay<TIn, false, true>;
    __shared__ __attribute__((aligned(16))) char smem[L::BYTES];
    const int64_t w = blockIdx.x, h = blockIdx.y;
    Work wk;
    if (!find_work(a, w, wk)) return;
    f32x4 M[4], N[4];
    init_seg_map(M, N);
    sg_walk<TIn, false, CK, false, true>(a, wk, h, M, N, wk.p == 0 && a.s0 == nullptr, smem);
    store_seg_map<Prec<TIn>::NS>(a, w, h, M, N);
}

// K3: outputs of one segment from S_in[p] (in the N slot after the scan).  OBF: bf16 output.
template <typename TIn, bool CK, bool OBF>
__global__ __launch_bounds__(256, (sg_occupancy<SLay<TIn, true, false>>())) void gdn_sg_seg_out_kernel(PrefillParams a) {
    using L = SLay<TIn, true, false>;
    __shared__ __attribute__((aligned(16))) char smem[L::BYTES];
    const int64_t w = blockIdx.x, h = blockIdx.y;
    Work wk;
    if (!find_work(a, w, wk)) return;
    f32x4 S[4];
    load_seg_state(a, w, h, S);
    sg_walk<TIn, true, CK, OBF, false>(a, wk, h, S, S, false, smem);
}

// ---------------------------------------------------------------------------------------
// Host launchers.
// ---------------------------------------------------------------------------------------
template <typename TIn, bool CK>
static hipError_t launch_sg_ck(const PrefillParams& a, int64_t n_work, int which, hipStream_t stream) {
    const dim3 grid((unsigned)n_work, (unsigned)a.H);
    if (which == 0) hipLaunchKernelGGL((gdn_sg_seg_mn_kernel<TIn, CK>), grid, dim3(256), 0, stream, a);
    else if (a.o_dt == DT_BF16) hipLaunchKernelGGL((gdn_sg_seg_out_kernel<TIn, CK, true>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((gdn_sg_seg_out_kernel<TIn, CK, false>), grid, dim3(256), 0, stream, a);
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
// checked row addressing, launched unless T % 4 == 0; the output dtype does not change the
// kernel's LDS, and the bf16-output instance is the one queried).
int gdn_sg_seg_out_blocks_per_cu(int io_dt, bool ck) {
    const void* k =
        io_dt == DT_F16 ? (ck ? reinterpret_cast<const void*>(gdn_sg_seg_out_kernel<_Float16, true, true>)
                              : reinterpret_cast<const void*>(gdn_sg_seg_out_kernel<_Float16, false, true>))
        : io_dt == DT_F32 ? (ck ? reinterpret_cast<const void*>(gdn_sg_seg_out_kernel<float, true, true>)
                                : reinterpret_cast<const void*>(gdn_sg_seg_out_kernel<float, false, true>))
                          : (ck ? reinterpret_cast<const void*>(gdn_sg_seg_out_kernel<__bf16, true, true>)
                                : reinterpret_cast<const void*>(gdn_sg_seg_out_kernel<__bf16, false, true>));
    int nb = 0;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k, 256, 0);
    return (e == hipSuccess && nb > 0) ? nb : 1;
}

}  // namespace triune
