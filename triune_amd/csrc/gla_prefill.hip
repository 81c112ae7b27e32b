// gla_prefill.hip -- chunked GLA prefill for gfx950 (dense [B,T,H,D] and packed varlen).
//
// Semantics (reference: triune/kernels/fast_gla.py:569-689 _run_gla_chunks, :206-316 the
// Triton TC kernel, :692-778 fast_chunk_gla dispatch):
//   S_t = diag(exp(min(g_t, 0))) S_{t-1} + k_t v_t^T ,   o_t = S_t^T q_t
// for every (sequence, head), starting from S0 (or zero), returning every o_t and S_T.
//
// Work decomposition.  A sequence is cut into segments of P chunks of 64 tokens.
//   K1 seg_state : per (segment, head, Dv slice) the segment's local end state from zero,
//                  L = sum over its tokens, and the segment's summed log-decay.
//   K2 (recurrent_scan.hip): exclusive affine scan over the segments of each (sequence, head)
//                  S_in[p+1] = exp(Gseg_p) * S_in[p] + L_p, written in place of L; final state.
//   K3 seg_output: per (segment, head, Dv slice) walks its chunks from S_in[p], writes o.
// Within a chunk (C = 64 tokens, G = inclusive cumulative log-decay from the chunk start,
// m = G_C / 2 per key dim):
//   Qt = q * exp(G - m), Kt = k * exp(m - G)         (|exponents| <= span/2)
//   A^T[s][t] = sum_d Kt[s][d] Qt[t][d]  for s <= t  (causal, diagonal included)
//   O^T = (exp(m) * S)^T Qt^T + V^T A^T
//   S  <- exp(G_C) * S + exp(m) * (Kt^T V)
// Products run on v_mfma_f32_16x16x32_bf16.  Operands that are not exactly bf16 are split
// into 2 (16-bit I/O) or 3 (fp32 I/O) bf16 parts and the part products with combined order
// below the split depth are accumulated in fp32.  Chunks whose key-dim decay span exceeds
// SPAN_MAX (or that hold the reference's unclamped 1-token tail) run token by token.
#include "kernels.h"

namespace triune {

constexpr int CHUNK = 64;
constexpr float SPAN_MAX = 64.f;

struct Work {
    int64_t seq, b, row0, t_begin, t_end, len;
    int p;
};

__device__ __forceinline__ bool find_work(const PrefillParams& a, int64_t w, Work& wk) {
    if (!a.varlen) {
        int64_t seq = w / a.nseg_dense;
        if (seq >= a.n_seqs) return false;
        wk.seq = seq;
        wk.b = seq;
        wk.row0 = 0;
        wk.p = (int)(w - seq * a.nseg_dense);
        wk.len = a.T;
    } else {
        int64_t total = a.seg_off[a.n_seqs];
        if (w >= total) return false;
        int64_t lo = 0, hi = a.n_seqs - 1;  // largest seq with seg_off[seq] <= w
        while (lo < hi) {
            int64_t mid = (lo + hi + 1) >> 1;
            if (a.seg_off[mid] <= w) lo = mid;
            else hi = mid - 1;
        }
        wk.seq = lo;
        wk.b = 0;
        wk.row0 = a.cu[lo];
        wk.p = (int)(w - a.seg_off[lo]);
        wk.len = (int64_t)a.cu[lo + 1] - (int64_t)a.cu[lo];
    }
    wk.t_begin = (int64_t)wk.p * a.P * CHUNK;
    wk.t_end = wk.t_begin + (int64_t)a.P * CHUNK;
    if (wk.t_end > wk.len) wk.t_end = wk.len;
    return wk.t_begin < wk.t_end;
}

template <typename T>
__device__ __forceinline__ const T* tok_ptr(const TokTensor& x, const Work& wk, int64_t t, int64_t h,
                                            int d) {
    return reinterpret_cast<const T*>(x.p) + wk.b * x.sb + (wk.row0 + t) * x.st + h * x.sh + d;
}

__device__ __forceinline__ const void* tok_ptr_dt(const TokTensor& x, int dt, const Work& wk, int64_t t,
                                                  int64_t h, int d) {
    int64_t off = wk.b * x.sb + (wk.row0 + t) * x.st + h * x.sh + d;
    return reinterpret_cast<const char*>(x.p) + off * dt_size(dt);
}

// Number of bf16 parts that hold an input element exactly / that derived operands carry.
template <typename T> struct Prec;
template <> struct Prec<__bf16> { static constexpr int NX = 1, NS = 2; };
template <> struct Prec<_Float16> { static constexpr int NX = 2, NS = 2; };
template <> struct Prec<float> { static constexpr int NX = 3, NS = 3; };

// Permutation matrix used as B operand to transpose an A-operand fragment: lane (g4, r16)
// holds 1 in slot j iff column 8*g4 + j of the A fragment's 32-column group is the column
// that label r16 of a 16-column block of parity par maps to:
//   label(16*cb + n) -> column 32*(cb >> 1) + 8*(n >> 2) + 4*(cb & 1) + (n & 3).
__device__ __forceinline__ bf16x8 perm_frag(int par, int g4, int r16) {
    bf16x8 f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
        f[j] = (__bf16)((g4 == (r16 >> 2) && j == 4 * par + (r16 & 3)) ? 1.f : 0.f);
    return f;
}

__device__ __forceinline__ int label_col(int blk, int n) {  // see perm_frag
    return 32 * (blk >> 1) + 8 * (n >> 2) + 4 * (blk & 1) + (n & 3);
}

// Two accumulator tiles (rows 4*g4+i of tiles lo, hi) as the eight K slots of a fragment.
template <int N>
__device__ __forceinline__ Split8<N> frag_from_tiles(const f32x4& lo, const f32x4& hi, float scale_lo[4],
                                                     float scale_hi[4]) {
    float x[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        x[i] = lo[i] * scale_lo[i];
        x[4 + i] = hi[i] * scale_hi[i];
    }
    return split8<N>(x);
}

__device__ __forceinline__ bf16x8 frag_exact(const f32x4& lo, const f32x4& hi) {
    bf16x8 f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[i] = (__bf16)lo[i];
        f[4 + i] = (__bf16)hi[i];
    }
    return f;
}

// Chunk totals of clamped g for the lane's dims (32*ks + 8*g4 + j); returns whether the chunk
// can take the factored MFMA path (wave-uniform).
template <int NKS>
__device__ __forceinline__ bool chunk_totals(const PrefillParams& a, const Work& wk, int64_t h, int64_t tc,
                                             int nv, int g4, int r16, int lane, float (&GC)[NKS][8],
                                             bool tail_unclamped) {
    bool bad = tail_unclamped;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
        float tot[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) tot[j] = 0.f;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
            int t = 16 * mb + r16;
            float gx[8];
            load8_dt(tok_ptr_dt(a.g, a.g_dt, wk, tc + t, h, 32 * ks + 8 * g4), a.g_dt, t < nv, gx);
#pragma unroll
            for (int j = 0; j < 8; ++j) tot[j] += fminf(gx[j], 0.f);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            float s = row_inclusive_scan(tot[j]);
            GC[ks][j] = lane_bcast(s, (lane & 48) | 15);
            bad |= !(GC[ks][j] >= -SPAN_MAX);
        }
    }
    return !__any(bad);
}

// Inclusive cumulative clamped log-decay for the four 16-token blocks of one dim k-step.
__device__ __forceinline__ void chunk_cumsum(float (&gx)[4][8], int lane) {
    float carry[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) carry[j] = 0.f;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            float s = row_inclusive_scan(fminf(gx[mb][j], 0.f));
            gx[mb][j] = s + carry[j];
            if (mb < 3) carry[j] += lane_bcast(s, (lane & 48) | 15);
        }
    }
}

// Token-by-token chunk update (large decay spans, unclamped tail).  S tile (db, jb) element i
// is S[dim 32*(db>>1) + 8*g4 + 4*(db&1) + i][col v0 + label_col(jb, r16)].
template <typename TIn, int DK, int DVS, bool WITH_OUT>
__device__ void chunk_tokenwise(const PrefillParams& a, const Work& wk, int64_t h, int v0, int64_t tc, int nv,
                                int g4, int r16, f32x4 (&S)[DK / 16][DVS / 16]) {
    constexpr int NKS = DK / 32, NDB = DK / 16, NJB = DVS / 16;
    for (int t = 0; t < nv; ++t) {
        int64_t tt = tc + t;
        bool unclamped = (a.flags & 1) && (tt == wk.len - 1);
        float gq[NKS][8], kq[NKS][8], qq[NKS][8];
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
            load8_dt(tok_ptr_dt(a.g, a.g_dt, wk, tt, h, 32 * ks + 8 * g4), a.g_dt, true, gq[ks]);
            load8<TIn>(tok_ptr<TIn>(a.k, wk, tt, h, 32 * ks + 8 * g4), true, kq[ks]);
            if (WITH_OUT) load8<TIn>(tok_ptr<TIn>(a.q, wk, tt, h, 32 * ks + 8 * g4), true, qq[ks]);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                float gg = unclamped ? gq[ks][j] : fminf(gq[ks][j], 0.f);
                gq[ks][j] = expf(gg);
            }
        }
        float vv[NJB];
        const TIn* vrow = tok_ptr<TIn>(a.v, wk, tt, h, v0);
#pragma unroll
        for (int jb = 0; jb < NJB; ++jb) vv[jb] = (float)vrow[label_col(jb, r16)];
        float part[NJB];
#pragma unroll
        for (int jb = 0; jb < NJB; ++jb) part[jb] = 0.f;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int jb = 0; jb < NJB; ++jb)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    int ks = db >> 1, j = 4 * (db & 1) + i;
                    float s = gq[ks][j] * S[db][jb][i] + kq[ks][j] * vv[jb];
                    S[db][jb][i] = s;
                    if (WITH_OUT) part[jb] += qq[ks][j] * s;
                }
        if (WITH_OUT) {
#pragma unroll
            for (int jb = 0; jb < NJB; ++jb) {
                float x = part[jb];
                x += __shfl_xor(x, 16);
                x += __shfl_xor(x, 32);
                part[jb] = x;
            }
            if (g4 == 0) {
                char* orow = reinterpret_cast<char*>(a.o) +
                             (wk.b * a.o_sb + (wk.row0 + tt) * a.o_st + h * a.o_sh + v0) * dt_size(a.o_dt);
#pragma unroll
                for (int jb = 0; jb < NJB; ++jb) {
                    int col = label_col(jb, r16);
                    if (a.o_dt == DT_F32) reinterpret_cast<float*>(orow)[col] = part[jb];
                    else if (a.o_dt == DT_BF16) reinterpret_cast<__bf16*>(orow)[col] = (__bf16)part[jb];
                    else reinterpret_cast<_Float16*>(orow)[col] = (_Float16)part[jb];
                }
            }
        }
    }
}

// One segment: walk its chunks from S (in registers), optionally writing outputs.
template <typename TIn, int DK, int DVS, bool WITH_OUT>
__device__ void segment_walk(const PrefillParams& a, const Work& wk, int64_t h, int v0,
                             f32x4 (&S)[DK / 16][DVS / 16], float (&Gseg)[DK / 32][8]) {
    constexpr int NKS = DK / 32, NDB = DK / 16, NJB = DVS / 16, NVC = DVS / 32;
    constexpr int NX = Prec<TIn>::NX, NS = Prec<TIn>::NS;
    const int lane = threadIdx.x & 63, r16 = lane & 15, g4 = lane >> 4;
    const bf16x8 perm0 = perm_frag(0, g4, r16), perm1 = perm_frag(1, g4, r16);

    for (int64_t tc = wk.t_begin; tc < wk.t_end; tc += CHUNK) {
        const int nv = (int)((wk.t_end - tc) < CHUNK ? (wk.t_end - tc) : CHUNK);
        const bool tail_unclamped = (a.flags & 1) && (tc + nv == wk.len);
        float GC[NKS][8];
        const bool fast = chunk_totals<NKS>(a, wk, h, tc, nv, g4, r16, lane, GC, tail_unclamped);
        if (!fast) {
            chunk_tokenwise<TIn, DK, DVS, WITH_OUT>(a, wk, h, v0, tc, nv, g4, r16, S);
            // GC holds clamped totals; an unclamped tail token adds its positive part back.
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
                float gx[8];
                load8_dt(tok_ptr_dt(a.g, a.g_dt, wk, wk.len - 1, h, 32 * ks + 8 * g4), a.g_dt, tail_unclamped, gx);
#pragma unroll
                for (int j = 0; j < 8; ++j) Gseg[ks][j] += GC[ks][j] + fmaxf(gx[j], 0.f);
            }
            continue;
        }

        // ---- V: row fragments -> transposed fragments (tokens along K) -------------------
        // vf[p][jb][ks2]: lane holds V[token 32*ks2 + pi(g4, j)][col v0 + label_col(jb, r16)]
        Split8<NX> vf[NJB][2];
        {
            f32x4 vt[NX][NJB][4];
#pragma unroll
            for (int c = 0; c < NVC; ++c)
#pragma unroll
                for (int mb = 0; mb < 4; ++mb) {
                    int t = 16 * mb + r16;
                    float x[8];
                    load8<TIn>(tok_ptr<TIn>(a.v, wk, tc + t, h, v0 + 32 * c + 8 * g4), t < nv, x);
                    Split8<NX> xs = split8<NX>(x);
#pragma unroll
                    for (int pp = 0; pp < NX; ++pp) {
                        vt[pp][2 * c][mb] = mfma(xs.p[pp], perm0, zero4());
                        vt[pp][2 * c + 1][mb] = mfma(xs.p[pp], perm1, zero4());
                    }
                }
#pragma unroll
            for (int jb = 0; jb < NJB; ++jb)
#pragma unroll
                for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
                    for (int pp = 0; pp < NX; ++pp) vf[jb][k2].p[pp] = frag_exact(vt[pp][jb][2 * k2], vt[pp][jb][2 * k2 + 1]);
        }

        f32x4 At[4][4];  // At[sb][tb], used for sb <= tb
        f32x4 Ot[NJB][4];
        if (WITH_OUT) {
#pragma unroll
            for (int sb = 0; sb < 4; ++sb)
#pragma unroll
                for (int tb = 0; tb < 4; ++tb) At[sb][tb] = zero4();
#pragma unroll
            for (int jb = 0; jb < NJB; ++jb)
#pragma unroll
                for (int tb = 0; tb < 4; ++tb) Ot[jb][tb] = zero4();
        }

#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
            float G[4][8], kx[4][8];
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) {
                int t = 16 * mb + r16;
                load8_dt(tok_ptr_dt(a.g, a.g_dt, wk, tc + t, h, 32 * ks + 8 * g4), a.g_dt, t < nv, G[mb]);
                load8<TIn>(tok_ptr<TIn>(a.k, wk, tc + t, h, 32 * ks + 8 * g4), t < nv, kx[mb]);
            }
            chunk_cumsum(G, lane);
            float m[8], em[8], eG[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                m[j] = 0.5f * GC[ks][j];
                em[j] = fast_exp(m[j]);
                eG[j] = em[j] * em[j];
                Gseg[ks][j] += GC[ks][j];
            }
            // key side Kt = k * exp(m - G)
            Split8<NS> kt[4];
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) {
                float x[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) x[j] = kx[mb][j] * fast_exp(m[j] - G[mb][j]);
                kt[mb] = split8<NS>(x);
            }

            if (WITH_OUT) {
                Split8<NS> qt[4];
#pragma unroll
                for (int mb = 0; mb < 4; ++mb) {
                    int t = 16 * mb + r16;
                    float x[8];
                    load8<TIn>(tok_ptr<TIn>(a.q, wk, tc + t, h, 32 * ks + 8 * g4), t < nv, x);
#pragma unroll
                    for (int j = 0; j < 8; ++j) x[j] *= fast_exp(G[mb][j] - m[j]);
                    qt[mb] = split8<NS>(x);
                }
                // A^T[sb][tb] += Kt[sb] Qt[tb]^T
#pragma unroll
                for (int sb = 0; sb < 4; ++sb)
#pragma unroll
                    for (int tb = sb; tb < 4; ++tb) At[sb][tb] = mfma_split<NS, NS, NS>(kt[sb], qt[tb], At[sb][tb]);
                // O^T[jb][tb] += (exp(m) S)^T[jb] Qt[tb]^T over this k-step's dims
#pragma unroll
                for (int jb = 0; jb < NJB; ++jb) {
                    float slo[4], shi[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        slo[i] = em[i];
                        shi[i] = em[4 + i];
                    }
                    Split8<NS> sf = frag_from_tiles<NS>(S[2 * ks][jb], S[2 * ks + 1][jb], slo, shi);
#pragma unroll
                    for (int tb = 0; tb < 4; ++tb) Ot[jb][tb] = mfma_split<NS, NS, NS>(sf, qt[tb], Ot[jb][tb]);
                }
            }

            // Kt^T fragments for dim blocks 2ks, 2ks+1 (tokens along K), then the state rows.
#pragma unroll
            for (int dl = 0; dl < 2; ++dl) {
                const bf16x8& pm = dl ? perm1 : perm0;
                Split8<NS> ktT[2];
#pragma unroll
                for (int pp = 0; pp < NS; ++pp) {
                    f32x4 tt[4];
#pragma unroll
                    for (int mb = 0; mb < 4; ++mb) tt[mb] = mfma(kt[mb].p[pp], pm, zero4());
                    ktT[0].p[pp] = frag_exact(tt[0], tt[1]);
                    ktT[1].p[pp] = frag_exact(tt[2], tt[3]);
                }
                const int db = 2 * ks + dl;
#pragma unroll
                for (int jb = 0; jb < NJB; ++jb) {
                    f32x4 P = zero4();
#pragma unroll
                    for (int k2 = 0; k2 < 2; ++k2) P = mfma_split<NS, NX, NS>(ktT[k2], vf[jb][k2], P);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        int j = 4 * dl + i;
                        S[db][jb][i] = eG[j] * S[db][jb][i] + em[j] * P[i];
                    }
                }
            }
        }

        if (WITH_OUT) {
            // causal mask on diagonal tiles: row s = 4*g4 + i (key), column t = r16 (query)
#pragma unroll
            for (int tb = 0; tb < 4; ++tb)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (4 * g4 + i > r16) At[tb][tb][i] = 0.f;
            // O^T += V^T A^T
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) {
#pragma unroll
                for (int k2 = 0; k2 < 2; ++k2) {
                    if (2 * k2 > tb) continue;
                    float one[4] = {1.f, 1.f, 1.f, 1.f};
                    f32x4 hiTile = (2 * k2 + 1 <= tb) ? At[2 * k2 + 1][tb] : zero4();
                    Split8<NS> af = frag_from_tiles<NS>(At[2 * k2][tb], hiTile, one, one);
#pragma unroll
                    for (int jb = 0; jb < NJB; ++jb) Ot[jb][tb] = mfma_split<NX, NS, NS>(vf[jb][k2], af, Ot[jb][tb]);
                }
            }
            // store: lane holds O[token 16*tb + r16][cols v0 + 32*c + 8*g4 + 0..7]
            char* obase = reinterpret_cast<char*>(a.o);
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) {
                int t = 16 * tb + r16;
                if (t >= nv) continue;
#pragma unroll
                for (int c = 0; c < NVC; ++c) {
                    float x[8];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        x[i] = Ot[2 * c][tb][i];
                        x[4 + i] = Ot[2 * c + 1][tb][i];
                    }
                    int64_t off = wk.b * a.o_sb + (wk.row0 + tc + t) * a.o_st + h * a.o_sh + v0 + 32 * c + 8 * g4;
                    store8_dt(obase + off * dt_size(a.o_dt), a.o_dt, x);
                }
            }
        }
    }
}

template <int DK, int DVS>
__device__ __forceinline__ int64_t state_index(int db, int jb, int i, int g4, int r16, int v0, int Dv) {
    int dim = 32 * (db >> 1) + 8 * g4 + 4 * (db & 1) + i;
    int col = v0 + label_col(jb, r16);
    return (int64_t)dim * Dv + col;
}

// K1: local end state of each segment (from zero) and its summed log-decay.
template <typename TIn, int DK, int DVS>
__global__ __launch_bounds__(64) void gla_seg_state_kernel(PrefillParams a) {
    const int64_t w = blockIdx.x;
    const int64_t h = blockIdx.y;
    const int v0 = blockIdx.z * DVS;
    Work wk;
    if (!find_work(a, w, wk)) return;
    const int lane = threadIdx.x & 63, r16 = lane & 15, g4 = lane >> 4;
    f32x4 S[DK / 16][DVS / 16];
    float Gseg[DK / 32][8];
#pragma unroll
    for (int db = 0; db < DK / 16; ++db)
#pragma unroll
        for (int jb = 0; jb < DVS / 16; ++jb) S[db][jb] = zero4();
#pragma unroll
    for (int ks = 0; ks < DK / 32; ++ks)
#pragma unroll
        for (int j = 0; j < 8; ++j) Gseg[ks][j] = 0.f;
    segment_walk<TIn, DK, DVS, false>(a, wk, h, v0, S, Gseg);
    float* st = a.ws_state + (w * a.H + h) * (int64_t)a.Dk * a.Dv;
#pragma unroll
    for (int db = 0; db < DK / 16; ++db)
#pragma unroll
        for (int jb = 0; jb < DVS / 16; ++jb)
#pragma unroll
            for (int i = 0; i < 4; ++i) st[state_index<DK, DVS>(db, jb, i, g4, r16, v0, a.Dv)] = S[db][jb][i];
    if (blockIdx.z == 0 && r16 == 0) {
        float* gs = a.ws_gamma + (w * a.H + h) * (int64_t)a.Dk;
#pragma unroll
        for (int ks = 0; ks < DK / 32; ++ks)
#pragma unroll
            for (int j = 0; j < 8; ++j) gs[32 * ks + 8 * g4 + j] = Gseg[ks][j];
    }
}

// K3: outputs of each segment from its carried-in state (ws_state after the scan).
template <typename TIn, int DK, int DVS>
__global__ __launch_bounds__(64) void gla_seg_output_kernel(PrefillParams a) {
    const int64_t w = blockIdx.x;
    const int64_t h = blockIdx.y;
    const int v0 = blockIdx.z * DVS;
    Work wk;
    if (!find_work(a, w, wk)) return;
    const int lane = threadIdx.x & 63, r16 = lane & 15, g4 = lane >> 4;
    f32x4 S[DK / 16][DVS / 16];
    float Gseg[DK / 32][8];
    const float* st = a.ws_state + (w * a.H + h) * (int64_t)a.Dk * a.Dv;
#pragma unroll
    for (int db = 0; db < DK / 16; ++db)
#pragma unroll
        for (int jb = 0; jb < DVS / 16; ++jb)
#pragma unroll
            for (int i = 0; i < 4; ++i) S[db][jb][i] = st[state_index<DK, DVS>(db, jb, i, g4, r16, v0, a.Dv)];
#pragma unroll
    for (int ks = 0; ks < DK / 32; ++ks)
#pragma unroll
        for (int j = 0; j < 8; ++j) Gseg[ks][j] = 0.f;
    segment_walk<TIn, DK, DVS, true>(a, wk, h, v0, S, Gseg);
}

// K0 (varlen): segment offsets from cu_seqlens, one thread block.
__global__ __launch_bounds__(256) void gla_varlen_plan_kernel(const int32_t* cu, int64_t n_seqs, int P,
                                                               int32_t* seg_off) {
    // serial prefix over sequences in chunks of 256 (n_seqs is small: a batch of requests)
    __shared__ int32_t part[256];
    int32_t base = 0;
    if (threadIdx.x == 0) seg_off[0] = 0;
    for (int64_t s0 = 0; s0 < n_seqs; s0 += 256) {
        int64_t s = s0 + threadIdx.x;
        int32_t n = 0;
        if (s < n_seqs) {
            int64_t len = (int64_t)cu[s + 1] - (int64_t)cu[s];
            int64_t chunks = (len + CHUNK - 1) / CHUNK;
            n = (int32_t)((chunks + P - 1) / P);
        }
        part[threadIdx.x] = n;
        __syncthreads();
        for (int off = 1; off < 256; off <<= 1) {
            int32_t add = threadIdx.x >= off ? part[threadIdx.x - off] : 0;
            __syncthreads();
            part[threadIdx.x] += add;
            __syncthreads();
        }
        if (s < n_seqs) seg_off[s + 1] = base + part[threadIdx.x];
        base += part[255];
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------------------
// Host launchers.
// ---------------------------------------------------------------------------------------
int prefill_dv_slice(int Dk, int Dv) {
    if (Dk == 64 && Dv % 64 == 0) return 64;
    return 32;
}

template <typename TIn>
static hipError_t launch_seg_t(const PrefillParams& a, int64_t n_work, int dvs, bool with_out, hipStream_t stream) {
    dim3 grid((unsigned)n_work, (unsigned)a.H, (unsigned)(a.Dv / dvs));
    dim3 block(64);
#define TRIUNE_SEG_CASE(DK_, DVS_)                                                                      \
    if (a.Dk == DK_ && dvs == DVS_) {                                                                   \
        if (with_out) hipLaunchKernelGGL((gla_seg_output_kernel<TIn, DK_, DVS_>), grid, block, 0, stream, a); \
        else hipLaunchKernelGGL((gla_seg_state_kernel<TIn, DK_, DVS_>), grid, block, 0, stream, a);          \
        return hipGetLastError();                                                                       \
    }
    TRIUNE_SEG_CASE(64, 64)
    TRIUNE_SEG_CASE(64, 32)
    TRIUNE_SEG_CASE(128, 32)
    TRIUNE_SEG_CASE(32, 32)
#undef TRIUNE_SEG_CASE
    return hipErrorInvalidValue;
}

static hipError_t launch_seg(const PrefillParams& a, int64_t n_work, int dvs, int io_dt, bool with_out,
                             hipStream_t stream) {
    if (io_dt == DT_BF16) return launch_seg_t<__bf16>(a, n_work, dvs, with_out, stream);
    if (io_dt == DT_F16) return launch_seg_t<_Float16>(a, n_work, dvs, with_out, stream);
    if (io_dt == DT_F32) return launch_seg_t<float>(a, n_work, dvs, with_out, stream);
    return hipErrorInvalidValue;
}

hipError_t launch_gla_seg_state(const PrefillParams& a, int64_t n_work, int dvs, int io_dt, hipStream_t stream) {
    return launch_seg(a, n_work, dvs, io_dt, false, stream);
}

hipError_t launch_gla_seg_output(const PrefillParams& a, int64_t n_work, int dvs, int io_dt, hipStream_t stream) {
    return launch_seg(a, n_work, dvs, io_dt, true, stream);
}

hipError_t launch_gla_varlen_plan(const int32_t* cu, int64_t n_seqs, int P, int32_t* seg_off, hipStream_t stream) {
    hipLaunchKernelGGL(gla_varlen_plan_kernel, dim3(1), dim3(256), 0, stream, cu, n_seqs, P, seg_off);
    return hipGetLastError();
}

}  // namespace triune
