/*
 * gla_oracle.c -- fp64 CPU restatement of the reference's GLA / Gated DeltaNet
 * arithmetic.  TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, as the checker.  Nothing in
 * triune_amd/ links, imports or calls it; the product path is the HIP library.
 *
 * Every function computes in double precision from the caller's (already rounded)
 * inputs, so the GPU kernels and the oracle consume identical values.
 *
 * Layouts (all contiguous, row-major):
 *   token tensors  q,k,g : [B, T, H, Dk]     v,o : [B, T, H, Dv]
 *   packed (varlen) tokens: [N_tok, H, D], sequence i owns rows [cu[i], cu[i+1])
 *   states S             : [B, H, Dk, Dv]    S[b,h,i,j], i = key index, j = value index
 *
 * Reference anchors (paths under the reference repository):
 *   GLA token recurrence     tests/test_attention_fallback.py:12-24, tests/test_kernels.py:270-277
 *                            S_t = diag(exp g_t) S_{t-1} + k_t v_t^T ,  o_t = S_t^T q_t
 *   g <= 0 clamp in prefill  triune/kernels/fast_gla.py:586 (_run_gla_chunks), :278 (Triton TC)
 *   no clamp at T == 1 and   triune/kernels/fast_gla.py:746-753 (T == 1 decode branch),
 *   for a 1-token remainder  triune/kernels/fast_gla.py:768-775 (T_rem == 1 branch)
 *   decode step              triune/kernels/fast_gla.py:746-753, csrc/engine/engine.cpp:419-475,
 *                            csrc/kernels/gla.cu:23-75
 *   exclusive affine scan    triune/kernels/fast_gla.py:34-64 (_recurrent_scan_fwd),
 *                            tests/test_kernels.py:236-243
 *   Gated DeltaNet variant   triune/kernels/fast_gla.py:781-836 (fast_recurrent_gated_deltanet),
 *                            :453-471 (Triton per-token loop, beta over value dim)
 *   varlen                   absent from the reference; defined as one independent GLA
 *                            recurrence per packed sequence with its own initial state.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define ORACLE_API __attribute__((visibility("default")))

/* Whether token t of a length-T call of fast_chunk_gla clamps g at 0.
 * fast_gla.py:746-753: T == 1 takes the decode branch (no clamp).
 * fast_gla.py:768-775: a remainder of exactly one token after >= 1 full chunk
 * takes the same unclamped decode expression.  Every other token goes through
 * _run_gla_chunks (clamp at :586) or the Triton TC kernel (clamp at :278). */
static int clamp_token(long t, long T, long chunk) {
    if (T == 1) return 0;
    if (chunk > 0 && T > chunk && (T % chunk) == 1 && t == T - 1) return 0;
    return 1;
}

/* One (sequence, head) GLA recurrence over n tokens.
 * q,k,g advance by tok_stride_k per token, v,o by tok_stride_v. */
static void gla_one_head(const double* q, const double* k, const double* v, const double* g,
                         long n, long tok_stride_k, long tok_stride_v, int Dk, int Dv,
                         const double* s0, double* o, double* s_out, long clamp_T, long chunk,
                         int clamp_mode) {
    double* S = (double*)malloc(sizeof(double) * (size_t)Dk * Dv);
    if (s0) memcpy(S, s0, sizeof(double) * (size_t)Dk * Dv);
    else memset(S, 0, sizeof(double) * (size_t)Dk * Dv);
    for (long t = 0; t < n; ++t) {
        const double* qt = q + t * tok_stride_k;
        const double* kt = k + t * tok_stride_k;
        const double* gt = g + t * tok_stride_k;
        const double* vt = v + t * tok_stride_v;
        int do_clamp = clamp_mode == 1 ? 1 : (clamp_mode == 0 ? 0 : clamp_token(t, clamp_T, chunk));
        for (int i = 0; i < Dk; ++i) {
            double gi = gt[i];
            if (do_clamp && gi > 0.0) gi = 0.0;
            double d = exp(gi);
            double ki = kt[i];
            double* row = S + (size_t)i * Dv;
            for (int j = 0; j < Dv; ++j) row[j] = d * row[j] + ki * vt[j];
        }
        double* ot = o + t * tok_stride_v;
        for (int j = 0; j < Dv; ++j) ot[j] = 0.0;
        for (int i = 0; i < Dk; ++i) {
            double qi = qt[i];
            const double* row = S + (size_t)i * Dv;
            for (int j = 0; j < Dv; ++j) ot[j] += qi * row[j];
        }
    }
    if (s_out) memcpy(s_out, S, sizeof(double) * (size_t)Dk * Dv);
    free(S);
}

/* GLA forward with the reference's fast_chunk_gla clamp semantics.
 * clamp_mode: 2 = follow fast_chunk_gla dispatch for (T, chunk); 1 = always clamp g<=0;
 * 0 = never clamp.  s0 may be NULL (zero initial state); s_out may be NULL. */
ORACLE_API void oracle_gla_fwd(const double* q, const double* k, const double* v, const double* g,
                               const double* s0, double* o, double* s_out, long B, long T, long H,
                               int Dk, int Dv, long chunk, int clamp_mode) {
    long bh_total = B * H;
#pragma omp parallel for schedule(dynamic)
    for (long bh = 0; bh < bh_total; ++bh) {
        long b = bh / H, h = bh % H;
        long sk = H * Dk, sv = H * Dv;
        const double* qb = q + (b * T) * sk + h * Dk;
        const double* kb = k + (b * T) * sk + h * Dk;
        const double* gb = g + (b * T) * sk + h * Dk;
        const double* vb = v + (b * T) * sv + h * Dv;
        double* ob = o + (b * T) * sv + h * Dv;
        const double* s0b = s0 ? s0 + bh * (long)Dk * Dv : NULL;
        double* sob = s_out ? s_out + bh * (long)Dk * Dv : NULL;
        gla_one_head(qb, kb, vb, gb, T, sk, sv, Dk, Dv, s0b, ob, sob, T, chunk, clamp_mode);
    }
}

/* Packed ragged GLA: sequence i covers rows [cu[i], cu[i+1]) of [N_tok, H, D] tensors,
 * starts from s0[i] (or zero) and writes its final state to s_out[i].  g is clamped at 0
 * for every token (varlen rows are prefill rows). */
ORACLE_API void oracle_gla_varlen_fwd(const double* q, const double* k, const double* v,
                                      const double* g, const int32_t* cu, long n_seqs,
                                      const double* s0, double* o, double* s_out, long H, int Dk,
                                      int Dv) {
    long total = n_seqs * H;
#pragma omp parallel for schedule(dynamic)
    for (long ih = 0; ih < total; ++ih) {
        long i = ih / H, h = ih % H;
        long r0 = cu[i], n = (long)cu[i + 1] - (long)cu[i];
        long sk = H * Dk, sv = H * Dv;
        const double* s0i = s0 ? s0 + ih * (long)Dk * Dv : NULL;
        double* soi = s_out ? s_out + ih * (long)Dk * Dv : NULL;
        gla_one_head(q + r0 * sk + h * Dk, k + r0 * sk + h * Dk, v + r0 * sv + h * Dv,
                     g + r0 * sk + h * Dk, n, sk, sv, Dk, Dv, s0i, o + r0 * sv + h * Dv, soi, n, 0,
                     1);
    }
}

/* Closed form of the same map, with no recurrence:
 *   o_t[j] = sum_i q_t[i] ( e^{G_t[i]} S0[i][j] + sum_{s<=t} e^{G_t[i]-G_s[i]} k_s[i] v_s[j] )
 *   S_T[i][j] = e^{G_T[i]} S0[i][j] + sum_s e^{G_T[i]-G_s[i]} k_s[i] v_s[j]
 * with G_t = sum_{tau<=t} g_tau (g clamped at 0).  O(T^2 Dk Dv): tiny inputs only.
 * Used to pin oracle_gla_fwd, not as a product reference. */
ORACLE_API void oracle_gla_closed_form(const double* q, const double* k, const double* v,
                                       const double* g, const double* s0, double* o,
                                       double* s_out, long B, long T, long H, int Dk, int Dv) {
    double* G = (double*)malloc(sizeof(double) * (size_t)(T + 1) * Dk);
    for (long b = 0; b < B; ++b)
        for (long h = 0; h < H; ++h) {
            long sk = H * Dk, sv = H * Dv;
            const double* s0b = s0 ? s0 + (b * H + h) * (long)Dk * Dv : NULL;
            for (int i = 0; i < Dk; ++i) G[i] = 0.0;
            for (long t = 0; t < T; ++t)
                for (int i = 0; i < Dk; ++i) {
                    double gi = g[(b * T + t) * sk + h * Dk + i];
                    if (gi > 0.0) gi = 0.0;
                    G[(t + 1) * Dk + i] = G[t * Dk + i] + gi;
                }
            for (long t = 0; t <= T; ++t) {
                /* t < T: output row t (cumulative index t+1); t == T: final state */
                long ct = (t < T) ? t + 1 : T;
                for (int j = 0; j < Dv; ++j) {
                    double acc_o = 0.0;
                    for (int i = 0; i < Dk; ++i) {
                        double sij = s0b ? exp(G[ct * Dk + i]) * s0b[(long)i * Dv + j] : 0.0;
                        for (long s = 0; s < ct; ++s)
                            sij += exp(G[ct * Dk + i] - G[(s + 1) * Dk + i]) *
                                   k[(b * T + s) * sk + h * Dk + i] * v[(b * T + s) * sv + h * Dv + j];
                        if (t < T) acc_o += q[(b * T + t) * sk + h * Dk + i] * sij;
                        else if (s_out) s_out[((b * H + h) * (long)Dk + i) * Dv + j] = sij;
                    }
                    if (t < T) o[(b * T + t) * sv + h * Dv + j] = acc_o;
                }
            }
        }
    free(G);
}

/* One recurrent decode step over rows bh (no clamp; fast_gla.py:746-753):
 *   S[bh] <- diag(exp g[bh]) S[bh] + k[bh] v[bh]^T ;  o[bh] = S[bh]^T q[bh]
 * q,k,g: [BH, Dk]; v,o: [BH, Dv]; S: [BH, Dk, Dv] updated in place. */
ORACLE_API void oracle_gla_decode_step(const double* q, const double* k, const double* v,
                                       const double* g, double* S, double* o, long BH, int Dk,
                                       int Dv) {
#pragma omp parallel for schedule(static)
    for (long bh = 0; bh < BH; ++bh) {
        double* Sb = S + bh * (long)Dk * Dv;
        double* ob = o + bh * Dv;
        for (int j = 0; j < Dv; ++j) ob[j] = 0.0;
        for (int i = 0; i < Dk; ++i) {
            double d = exp(g[bh * Dk + i]);
            double ki = k[bh * Dk + i], qi = q[bh * Dk + i];
            double* row = Sb + (long)i * Dv;
            for (int j = 0; j < Dv; ++j) {
                row[j] = d * row[j] + ki * v[bh * Dv + j];
                ob[j] += qi * row[j];
            }
        }
    }
}

/* Exclusive affine scan (FusedRecurrentScan forward, fast_gla.py:34-64, :109-149):
 * for each lane m of M = B*H*Dk*Dv and n = 0..N-1:
 *   s_all[m][n] = s ;  s = s * decay[m][n] + kv[m][n]      (s starts at init[m])
 * kv, s_all: [B,H,N,Dk,Dv]; decay: [B,H,N,Dk] (broadcast over Dv); init, fin: [B,H,Dk,Dv]. */
ORACLE_API void oracle_recurrent_scan_fwd(const double* kv, const double* decay, const double* init,
                                          double* s_all, double* fin, long B, long H, long N, int Dk,
                                          int Dv) {
    long DD = (long)Dk * Dv;
#pragma omp parallel for schedule(static)
    for (long bh = 0; bh < B * H; ++bh)
        for (long e = 0; e < DD; ++e) {
            long i = e / Dv;
            double s = init ? init[bh * DD + e] : 0.0;
            for (long n = 0; n < N; ++n) {
                long idx = (bh * N + n) * DD + e;
                s_all[idx] = s;
                s = s * decay[(bh * N + n) * Dk + i] + kv[idx];
            }
            fin[bh * DD + e] = s;
        }
}

/* Backward of the exclusive affine scan above (reference: _recurrent_scan_bwd,
 * triune/kernels/fast_gla.py:67-107, and FusedRecurrentScan.backward :151-203):
 *   d = d_fin;  for n = N-1..0:  d_kv[n] = d;  d_decay[n][i] = sum_j d[i][j] s_all[n][i][j];
 *                                d = d_s_all[n] + decay[n] * d;
 *   d_init = d.
 * d_s_all / d_fin may be NULL (zero).  d_decay is [B,H,N,Dk] (summed over Dv). */
ORACLE_API void oracle_recurrent_scan_bwd(const double* d_s_all, const double* d_fin, const double* decay,
                                          const double* s_all, double* d_kv, double* d_decay, double* d_init,
                                          long B, long H, long N, int Dk, int Dv) {
    long DD = (long)Dk * Dv;
#pragma omp parallel for schedule(static)
    for (long bh = 0; bh < B * H; ++bh) {
        double* d = (double*)malloc(sizeof(double) * (size_t)DD);
        for (long e = 0; e < DD; ++e) d[e] = d_fin ? d_fin[bh * DD + e] : 0.0;
        for (long n = N - 1; n >= 0; --n) {
            long base = (bh * N + n) * DD;
            for (int i = 0; i < Dk; ++i) {
                double acc = 0.0, dec = decay[(bh * N + n) * Dk + i];
                for (int j = 0; j < Dv; ++j) {
                    long e = (long)i * Dv + j;
                    d_kv[base + e] = d[e];
                    acc += d[e] * s_all[base + e];
                    d[e] = (d_s_all ? d_s_all[base + e] : 0.0) + dec * d[e];
                }
                d_decay[(bh * N + n) * Dk + i] = acc;
            }
        }
        for (long e = 0; e < DD; ++e) d_init[bh * DD + e] = d[e];
        free(d);
    }
}

/* Gradients of oracle_gla_fwd (same clamp semantics) for upstream gradients do [B,T,H,Dv] and
 * ds_fin [B,H,Dk,Dv] (either may be NULL = zero).  With D_t the total gradient reaching S_t:
 *   D_{T-1} = ds_fin + q_{T-1} do_{T-1}^T ,  D_{t-1} = q_{t-1} do_{t-1}^T + diag(a_t) D_t
 *   dq_t = S_t do_t ,  dk_t = D_t v_t ,  dv_t = D_t^T k_t ,
 *   d(g_eff)_t[i] = a_t[i] sum_j D_t[i][j] S_{t-1}[i][j] ,  ds0 = diag(a_0) D_0
 * with a_t = exp(g_eff_t).  A clamped token passes its gradient where g <= 0 (the derivative of
 * torch.clamp(g, max=0), fast_gla.py:586) and none where g > 0; an unclamped token passes it all.
 * The forward keeps every state (T+1 of them per head), so sizes stay test-sized. */
static void gla_bwd_one_head(const double* q, const double* k, const double* v, const double* g,
                             const double* dout, long T, long sk, long sv, int Dk, int Dv, const double* s0,
                             const double* dsf, double* dq, double* dk, double* dv, double* dg, double* ds0,
                             long chunk, int clamp_mode) {
    const size_t DD = (size_t)Dk * Dv;
    double* hist = (double*)malloc(sizeof(double) * DD * (size_t)(T + 1));  /* hist[t+1] = S_t */
    double* D = (double*)malloc(sizeof(double) * DD);
    if (s0) memcpy(hist, s0, sizeof(double) * DD);
    else memset(hist, 0, sizeof(double) * DD);
    for (long t = 0; t < T; ++t) {
        const double* kt = k + t * sk;
        const double* gt = g + t * sk;
        const double* vt = v + t * sv;
        int do_clamp = clamp_mode == 1 ? 1 : (clamp_mode == 0 ? 0 : clamp_token(t, T, chunk));
        const double* P = hist + (size_t)t * DD;
        double* S = hist + (size_t)(t + 1) * DD;
        for (int i = 0; i < Dk; ++i) {
            double gi = gt[i];
            if (do_clamp && gi > 0.0) gi = 0.0;
            double a = exp(gi);
            for (int j = 0; j < Dv; ++j) S[(size_t)i * Dv + j] = a * P[(size_t)i * Dv + j] + kt[i] * vt[j];
        }
    }
    for (size_t e = 0; e < DD; ++e) D[e] = dsf ? dsf[e] : 0.0;
    for (long t = T - 1; t >= 0; --t) {
        const double* qt = q + t * sk;
        const double* kt = k + t * sk;
        const double* gt = g + t * sk;
        const double* vt = v + t * sv;
        const double* dot = dout ? dout + t * sv : NULL;
        int do_clamp = clamp_mode == 1 ? 1 : (clamp_mode == 0 ? 0 : clamp_token(t, T, chunk));
        const double* S = hist + (size_t)(t + 1) * DD;
        const double* P = hist + (size_t)t * DD;
        if (dot)
            for (int i = 0; i < Dk; ++i)
                for (int j = 0; j < Dv; ++j) D[(size_t)i * Dv + j] += qt[i] * dot[j];
        for (int i = 0; i < Dk; ++i) {
            double aq = 0.0, ak = 0.0, ag = 0.0;
            for (int j = 0; j < Dv; ++j) {
                size_t e = (size_t)i * Dv + j;
                if (dot) aq += S[e] * dot[j];
                ak += D[e] * vt[j];
                ag += D[e] * P[e];
            }
            double gi = gt[i];
            int pass = !(do_clamp && gi > 0.0);
            if (do_clamp && gi > 0.0) gi = 0.0;
            double a = exp(gi);
            dq[t * sk + i] = aq;
            dk[t * sk + i] = ak;
            dg[t * sk + i] = pass ? a * ag : 0.0;
        }
        for (int j = 0; j < Dv; ++j) {
            double acc = 0.0;
            for (int i = 0; i < Dk; ++i) acc += D[(size_t)i * Dv + j] * kt[i];
            dv[t * sv + j] = acc;
        }
        for (int i = 0; i < Dk; ++i) {
            double gi = gt[i];
            if (do_clamp && gi > 0.0) gi = 0.0;
            double a = exp(gi);
            for (int j = 0; j < Dv; ++j) D[(size_t)i * Dv + j] *= a;
        }
    }
    if (ds0) memcpy(ds0, D, sizeof(double) * DD);
    free(D);
    free(hist);
}

ORACLE_API void oracle_gla_bwd(const double* q, const double* k, const double* v, const double* g,
                               const double* s0, const double* dout, const double* dsf, double* dq, double* dk,
                               double* dv, double* dg, double* ds0, long B, long T, long H, int Dk, int Dv,
                               long chunk, int clamp_mode) {
#pragma omp parallel for schedule(dynamic)
    for (long bh = 0; bh < B * H; ++bh) {
        long b = bh / H, h = bh % H;
        long sk = H * Dk, sv = H * Dv;
        long ok = (b * T) * sk + h * Dk, ov = (b * T) * sv + h * Dv;
        const double* s0b = s0 ? s0 + bh * (long)Dk * Dv : NULL;
        const double* dsb = dsf ? dsf + bh * (long)Dk * Dv : NULL;
        gla_bwd_one_head(q + ok, k + ok, v + ov, g + ok, dout ? dout + ov : NULL, T, sk, sv, Dk, Dv, s0b, dsb,
                         dq + ok, dk + ok, dv + ov, dg + ok, ds0 ? ds0 + bh * (long)Dk * Dv : NULL, chunk,
                         clamp_mode);
    }
}

/* Gated DeltaNet, the reference variant (fast_gla.py:781-836 and :453-471):
 *   u_t   = v_t - S_{t-1}^T k_t              (prediction from the un-decayed state)
 *   S_t   = diag(exp(min(g_t,0))) S_{t-1} + W_t
 *   W_t   = k_t u_t^T scaled by beta
 *   o_t   = S_t^T q_t
 * beta_kind: 0 none (beta = 1); 1 per (token, head) scalar, beta [B,T,H];
 *            2 per key dim (rows of W, the PyTorch path fast_gla.py:823-827), beta [B,T,H,Dk];
 *            3 per value dim (columns of W, the Triton path fast_gla.py:464-465), beta [B,T,H,Dv]. */
ORACLE_API void oracle_gdn_fwd(const double* q, const double* k, const double* v, const double* g,
                               const double* beta, int beta_kind, const double* s0, double* o,
                               double* s_out, long B, long T, long H, int Dk, int Dv) {
#pragma omp parallel for schedule(dynamic)
    for (long bh = 0; bh < B * H; ++bh) {
        long b = bh / H, h = bh % H;
        long sk = H * Dk, sv = H * Dv;
        double* S = (double*)malloc(sizeof(double) * (size_t)Dk * Dv);
        double* u = (double*)malloc(sizeof(double) * (size_t)Dv);
        if (s0) memcpy(S, s0 + bh * (long)Dk * Dv, sizeof(double) * (size_t)Dk * Dv);
        else memset(S, 0, sizeof(double) * (size_t)Dk * Dv);
        for (long t = 0; t < T; ++t) {
            const double* qt = q + (b * T + t) * sk + h * Dk;
            const double* kt = k + (b * T + t) * sk + h * Dk;
            const double* gt = g + (b * T + t) * sk + h * Dk;
            const double* vt = v + (b * T + t) * sv + h * Dv;
            for (int j = 0; j < Dv; ++j) {
                double pred = 0.0;
                for (int i = 0; i < Dk; ++i) pred += kt[i] * S[(long)i * Dv + j];
                u[j] = vt[j] - pred;
            }
            for (int i = 0; i < Dk; ++i) {
                double gi = gt[i] > 0.0 ? 0.0 : gt[i];
                double d = exp(gi);
                double rs = 1.0;
                if (beta_kind == 1) rs = beta[(b * T + t) * H + h];
                else if (beta_kind == 2) rs = beta[(b * T + t) * sk + h * Dk + i];
                for (int j = 0; j < Dv; ++j) {
                    double cs = (beta_kind == 3) ? beta[(b * T + t) * sv + h * Dv + j] : 1.0;
                    S[(long)i * Dv + j] = d * S[(long)i * Dv + j] + rs * cs * kt[i] * u[j];
                }
            }
            double* ot = o + (b * T + t) * sv + h * Dv;
            for (int j = 0; j < Dv; ++j) {
                double acc = 0.0;
                for (int i = 0; i < Dk; ++i) acc += qt[i] * S[(long)i * Dv + j];
                ot[j] = acc;
            }
        }
        if (s_out) memcpy(s_out + bh * (long)Dk * Dv, S, sizeof(double) * (size_t)Dk * Dv);
        free(S);
        free(u);
    }
}

/* Gradients of oracle_gdn_fwd for upstream gradients do [B,T,H,Dv] and ds_fin [B,H,Dk,Dv] (NULL =
 * zero): the reference differentiates fast_recurrent_gated_deltanet (fast_gla.py:781-836) with
 * autograd whenever a gradient is needed (fast_chunk_gated_deltanet, fast_gla.py:885-904).  With
 * P = S_{t-1}, a = exp(min(g_t, 0)), W = w uu^T where w_i = rs_i k_i, uu_j = cs_j u_j (rs, cs the
 * row and column beta factors, 1 where the kind has none), and D the gradient reaching S_t:
 *   D += q do^T ;  dq_i = sum_j S_t[i][j] do_j
 *   c_j = sum_i D[i][j] w_i ;  du_j = cs_j c_j ;  dv_j = du_j ;  dpred_j = -du_j
 *   e_i = sum_j D[i][j] uu_j ;  dk_i = rs_i e_i + sum_j P[i][j] dpred_j
 *   dbeta: head sum_j u_j c_j ; key k_i e_i ; value u_j c_j
 *   dg_i = a_i sum_j D[i][j] P[i][j] where g_i <= 0 (torch.clamp(max=0) passes its gradient
 *          there), else 0
 *   D <- diag(a) D + k dpred^T ;  ds0 = D after token 0.
 * dbeta has beta's shape ([B,T,H] or [B,T,H,D]); every state is kept (test sizes). */
ORACLE_API void oracle_gdn_bwd(const double* q, const double* k, const double* v, const double* g,
                               const double* beta, int beta_kind, const double* s0, const double* dout,
                               const double* dsf, double* dq, double* dk, double* dv, double* dg,
                               double* dbeta, double* ds0, long B, long T, long H, int Dk, int Dv) {
#pragma omp parallel for schedule(dynamic)
    for (long bh = 0; bh < B * H; ++bh) {
        long b = bh / H, h = bh % H;
        long sk = H * Dk, sv = H * Dv;
        const size_t DD = (size_t)Dk * Dv;
        double* hist = (double*)malloc(sizeof(double) * DD * (size_t)(T + 1)); /* hist[t] = S_{t-1} */
        double* U = (double*)malloc(sizeof(double) * (size_t)(T > 0 ? T : 1) * Dv); /* u_t */
        double* D = (double*)malloc(sizeof(double) * DD);
        double* c = (double*)malloc(sizeof(double) * (size_t)Dv);
        double* dp = (double*)malloc(sizeof(double) * (size_t)Dv);
        if (s0) memcpy(hist, s0 + bh * (long)DD, sizeof(double) * DD);
        else memset(hist, 0, sizeof(double) * DD);
#define RS(t, i) (beta_kind == 2 ? beta[(b * T + (t)) * sk + h * Dk + (i)] : 1.0)
#define CS(t, j) (beta_kind == 1 ? beta[(b * T + (t)) * H + h] : beta_kind == 3 ? beta[(b * T + (t)) * sv + h * Dv + (j)] : 1.0)
        for (long t = 0; t < T; ++t) {
            const double* kt = k + (b * T + t) * sk + h * Dk;
            const double* gt = g + (b * T + t) * sk + h * Dk;
            const double* vt = v + (b * T + t) * sv + h * Dv;
            const double* P = hist + (size_t)t * DD;
            double* S = hist + (size_t)(t + 1) * DD;
            double* u = U + t * Dv;
            for (int j = 0; j < Dv; ++j) {
                double pred = 0.0;
                for (int i = 0; i < Dk; ++i) pred += kt[i] * P[(size_t)i * Dv + j];
                u[j] = vt[j] - pred;
            }
            for (int i = 0; i < Dk; ++i) {
                double a = exp(gt[i] > 0.0 ? 0.0 : gt[i]);
                for (int j = 0; j < Dv; ++j)
                    S[(size_t)i * Dv + j] = a * P[(size_t)i * Dv + j] + RS(t, i) * kt[i] * CS(t, j) * u[j];
            }
        }
        for (size_t e = 0; e < DD; ++e) D[e] = dsf ? dsf[bh * (long)DD + e] : 0.0;
        for (long t = T - 1; t >= 0; --t) {
            const long ok = (b * T + t) * sk + h * Dk, ov = (b * T + t) * sv + h * Dv;
            const double* qt = q + ok;
            const double* kt = k + ok;
            const double* gt = g + ok;
            const double* dot = dout ? dout + ov : NULL;
            const double* P = hist + (size_t)t * DD;
            const double* S = hist + (size_t)(t + 1) * DD;
            const double* u = U + t * Dv;
            if (dot)
                for (int i = 0; i < Dk; ++i)
                    for (int j = 0; j < Dv; ++j) D[(size_t)i * Dv + j] += qt[i] * dot[j];
            double dbh = 0.0;
            for (int j = 0; j < Dv; ++j) {
                double acc = 0.0;
                for (int i = 0; i < Dk; ++i) acc += D[(size_t)i * Dv + j] * RS(t, i) * kt[i];
                c[j] = acc;
                const double du = CS(t, j) * acc;
                dv[ov + j] = du;
                dp[j] = -du;
                dbh += u[j] * acc;
                if (beta_kind == 3) dbeta[ov + j] = u[j] * acc;
            }
            if (beta_kind == 1) dbeta[(b * T + t) * H + h] = dbh;
            for (int i = 0; i < Dk; ++i) {
                double aq = 0.0, e = 0.0, f = 0.0, ag = 0.0;
                for (int j = 0; j < Dv; ++j) {
                    const size_t x = (size_t)i * Dv + j;
                    if (dot) aq += S[x] * dot[j];
                    e += D[x] * CS(t, j) * u[j];
                    f += P[x] * dp[j];
                    ag += D[x] * P[x];
                }
                const double a = exp(gt[i] > 0.0 ? 0.0 : gt[i]);
                dq[ok + i] = aq;
                dk[ok + i] = RS(t, i) * e + f;
                dg[ok + i] = gt[i] <= 0.0 ? a * ag : 0.0;
                if (beta_kind == 2) dbeta[ok + i] = kt[i] * e;
            }
            for (int i = 0; i < Dk; ++i) {
                const double a = exp(gt[i] > 0.0 ? 0.0 : gt[i]);
                for (int j = 0; j < Dv; ++j) D[(size_t)i * Dv + j] = a * D[(size_t)i * Dv + j] + kt[i] * dp[j];
            }
        }
#undef RS
#undef CS
        if (ds0) memcpy(ds0 + bh * (long)DD, D, sizeof(double) * DD);
        free(dp);
        free(c);
        free(D);
        free(U);
        free(hist);
    }
}

ORACLE_API int oracle_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
