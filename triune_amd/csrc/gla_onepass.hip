// gla_onepass.hip -- single-launch chunked GLA prefill for calls of few chunks (gfx950).
//
// The three-launch prefill (segment states, carry scan, outputs; gla_prefill.h) pays two kernel
// boundaries and a serial scan over segments.  At the prefill tiles VectorisedGLA runs (B = 4,
// T = 1024, H = 6: 16 chunks per (sequence, head), triune/model/attention.py:425-451, 458-499)
// those fixed costs are most of the call.  Here the whole call is one launch.  One workgroup of
// eight waves owns two consecutive 64-token chunks ("a pair") of one (sequence, head), four waves
// per chunk:
//   1. each chunk's rows are loaded once; with PREP, q, k, g are raw projections and stage 1 forms
//      q, k <- RoPE(normalize(elu(x) + 1)), g <- logsigmoid(g) (attention.py:14-79), rounds them to
//      the I/O dtype and writes them back in place, as the reference's prep kernel does;
//   2. stage 1 of the chunk kernel (factored operands Qt, Kt in LDS) and the chunk's local end
//      state L = e^m (Kt^T V);
//   3. the pair's state map (e^{G_C}, L) -- the second chunk's applied to the first's -- is
//      published to the workspace, followed by a flag;
//   4. what does not depend on the state entering the chunk, while the earlier pairs publish:
//      stage 2 (the causal A^T tiles) and the outputs' in-chunk part O^T = V^T A^T;
//   5. the state entering the pair is folded from s0 and the earlier pairs' published maps,
//      S <- e^{G_C(j)} S + L_j for j = 0 .. p-1 (the affine scan the carry kernel runs); the second
//      chunk applies the first chunk's map to it;
//   6. each chunk's outputs O^T += (e^m S)^T Qt^T; the last chunk stores the final state.
// Workgroup barriers that order only LDS traffic wait for LDS alone (lds_sync), so the in-place
// write-back of step 1 stays in flight until the wait before the flag.
// Chunks whose decay span exceeds the factored range (or that hold the unclamped 1-token tail)
// stage their rows in LDS and walk the tokens one by one, for the local state and the outputs.
//
// Waiting on another workgroup's flag is safe only if that workgroup runs: the host launches this
// kernel only when every workgroup of the grid is resident at once, and a workgroup waits only for
// earlier pairs of its own (sequence, head).  Every wait is bounded (about a second); one that runs
// out records an error bit in the control block and the kernel still ends.
//
// Flags need no clearing between calls: the control block (caller-owned, zero before its first
// use, reused stream-ordered) holds an epoch; a call publishes epoch + 1, and once every
// workgroup has read the epoch (a count) the last one counted advances it at its end, so flags
// left by earlier calls never match.
//
// Where the published maps live.  Dispatch hands workgroup x to XCD x mod 8 (round robin; with
// fewer XCDs per partition, a divisor of 8, the residue still fixes the XCD), and all pairs of a
// (sequence, head) are given to workgroups x of one residue, so one XCD holds every pair of it.
// The maps are written with plain stores into that XCD's L2 and read back with L1-bypassing
// loads; each flag (written and read device-coherently, sc1) carries the XCD of its writer, and a
// reader on another XCD would record error bit 2 (the maps would not be in its L2) and read them
// device-coherently.  The stores' completion (vmcnt) precedes the barrier after which the flag is
// stored.
#include "gla_prefill.h"

#include <hip/hip_ext.h>

namespace triune {

namespace {

constexpr int OP_D = 64;                     // head dim (Dk = Dv) of the single-launch kernel
constexpr int OP_GROUPS = 2;                 // chunks per workgroup
constexpr int OP_THREADS = 256 * OP_GROUPS;  // four waves per chunk, one per 16 value columns
constexpr int OP_MAX_PAIRS = 32;             // at most 64 chunks per sequence
constexpr uint32_t OP_SPIN_MAX = 1u << 20;
constexpr int OP_SC0 = 0x01;  // cache-policy bits of a buffer access: sc0 (L1 bypass)
constexpr int OP_SC1 = 0x10;  // sc1 (device-coherent: past the XCD's L2)
// s_getreg operand of HW_REG_XCC_ID, bits [3:0]: the XCD this wave runs on
constexpr int OP_HWREG_XCC_ID = 20 | (0 << 6) | (3 << 11);

// LDS of a workgroup: one chunk region per group (the chunk kernel's layout), the first chunk's
// local state L for the second ([4][256 threads][4 floats]), the decay factors of the earlier pairs.
template <typename TIn, bool PREP>
struct OpLay {
    using L = Lay<TIn, OP_D, OP_D, true, PREP>;
    static constexpr int GB = (L::BYTES + 255) / 256 * 256;
    static constexpr int OFF_X = OP_GROUPS * GB;
    static constexpr int OFF_E = OFF_X + 256 * 16 * 4;
    static constexpr int BYTES = OFF_E + OP_MAX_PAIRS * OP_D * 4;
    static_assert(BYTES <= 160 * 1024, "LDS budget");
    // a chunk that walks token by token stages q, k, v (TIn) and g (up to fp32) rows [64][64] in
    // its region's Qt / Kt / A^T planes
    static_assert(3 * 64 * 64 * (int)sizeof(TIn) + 64 * 64 * 4 <= L::OFF_VP, "staged rows fit");
};

// The state entering pair p from s0's value in S and the published maps of pairs j < p:
// S <- e^{G_C(j)} S + L_j in order, on the rows 32 HALF .. 32 HALF + 31 of the state (vectors
// db = 2 HALF, 2 HALF + 1); each chunk group folds one half and the caller exchanges them, so a
// workgroup reads every map once.  The decay factors are staged in LDS (sEGj, p x 64 floats) by
// the whole workgroup; each thread then loads its 8 values of up to eight L_j at a time (slots
// past the last map read through a resource without records, which moves no data).  maps: L_0 of
// this (sequence, head).
template <int CPOL, int HALF>
__device__ __forceinline__ void fold_half(const float* maps, __amdgpu_buffer_rsrc_t rE, float* sEGj, int pj,
                                          f32x4 (&S)[4], int g4) {
    auto ld4 = [](__amdgpu_buffer_rsrc_t r, int off) {
        return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, CPOL));
    };
    for (int i = (int)threadIdx.x; i < pj * 16; i += OP_THREADS)
        *reinterpret_cast<f32x4*>(sEGj + 4 * i) = ld4(rE, 16 * i);
    __syncthreads();
    // L_j as [4][256 threads][4 floats]: the values of vector db of every thread of a group are
    // 4 KB in a row, so each 16-byte-per-lane load of a wave reads 1 KB of whole cache lines
    const int lo = ((int)threadIdx.x & 255) * 16 + 4096 * 2 * HALF;
    for (int j = 0; j < pj; j += 8) {
        const int n = pj - j < 8 ? pj - j : 8;
        f32x4 lj[8][2];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float*>(maps) + (int64_t)(j + u) * (OP_D * OP_D), (short)0, u < n ? OP_D * OP_D * 4 : 0,
                0x00020000);
#pragma unroll
            for (int dh = 0; dh < 2; ++dh) lj[u][dh] = ld4(r, lo + 4096 * dh);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (u >= n) break;
#pragma unroll
            for (int dh = 0; dh < 2; ++dh) {
                const int db = 2 * HALF + dh;
                const f32x4 e = *reinterpret_cast<const f32x4*>(sEGj + (j + u) * OP_D + 16 * db + 4 * g4);
#pragma unroll
                for (int i = 0; i < 4; ++i) S[db][i] = fmaf(e[i], S[db][i], lj[u][dh][i]);
            }
        }
    }
}

// Token-by-token walk of a chunk whose rows are staged in LDS (q, k, v as TIn and g as TG, each
// [64][64] row-major from `stg`) for a wave's 16 value columns, from the state in S (updated in
// place); t_unc: the token (index in the chunk) whose gate stays unclamped, or out of range.  With
// OUT the outputs go straight to memory (inputs come from LDS, so o may alias g without a barrier).
template <typename TIn, typename TG, bool OUT>
__device__ void walk_staged(const char* stg, int nv, int64_t t_unc, int c0, int g4, int r16, f32x4 (&S)[4],
                            const OutCtx& oc, int64_t tc) {
    const TIn* sq = reinterpret_cast<const TIn*>(stg);
    const TIn* sk = sq + 64 * 64;
    const TIn* sv = sk + 64 * 64;
    const TG* sg = reinterpret_cast<const TG*>(sv + 64 * 64);
    const int oes = dt_size(oc.dt);
    for (int t = 0; t < nv; ++t) {
        float dcy[4][4], kk[4][4], qq[4][4];
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int d = t * 64 + 16 * db + 4 * g4 + i;
                const float gg = (float)sg[d];
                dcy[db][i] = fast_exp(t == t_unc ? gg : min0(gg));
                kk[db][i] = (float)sk[d];
                qq[db][i] = OUT ? (float)sq[d] : 0.f;
            }
        const float vv = (float)sv[t * 64 + c0 + r16];
        float part = 0.f;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float s = dcy[db][i] * S[db][i] + kk[db][i] * vv;
                S[db][i] = s;
                part += qq[db][i] * s;
            }
        if constexpr (OUT) {
            part += __shfl_xor(part, 16);
            part += __shfl_xor(part, 32);
            if (g4 == 0) {
                char* op = oc.op + (tc + t) * oc.ost + (int64_t)(c0 + r16) * oes;
                if (oc.dt == DT_F32) *reinterpret_cast<float*>(op) = part;
                else if (oc.dt == DT_BF16) *reinterpret_cast<__bf16*>(op) = (__bf16)part;
                else *reinterpret_cast<_Float16*>(op) = (_Float16)part;
            }
        }
    }
}

// Rows 4*tg + j (j < 4) of one input, N elements from column col, into a staged [64][64] plane.
template <typename T, int N>
__device__ __forceinline__ void stage_rows(char* plane, const Vec<T, N> (&v)[4], int tg, int col) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t* p = reinterpret_cast<uint32_t*>(reinterpret_cast<T*>(plane) + (4 * tg + j) * 64 + col);
#pragma unroll
        for (int w = 0; w < Vec<T, N>::W; ++w) p[w] = v[j].w[w];
    }
}

}  // namespace

// CK: checked row addressing (T not a multiple of 4).  PREP: q, k, g are raw projections.
// OBF: bf16 outputs known at compile time.
template <typename TIn, typename TG, bool CK, bool PREP, bool OBF>
__global__ __launch_bounds__(OP_THREADS, 1) void gla_onepass_kernel(PrefillParams a, OnePassCtl ctl) {
    constexpr int DK = OP_D, DV = OP_D;
    using L = Lay<TIn, DK, DV, true, PREP>;
    using OL = OpLay<TIn, PREP>;
    using PR = Prec<TIn>;
    constexpr int NW = L::NW, DPW = L::DPW, DL = DPW / 4, NKS = DK / 32, NS = PR::NS, NX = PR::NX;
    __shared__ __attribute__((aligned(16))) char lds[OL::BYTES];

    // ---- work item: pair p of (sequence, head) bh; every pair of bh on one XCD ----------------
    const int64_t xb = blockIdx.x, x8 = xb & 7, kx = xb >> 3;
    const int64_t p = kx / ctl.nh8, bh = x8 + 8 * (kx - p * ctl.nh8);
    const int64_t BH = a.n_seqs * a.H;
    if (bh >= BH || p >= ctl.npair) return;
    const int64_t b = bh / a.H, h = bh - b * a.H;
    const int wave8 = wave_id(), grp = wave8 >> 2, wave = wave8 & 3;  // chunk group, wave in it
    // The second chunk's group ends the pair's chain (it also applies the first chunk's map to the
    // entering state), so its waves issue one priority level up (from raw projections 20.4 -> 20.0
    // us per call at the 1024-token tile, same-box A/B; plain inputs unchanged).
    if (grp == 1) __builtin_amdgcn_s_setprio(1);
    const int lane = threadIdx.x & 63, r16 = lane & 15, g4 = lane >> 4, tg = lane >> 2, row = lane & 3;
    const int tid = (int)threadIdx.x & 255;  // thread index in the group
    const int64_t c = 2 * p + grp;            // this group's chunk (past the end: an empty chunk)
    Work wk;
    wk.seq = b; wk.b = b; wk.row0 = 0; wk.p = (int)c; wk.len = a.T;
    wk.t_begin = c * CHUNK;
    wk.t_end = wk.t_begin + CHUNK < a.T ? wk.t_begin + CHUNK : a.T;
    if (wk.t_end < wk.t_begin) wk.t_end = wk.t_begin;
    const int64_t tc = wk.t_begin;
    const int nv = (int)(wk.t_end - tc);
    const bool last_pair = p == ctl.npair - 1;
    const bool has_last = c == ctl.nch - 1;  // this group holds the sequence's last chunk

    char* smem = lds + grp * OL::GB;
    char* sQT = smem + L::OFF_QT;
    char* sKT = smem + L::OFF_KT;
    char* sAT = smem + L::OFF_AT;
    char* sVP = smem + L::OFF_VP + wave * NX * L::VPP;
    float* sEM = reinterpret_cast<float*>(smem + L::OFF_FAC);
    float* sEG = sEM + DK;
    int* sFLAG = reinterpret_cast<int*>(smem + L::OFF_FLAG);
    float* sX = reinterpret_cast<float*>(lds + OL::OFF_X);
    float* sEGj = reinterpret_cast<float*>(lds + OL::OFF_E);
    const int c0 = wave * 16;
    const int dl0 = stage1_dim0<DK, DPW, PREP>(wave, row);


    const ChunkAddr ad = chunk_addr<true, TIn, TG>(a, wk, h, tg, dl0, c0 + 4 * row);
    ChunkIn<TIn, TG, DL> cur;
    chunk_load<true, CK>(cur, ad, tc, nv > 0);
    const int64_t t_unclamped = (!PREP && (a.flags & 1)) ? wk.len - 1 : -1;
    const bool tail_unclamped = nv > 0 && t_unclamped == tc + nv - 1;

    // ---- stage 1: (pre-processing,) decay scan, the fast / token-wise choice ------------------
    float G[4][DL], GC[DL], x[4][DL], y[4][DL];  // g, q, k
    Vec<TIn, DL> qo[4], ko[4];                    // PREP: the rounded pre-processed q, k
    Vec<TG, DL> go[4];                            // PREP: the rounded logsigmoid gate
    RopeIn<DL> rc;
    if constexpr (PREP) {
        RopeAddr rad;
        rad.c = tok_addr<float>(a.cs, wk, h, tg, dl0);
        rad.s = tok_addr<float>(a.sn, wk, h, tg, dl0);
        rope_load<CK>(rc, rad, tc, nv > 0 && a.use_rope != 0);
        chunk_float<CK>(cur.g, G, tg, nv);
        chunk_float<CK>(cur.q, x, tg, nv);
        chunk_float<CK>(cur.k, y, tg, nv);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < DL; ++i) {
                G[j][i] = logsigmoid(G[j][i]);  // never positive: the clamp is moot
                x[j][i] = elu1(x[j][i]);
                y[j][i] = elu1(y[j][i]);
            }
        if (nv < CHUNK) {  // rows past the chunk's end load as zeros and must stay zero
            zero_rows_past<DL>(G, tg, nv);
            zero_rows_past<DL>(x, tg, nv);
            zero_rows_past<DL>(y, tg, nv);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {  // the gate as the reference's scan reads it: rounded
            vec_pack<TG, DL>(G[j], go[j]);
            vec_float(go[j], G[j]);
        }
        float* sNRM = reinterpret_cast<float*>(smem + L::OFF_NRM);
        norm_partials<DL>(x, sNRM + wave * 64, tg, row);
        norm_partials<DL>(y, sNRM + (NW + wave) * 64, tg, row);
    } else {
        chunk_float<CK>(cur.g, G, tg, nv);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < DL; ++i) G[j][i] = min0(G[j][i]);
        chunk_float<CK>(cur.q, x, tg, nv);
        chunk_float<CK>(cur.k, y, tg, nv);
    }
    lds_put_v_rows<TIn, NX, CK>(sVP, L::VPP, L::VS, 4 * row, cur.v, tg, nv);
    chunk_cumsum<DL>(G, GC, lane);
    {
        bool bad = tail_unclamped;
#pragma unroll
        for (int i = 0; i < DL; ++i) bad |= !(GC[i] >= -SPAN_MAX);
        const bool any_bad = __any(bad);
        if (lane == 0) sFLAG[wave] = any_bad ? 1 : 0;
        if (tg == 0) {
#pragma unroll
            for (int i = 0; i < DL; ++i) {
                const float em = fast_exp(0.5f * GC[i]);
                sEM[dl0 + i] = em;
                sEG[dl0 + i] = em * em;
            }
        }
    }
    __syncthreads();  // every wave's flags (and PREP: norm partials)
    // Epoch of this call: flags of this call carry ep; the last workgroup to count its read of it
    // stores ep at its end.
    // Read once the chunk's loads are all out, and made uniform where the flag is stored, so its
    // latency runs under the rest of stage 1.
    const uint32_t ep_word = __hip_atomic_load(ctl.hdr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    bool fast = true;
#pragma unroll
    for (int w = 0; w < NW; ++w) fast = fast && (sFLAG[w] == 0);
    if constexpr (PREP) {
        if (a.use_rope) {
            rope_rows<DL>(x, rc, row);
            rope_rows<DL>(y, rc, row);
        }
        const float* sNRM = reinterpret_cast<const float*>(smem + L::OFF_NRM);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float iq = token_inv_norm<NW>(sNRM, 4 * tg + j);
            const float ik = token_inv_norm<NW>(sNRM + NW * 64, 4 * tg + j);
#pragma unroll
            for (int i = 0; i < DL; ++i) {
                x[j][i] *= iq;
                y[j][i] *= ik;
            }
            vec_pack<TIn, DL>(x[j], qo[j]);
            vec_pack<TIn, DL>(y[j], ko[j]);
            vec_float(qo[j], x[j]);  // from here on the rounded values
            vec_float(ko[j], y[j]);
        }
        rows_store<CK>(qo, chunk_rsrc(ad.q, tc, true), ad.q, tc);
        rows_store<CK>(ko, chunk_rsrc(ad.k, tc, true), ad.k, tc);
        rows_store<CK>(go, chunk_rsrc(ad.g, tc, true), ad.g, tc);
    }
    if (fast) {  // factors and the split Qt / Kt rows
        float mh[DL];  // -m log2(e), m = GC / 2
#pragma unroll
        for (int i = 0; i < DL; ++i) mh[i] = -0.5f * LOG2E * GC[i];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < DL; ++i) G[j][i] = __builtin_amdgcn_exp2f(fmaf(G[j][i], LOG2E, mh[i]));  // exp(G - m)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int i = 0; i < DL; ++i) x[j][i] *= G[j][i];
            lds_put_row<NS, DL>(sQT, L::ROWP, (4 * tg + j) * L::RS + dl0, x[j]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int i = 0; i < DL; ++i) y[j][i] *= __builtin_amdgcn_rcpf(G[j][i]);
            lds_put_row<NS, DL>(sKT, L::ROWP, (4 * tg + j) * L::RS + dl0, y[j]);
        }
    } else {  // the rows as the scan reads them, staged for the token-by-token walks
        char* stg = smem + L::OFF_QT;
        if constexpr (PREP) {
            stage_rows(stg, qo, tg, dl0);
            stage_rows(stg + 64 * 64 * sizeof(TIn), ko, tg, dl0);
            stage_rows(stg + 3 * 64 * 64 * sizeof(TIn), go, tg, dl0);
        } else {
            stage_rows(stg, cur.q, tg, dl0);
            stage_rows(stg + 64 * 64 * sizeof(TIn), cur.k, tg, dl0);
            stage_rows(stg + 3 * 64 * 64 * sizeof(TIn), cur.g, tg, dl0);
        }
        stage_rows(stg + 2 * 64 * 64 * sizeof(TIn), cur.v, tg, c0 + 4 * row);
    }
    // LDS rows of every wave; LDS only, so the write-back stores (PREP) stay in flight until the
    // wait before the flag
    lds_sync();

    // ---- the chunk's local end state P (this wave's columns, D layout) -----------------------
    const OutCtx oc = out_ctx(a, wk, h);
    const int64_t t_unc = t_unclamped - tc;  // in-chunk index of the unclamped token (or out of range)
    f32x4 P[4];
    if (fast) {
        // L = e^m (Kt^T V)
        Split8<NX> vf[2];
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) vf[k2] = lds_frag_tr<NX>(sVP, L::VPP, L::VS, 32 * k2, 0, g4, r16);
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            P[db] = zero4();
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2) {
                const Split8<NS> kf = lds_frag_tr<NS>(sKT, L::ROWP, L::RS, 32 * k2, 16 * db, g4, r16);
                P[db] = mfma_split<NS, NX, NS>(kf, vf[k2], P[db]);
            }
            const f32x4 em = *reinterpret_cast<const f32x4*>(sEM + 16 * db + 4 * g4);
#pragma unroll
            for (int i = 0; i < 4; ++i) P[db][i] *= em[i];
        }
    } else {
#pragma unroll
        for (int db = 0; db < 4; ++db) P[db] = zero4();
        walk_staged<TIn, TG, false>(smem + L::OFF_QT, nv, t_unc, c0, g4, r16, P, oc, tc);
    }

    // ---- publish the pair's map (e^{G_C(B)} e^{G_C(A)}, e^{G_C(B)} L_A + L_B) -----------------
    if (grp == 0) {
#pragma unroll
        for (int db = 0; db < 4; ++db) *reinterpret_cast<f32x4*>(sX + (db * 256 + tid) * 4) = P[db];
    }
    lds_sync();
    const float* sEG0 = reinterpret_cast<const float*>(lds + L::OFF_FAC) + DK;  // e^{G_C} of chunk A
    const int64_t slot = bh * ctl.npair + p;
    const __amdgpu_buffer_rsrc_t rL = __builtin_amdgcn_make_buffer_rsrc(
        a.ws_state + bh * ctl.npair * (int64_t)(DK * DV), (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rE =
        __builtin_amdgcn_make_buffer_rsrc(a.ws_gamma + bh * ctl.npair * DK, (short)0, 0x7fffffff, 0x00020000);
    if (grp == 1 && !last_pair) {
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        const int lo = (int)(p * (DK * DV) * 4) + tid * 16;  // [4][256 threads][4] (see fold_states)
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            const f32x4 la = *reinterpret_cast<const f32x4*>(sX + (db * 256 + tid) * 4);
            const f32x4 eb = *reinterpret_cast<const f32x4*>(sEG + 16 * db + 4 * g4);
            f32x4 m;
#pragma unroll
            for (int i = 0; i < 4; ++i) m[i] = fmaf(eb[i], la[i], P[db][i]);
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, m), rL, lo + 4096 * db, 0, 0);
        }
        if (tid < DK)
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(sEG0[tid] * sEG[tid]), rE,
                                                  (int)(p * DK * 4) + tid * 4, 0, 0);
    }
    // Stores complete (the map in this XCD's L2; PREP: the rows written back in stage 1, which
    // also precede every output of this workgroup, as o may alias g) before the flag.
    wait_vmem();
    __syncthreads();
    const uint32_t xcc = (uint32_t)__builtin_amdgcn_s_getreg(OP_HWREG_XCC_ID) & 0xfu;
    const uint32_t ep = (uint32_t)__builtin_amdgcn_readfirstlane((int)ep_word) + 1u;
    if (!last_pair && threadIdx.x == 0)
        __hip_atomic_store(ctl.flags + slot, (uint64_t)ep | ((uint64_t)xcc << 32), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    // Count this workgroup's epoch read (complete: its value is in ep).  The count wraps to zero
    // at the number of workgroups (an increment that wraps at total - 1), and the workgroup that
    // sees total - 1 counted last: every workgroup has read the epoch, so it may advance it; the
    // next call reads it after this kernel has ended.  The count orders nothing but itself and its
    // result is used only at the end, so the round trip runs under the rest of the pair (a
    // wrapping increment, unlike an add, is not rewritten into a combined add whose result the
    // wave must wait for at once).
    const uint32_t total = (uint32_t)(BH * ctl.npair);
    uint32_t counted = 0;
    if (threadIdx.x == 0) counted = __builtin_amdgcn_atomic_inc32(ctl.hdr + 1, total - 1u, __ATOMIC_RELAXED, "agent");

    // ---- while earlier pairs publish: stage 2 and the outputs' in-chunk part ------------------
    // Neither depends on the state entering the chunk: A^T tiles -> LDS, then O^T = V^T A^T.
    f32x4 Ot[4];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) Ot[tb] = zero4();
    if (fast) {
        // stage 2: causal tiles of A^T -> LDS
        {
            constexpr int MT = (10 + NW - 1) / NW;
            int sb[MT], tb[MT];
            f32x4 acc[MT];
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                tile_sb_tb(min(wave + t * NW, 9), sb[t], tb[t]);
                acc[t] = zero4();
            }
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
                Split8<NS> kf[MT], qf[MT];
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    kf[t] = lds_frag<NS>(sKT, L::ROWP, L::RS, 16 * sb[t] + r16, 32 * ks, g4);
                    qf[t] = lds_frag<NS>(sQT, L::ROWP, L::RS, 16 * tb[t] + r16, 32 * ks, g4);
                }
#pragma unroll
                for (int t = 0; t < MT; ++t) acc[t] = mfma_split<NS, NS, NS>(kf[t], qf[t], acc[t]);
            }
            f32x4 diag;
#pragma unroll
            for (int j = 0; j < 4; ++j) diag[j] = (4 * g4 + j > r16) ? 0.f : 1.f;
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const int i = wave + t * NW;
                if (i >= 10) continue;
                const f32x4 m = sb[t] == tb[t] ? diag : f32x4{1.f, 1.f, 1.f, 1.f};
                const float xx[4] = {acc[t][0] * m[0], acc[t][1] * m[1], acc[t][2] * m[2], acc[t][3] * m[3]};
                lds_put_row<NS, 4>(sAT, L::ATP, (i * 64 + lane) * 4, xx);
            }
        }
    }
    lds_sync();  // every wave's A^T tiles (both groups take it)
    // lanes j < p watch the flag word of pair j of this (sequence, head): the epoch of the call
    // that published it (low half) and the XCD its workgroup ran on (high half).  The first read
    // is issued here and checked after the in-chunk outputs.
    const uint64_t* fl = ctl.flags + bh * ctl.npair;
    uint64_t fw = 0;
    if (lane < p) fw = __hip_atomic_load(fl + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (fast) {
        Split8<NX> vf[2];
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) vf[k2] = lds_frag_tr<NX>(sVP, L::VPP, L::VS, 32 * k2, 0, g4, r16);
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {  // V^T A^T over key blocks <= tb
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2) {
                if (2 * k2 > tb) continue;
                const int i0 = tile_index(2 * k2, tb);
                const bool has_hi = 2 * k2 + 1 <= tb;
                const int i1 = has_hi ? tile_index(2 * k2 + 1, tb) : i0;
                Split8<NS> af;
#pragma unroll
                for (int pl = 0; pl < NS; ++pl) {
                    const __bf16* pp = reinterpret_cast<const __bf16*>(sAT + pl * L::ATP);
                    const bf16x4 lo = *reinterpret_cast<const bf16x4*>(pp + (i0 * 64 + lane) * 4);
                    const bf16x4 hi = *reinterpret_cast<const bf16x4*>(pp + (i1 * 64 + lane) * 4);
                    const __bf16 z = (__bf16)0.f;
                    af.p[pl] = has_hi ? bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]}
                                      : bf16x8{lo[0], lo[1], lo[2], lo[3], z, z, z, z};
                }
                Ot[tb] = mfma_split<NX, NS, NS>(vf[k2], af, Ot[tb]);
            }
        }
    }

    // ---- the state entering the chunk ------------------------------------------------------------
    f32x4 S[4];
    if (a.s0) {
        const float* s0 = a.s0 + bh * (int64_t)(DK * DV);
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) S[db][i] = s0[state_off(db, i, g4, r16, wave, DV)];
    } else {
#pragma unroll
        for (int db = 0; db < 4; ++db) S[db] = zero4();
    }
    bool same = true;  // every awaited map in this XCD's L2
    if (p > 0) {
        bool ok = false;
        for (uint32_t n = 0; n < OP_SPIN_MAX; ++n) {
            if (__all(lane >= p || (uint32_t)fw == ep)) {
                ok = true;
                same = __all(lane >= p || (uint32_t)(fw >> 32) == xcc);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
            if (lane < p) fw = __hip_atomic_load(fl + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (lane == 0 && (!ok || !same))
            __hip_atomic_fetch_or(ctl.hdr + 2, ok ? 2u : 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    f32x4 la[4];  // group 1: L_A, taken from sX before the halves pass through it
    if (grp == 1) {
#pragma unroll
        for (int db = 0; db < 4; ++db) la[db] = *reinterpret_cast<const f32x4*>(sX + (db * 256 + tid) * 4);
    }
    if (p > 0) {
        const float* maps = a.ws_state + bh * ctl.npair * (int64_t)(DK * DV);
        if (grp == 0) {
            if (same) fold_half<OP_SC0, 0>(maps, rE, sEGj, (int)p, S, g4);
            else fold_half<OP_SC1, 0>(maps, rE, sEGj, (int)p, S, g4);
        } else {
            if (same) fold_half<OP_SC0, 1>(maps, rE, sEGj, (int)p, S, g4);
            else fold_half<OP_SC1, 1>(maps, rE, sEGj, (int)p, S, g4);
        }
        // the halves through sX (thread tid of either group holds the same state entries; the
        // barrier inside the fold orders group 1's reads of L_A before these writes)
        auto put = [&](int db) { *reinterpret_cast<f32x4*>(sX + (db * 256 + tid) * 4) = S[db]; };
        auto get = [&](int db) { S[db] = *reinterpret_cast<const f32x4*>(sX + (db * 256 + tid) * 4); };
        if (grp == 0) {
            put(0);
            put(1);
        } else {
            put(2);
            put(3);
        }
        lds_sync();
        if (grp == 0) {
            get(2);
            get(3);
        } else {
            get(0);
            get(1);
        }
    }
    if (grp == 1) {  // through the pair's first chunk: S <- e^{G_C(A)} S + L_A
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            const f32x4 ea = *reinterpret_cast<const f32x4*>(sEG0 + 16 * db + 4 * g4);
#pragma unroll
            for (int i = 0; i < 4; ++i) S[db][i] = fmaf(ea[i], S[db][i], la[db][i]);
        }
    }

    // ---- outputs: O^T += (e^m S)^T Qt^T ------------------------------------------------------------
    if (fast) {
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
            const f32x4 e0 = *reinterpret_cast<const f32x4*>(sEM + 32 * ks + 4 * g4);
            const f32x4 e1 = *reinterpret_cast<const f32x4*>(sEM + 32 * ks + 16 + 4 * g4);
            float xx[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                xx[i] = S[2 * ks][i] * e0[i];
                xx[4 + i] = S[2 * ks + 1][i] * e1[i];
            }
            const Split8<NS> sf = split8<NS>(xx);
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) {
                const Split8<NS> qf = lds_frag<NS>(sQT, L::ROWP, L::RS, 16 * tb + r16, 32 * ks, g4);
                Ot[tb] = mfma_split<NS, NS, NS>(sf, qf, Ot[tb]);
            }
        }
        PendingOut pend;
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) pend.o[tb] = Ot[tb];
        pend.tc = tc;
        pend.nv = nv;
        pend.valid = true;
        // staged through this wave's own V plane (only this wave reads it, and vf is loaded)
        flush_out<OBF>(oc, c0, pend, reinterpret_cast<float*>(sVP), L::OS);
        if (has_last) {
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const f32x4 eg = *reinterpret_cast<const f32x4*>(sEG + 16 * db + 4 * g4);
#pragma unroll
                for (int i = 0; i < 4; ++i) S[db][i] = fmaf(eg[i], S[db][i], P[db][i]);
            }
        }
    } else {
        walk_staged<TIn, TG, true>(smem + L::OFF_QT, nv, t_unc, c0, g4, r16, S, oc, tc);
    }
    if (has_last && a.seq_final) {
        float* sf = a.seq_final + bh * (int64_t)(DK * DV);
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) sf[state_off(db, i, g4, r16, wave, DV)] = S[db][i];
    }

    // ---- the last workgroup to count advances the epoch (flags of this call become stale) -----
    if (threadIdx.x == 0 && counted == total - 1u)
        __hip_atomic_store(ctl.hdr, ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ev0 / ev1: if not null, events stamped with the kernel's own start and end (hipExtLaunchKernel).
template <typename TIn, typename TG, bool CK, bool PREP>
static hipError_t launch_op(const PrefillParams& a, const OnePassCtl& c, unsigned grid, hipStream_t stream,
                            hipEvent_t ev0, hipEvent_t ev1) {
    auto go = [&](auto kern) {
        if (ev0) hipExtLaunchKernelGGL(kern, dim3(grid), dim3(OP_THREADS), 0, stream, ev0, ev1, 0, a, c);
        else hipLaunchKernelGGL(kern, dim3(grid), dim3(OP_THREADS), 0, stream, a, c);
    };
    if (a.o_dt == DT_BF16) go(gla_onepass_kernel<TIn, TG, CK, PREP, true>);
    else go(gla_onepass_kernel<TIn, TG, CK, PREP, false>);
    return hipGetLastError();
}

template <typename TIn, typename TG, bool PREP>
static hipError_t launch_op_ck(const PrefillParams& a, const OnePassCtl& c, unsigned grid, hipStream_t stream,
                               hipEvent_t ev0, hipEvent_t ev1) {
    return a.T % 4 == 0 ? launch_op<TIn, TG, false, PREP>(a, c, grid, stream, ev0, ev1)
                        : launch_op<TIn, TG, true, PREP>(a, c, grid, stream, ev0, ev1);
}

// Grid: eight XCD lanes x ((sequence, head) pairs per XCD x chunk pairs).
unsigned gla_onepass_grid(int64_t BH, int64_t npair) { return (unsigned)(8 * ((BH + 7) / 8) * npair); }

int gla_onepass_max_pairs() { return OP_MAX_PAIRS; }

int gla_onepass_blocks_per_cu() {
    int nb = 0;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &nb, reinterpret_cast<const void*>(gla_onepass_kernel<_Float16, _Float16, true, true, false>), OP_THREADS, 0);
    return (e == hipSuccess && nb > 0) ? nb : 1;
}

bool gla_onepass_dtypes_ok(int io_dt, int g_dt, bool prep) {
    if (io_dt != DT_BF16 && io_dt != DT_F16) return false;
    return g_dt == io_dt || (!prep && g_dt == DT_F32);
}

hipError_t launch_gla_onepass(const PrefillParams& a, const OnePassCtl& c, int io_dt, bool prep, hipStream_t stream,
                              hipEvent_t ev0, hipEvent_t ev1) {
    const unsigned grid = gla_onepass_grid(a.n_seqs * a.H, c.npair);
    const bool g32 = a.g_dt == DT_F32;
    if (io_dt == DT_BF16) {
        if (prep) return launch_op_ck<__bf16, __bf16, true>(a, c, grid, stream, ev0, ev1);
        return g32 ? launch_op_ck<__bf16, float, false>(a, c, grid, stream, ev0, ev1)
                   : launch_op_ck<__bf16, __bf16, false>(a, c, grid, stream, ev0, ev1);
    }
    if (io_dt == DT_F16) {
        if (prep) return launch_op_ck<_Float16, _Float16, true>(a, c, grid, stream, ev0, ev1);
        return g32 ? launch_op_ck<_Float16, float, false>(a, c, grid, stream, ev0, ev1)
                   : launch_op_ck<_Float16, _Float16, false>(a, c, grid, stream, ev0, ev1);
    }
    return hipErrorInvalidValue;
}

}  // namespace triune
