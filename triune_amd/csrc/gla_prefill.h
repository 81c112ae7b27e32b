// gla_prefill.h -- chunked GLA prefill kernels for gfx950 (dense [B,T,H,D] and packed varlen):
// the device templates, instantiated by gla_prefill.hip and gla_prefill_prep.hip.
//
// Semantics (reference: triune/kernels/fast_gla.py:569-689 _run_gla_chunks, :206-316 the
// Triton TC kernel, :692-778 fast_chunk_gla dispatch):
//   S_t = diag(exp(min(g_t, 0))) S_{t-1} + k_t v_t^T ,   o_t = S_t^T q_t
// for every (sequence, head), starting from S0 (or zero), returning every o_t and S_T.
//
// Work decomposition.  A sequence is cut into segments of P chunks of 64 tokens.
//   K1 seg_state : per (segment, head) the segment's local end state from zero and its summed
//                  log-decay.
//   K2 (recurrent_scan.hip): exclusive affine scan over the segments of each (sequence, head)
//                  S_in[p+1] = exp(Gseg_p) * S_in[p] + L_p, written in place of L; final state.
//   K3 seg_output: per (segment, head) walks its chunks from S_in[p] and writes o.
// Within a chunk (C = 64 tokens, G = inclusive cumulative log-decay from the chunk start,
// m = G_C / 2 per key dim):
//   Qt = q * exp(G - m), Kt = k * exp(m - G)          (|exponents| <= span / 2)
//   A^T[s][t] = sum_d Kt[s][d] Qt[t][d]  for s <= t   (causal, diagonal included)
//   O^T = (exp(m) * S)^T Qt^T + V^T A^T
//   S  <- exp(G_C) * S + exp(m) * (Kt^T V)
// Products run on v_mfma_f32_16x16x32_bf16.  Operands that are not exactly bf16 are split
// into 2 (16-bit I/O) or 3 (fp32 I/O) bf16 parts; part products whose combined order is
// below the split depth are accumulated in fp32.
//
// One workgroup of NW = Dv/16 waves handles a (segment, head).  Per chunk:
//   stage 1  wave w (each lane 4 tokens x DPW/4 dims): cumulative decay, factors and split
//            Qt/Kt for key dims [w*DPW, (w+1)*DPW) -> token-major LDS planes; its own 16 value
//            columns of V -> a token-major plane of its own
//   stage 2  the ten 16x16 causal tiles of A^T, spread over the waves -> LDS
//   stage 3  wave w: O^T and the state update for value columns [16w, 16w+16); fragments with
//            the token as K index (Kt^T, V) come from the token-major planes through the
//            transposed LDS read
// The next chunk's inputs are loaded while the current chunk is processed: into registers, or
// (2-byte inputs at 64 x 64) q, k, g / k, g, v straight into LDS tiles of whole 128-byte rows.
// Chunks whose key-dim decay span exceeds SPAN_MAX (or that hold the reference's unclamped
// 1-token tail) run token by token on the same state registers.
#pragma once

#include "chunk_common.h"

namespace triune {

// PREP: the segment-state kernel pre-processes the raw q, k, g (see StateStep).
template <typename TIn, int DK, int DV, bool OUT, bool PREP = false>
struct Lay {
    using P = Prec<TIn>;
    static constexpr int NW = DV / 16;             // waves per workgroup
    static constexpr int DPW = DK / NW;            // key dims per wave in stage 1
    static constexpr int RS = DK + PAD;            // row stride (elements) of [token][dim] planes
    static constexpr int VS = 16;                  // row stride of a wave's [token][16 columns] V planes
    static constexpr int ROWP = CHUNK * RS * 2;    // bytes per [token][dim] plane
    static constexpr int VPP = CHUNK * VS * 2;     // bytes per V plane of one wave
    static constexpr int ATP = 10 * 64 * 4 * 2;    // bytes per plane of the ten A^T tiles
    // K3: Qt rows, Kt rows, A^T tiles.  K1: exp-weighted k rows (in the Kt slot).
    static constexpr int OFF_QT = 0;
    static constexpr int OFF_KT = OFF_QT + (OUT ? P::NS * ROWP : 0);
    static constexpr int OFF_AT = OFF_KT + P::NS * ROWP;
    static constexpr int OFF_VP = OFF_AT + (OUT ? P::NS * ATP : 0);
    static constexpr int OFF_FAC = OFF_VP + NW * P::NX * VPP;
    static constexpr int OFF_FLAG = OFF_FAC + 2 * DK * 4;
    // PREP: every wave's partial sums of squares of q and k rows, [2][NW][64 tokens] fp32
    static constexpr int OFF_NRM = OFF_FLAG + 16 * 4;
    static constexpr int BYTES = OFF_NRM + (PREP ? 2 * NW * 64 * 4 : 0);
    // fp32 staging of a wave's outputs, 16 tokens x 16 columns, row stride OS floats: the 16 lanes
    // of an LDS cycle hit distinct banks both when the MFMA layout writes and when quads read rows
    static constexpr int OS = 20;
    static_assert(DPW == 16 || DPW == 32, "stage-1 dims per wave");
    // Outputs are stored one chunk late (after the next chunk's loads are issued) where the
    // registers allow it (not at DK = 128)
    static constexpr bool DEFER = DK <= 64;
    static_assert(!DEFER || NW * 16 * OS * 4 <= P::NS * ATP, "output staging of every wave fits in the A^T planes");
    static_assert(DEFER || 16 * OS * 4 <= P::NX * VPP, "output staging fits in a wave's V planes");
    static_assert(BYTES <= 160 * 1024, "LDS budget");
};


// First of the DPW/4 consecutive key dims that lane row `row` of wave `wave` holds in stage 1.
// With the pre-processing (PREP) rows 0-1 of a quad hold low-half dims and rows 2-3 the matching
// high-half dims (d + DK/2), so a RoPE partner sits two lanes away in the same quad.
template <int DK, int DPW, bool PREP>
__device__ __forceinline__ int stage1_dim0(int wave, int row) {
    if constexpr (PREP) {
        static_assert(DPW == 16, "pre-processing needs 16 key dims per wave");
        return ((row & 2) ? DK / 2 : 0) + 8 * wave + 4 * (row & 1);
    } else {
        return wave * DPW + (DPW / 4) * row;
    }
}

// ---- stage-1 pre-processing (PREP; reference: triune/model/attention.py:14-79) -------------
// fp32 RoPE table values of a lane's four tokens at its DL key dims.
template <int DL>
struct RopeIn {
    Vec<float, DL> c[4], s[4];
};

struct RopeAddr {
    TokAddr c, s;
};

template <bool CK, int DL>
__device__ __forceinline__ void rope_load(RopeIn<DL>& r, const RopeAddr& ad, int64_t tc, bool valid) {
    rows_load<CK>(r.c, chunk_rsrc(ad.c, tc, valid), ad.c, tc);
    rows_load<CK>(r.s, chunk_rsrc(ad.s, tc, valid), ad.s, tc);
}

// Sum of squares of a lane's DL values per token, summed over its quad (this wave's 16 dims of
// the token) and stored by row 0 of the quad as this wave's partial: sp[token].
template <int DL>
__device__ __forceinline__ void norm_partials(const float (&x)[4][DL], float* sp, int tg, int row) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float q = 0.f;
#pragma unroll
        for (int i = 0; i < DL; ++i) q = fmaf(x[j][i], x[j][i], q);
        q = dpp_add<0xB1>(q);  // quad_perm [1, 0, 3, 2]
        q = dpp_add<0x4E>(q);  // quad_perm [2, 3, 0, 1]
        if (row == 0) sp[4 * tg + j] = q;
    }
}

// 1 / max(||row||, 1e-6) of token t from the NW waves' partials sp[w * 64 + t].
template <int NW>
__device__ __forceinline__ float token_inv_norm(const float* sp, int t) {
    float n = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) n += sp[w * 64 + t];
    return inv_norm(n);
}

// RoPE in place: out[d] = x[d] cos[d] - x[d + DK/2] sin[d] (low half), out[d + DK/2] =
// x[d + DK/2] cos[d + DK/2] + x[d] sin[d + DK/2] (high half); the partner value is lane ^ 2's.
template <int DL>
__device__ __forceinline__ void rope_rows(float (&x)[4][DL], const RopeIn<DL>& r, int row) {
    const float sgn = (row & 2) ? 1.f : -1.f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < DL; ++i) {
            const float p = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x[j][i]), 0x4E, 0xf, 0xf, false));
            x[j][i] = fmaf(sgn * p, __uint_as_float(r.s[j].w[i]), x[j][i] * __uint_as_float(r.c[j].w[i]));
        }
}

// Rows at or past nv (zeros from the loads) must stay zero after elu(x) + 1 and logsigmoid.
template <int DL>
__device__ __forceinline__ void zero_rows_past(float (&x)[4][DL], int tg, int nv) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const bool ok = 4 * tg + j < nv;
#pragma unroll
        for (int i = 0; i < DL; ++i) x[j][i] = ok ? x[j][i] : 0.f;
    }
}

// ---------------------------------------------------------------------------------------
// Token-by-token update of one wave's state columns (large decay spans, unclamped tail).
// S tile db holds S[16*db + 4*g4 + i][c0 + r16].
// ---------------------------------------------------------------------------------------
template <typename TIn, typename TG, int DK, bool OUT>
__device__ void chunk_tokenwise(const PrefillParams& a, const Work& wk, int64_t h, int c0, int64_t tc, int nv,
                                int g4, int r16, f32x4 (&S)[DK / 16]) {
    constexpr int NDB = DK / 16;
    for (int t = 0; t < nv; ++t) {
        const int64_t tt = tc + t;
        const bool unclamped = (a.flags & 1) && (tt == wk.len - 1);
        float dcy[NDB][4], kk[NDB][4], qq[NDB][4];
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            const int d = 16 * db + 4 * g4;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float gg = (float)tok_row<TG>(a.g, wk, tt, h, d)[i];
                dcy[db][i] = expf(unclamped ? gg : fminf(gg, 0.f));
                kk[db][i] = (float)tok_row<TIn>(a.k, wk, tt, h, d)[i];
                qq[db][i] = OUT ? (float)tok_row<TIn>(a.q, wk, tt, h, d)[i] : 0.f;
            }
        }
        const float vv = (float)tok_row<TIn>(a.v, wk, tt, h, c0)[r16];
        float part = 0.f;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float s = dcy[db][i] * S[db][i] + kk[db][i] * vv;
                S[db][i] = s;
                part += qq[db][i] * s;
            }
        if (OUT) {
            part += __shfl_xor(part, 16);
            part += __shfl_xor(part, 32);
            // o may alias g (the reference's VectorisedGLA passes out=g): every wave has read
            // token tt's gates before any wave overwrites them with outputs
            __syncthreads();
            if (g4 == 0) {
                const int64_t off = wk.b * a.o_sb + (wk.row0 + tt) * a.o_st + h * a.o_sh + c0 + r16;
                char* op = reinterpret_cast<char*>(a.o) + off * dt_size(a.o_dt);
                if (a.o_dt == DT_F32) *reinterpret_cast<float*>(op) = part;
                else if (a.o_dt == DT_BF16) *reinterpret_cast<__bf16*>(op) = (__bf16)part;
                else *reinterpret_cast<_Float16*>(op) = (_Float16)part;
            }
        }
    }
}

// Outputs of one chunk for a wave's 16 columns (lane (g4, r16) holds O[token 16*tb + r16]
// [columns 4*g4 .. 4*g4+3]), kept in registers until the next chunk has issued its loads.  On gfx9
// one counter tracks loads and stores, and a wait for a load while a store is outstanding drains
// both; stores issued right after the next loads are long complete when those loads are waited
// for, one chunk later.
// The output rows of one (sequence, head): token 0's address and the token stride in bytes, made
// once per workgroup so the chunk loop keeps two scalars instead of the output's strides.
struct OutCtx {
    char* op;
    int64_t ost;
    int dt;
};

__device__ __forceinline__ OutCtx out_ctx(const PrefillParams& a, const Work& wk, int64_t h) {
    OutCtx o;
    const int64_t es = dt_size(a.o_dt);
    o.op = reinterpret_cast<char*>(a.o) + uniform_i64((wk.b * a.o_sb + wk.row0 * a.o_st + h * a.o_sh) * es);
    o.ost = uniform_i64(a.o_st * es);
    o.dt = a.o_dt;
    return o;
}

// chunk_tokenwise for the output walk, reading rows through the walk's token-0 addresses (ad) and
// writing through oc; t_unclamped: the token whose gate stays unclamped (-1: none).
template <typename TIn, typename TG, int DK>
__device__ void chunk_tokenwise_out(const ChunkAddr& ad, const OutCtx& oc, int64_t t_unclamped, int c0, int64_t tc,
                                    int nv, int g4, int r16, f32x4 (&S)[DK / 16]) {
    constexpr int NDB = DK / 16;
    const int oes = dt_size(oc.dt);
    for (int t = 0; t < nv; ++t) {
        const int64_t tt = tc + t;
        const bool unclamped = tt == t_unclamped;
        const TG* gr = reinterpret_cast<const TG*>(ad.g.p0 + tt * ad.g.st);
        const TIn* kr = reinterpret_cast<const TIn*>(ad.k.p0 + tt * ad.k.st);
        const TIn* qr = reinterpret_cast<const TIn*>(ad.q.p0 + tt * ad.q.st);
        float dcy[NDB][4], kk[NDB][4], qq[NDB][4];
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int d = 16 * db + 4 * g4 + i;
                const float gg = (float)gr[d];
                dcy[db][i] = fast_exp(unclamped ? gg : min0(gg));
                kk[db][i] = (float)kr[d];
                qq[db][i] = (float)qr[d];
            }
        const float vv = (float)reinterpret_cast<const TIn*>(ad.v.p0 + tt * ad.v.st)[c0 + r16];
        float part = 0.f;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float s = dcy[db][i] * S[db][i] + kk[db][i] * vv;
                S[db][i] = s;
                part += qq[db][i] * s;
            }
        part += __shfl_xor(part, 16);
        part += __shfl_xor(part, 32);
        // o may alias g (the reference's VectorisedGLA passes out=g): every wave has read token
        // tt's gates before any wave overwrites them with outputs
        __syncthreads();
        if (g4 == 0) {
            char* op = oc.op + tt * oc.ost + (int64_t)(c0 + r16) * oes;
            if (oc.dt == DT_F32) *reinterpret_cast<float*>(op) = part;
            else if (oc.dt == DT_BF16) *reinterpret_cast<__bf16*>(op) = (__bf16)part;
            else *reinterpret_cast<_Float16*>(op) = (_Float16)part;
        }
    }
}

struct PendingOut {
    f32x4 o[4];
    int64_t tc;
    int nv;
    bool valid;
};

// Stage the pending outputs 16 tokens at a time through `stage` (this wave's 16 x OS floats of
// LDS) and store them with the four lanes of a quad covering one token's 16 columns.
template <bool OBF>
__device__ __forceinline__ void flush_out(const OutCtx& oc, int c0, const PendingOut& p, float* stage, int os) {
    const int lane = threadIdx.x & 63, r16 = lane & 15, g4 = lane >> 4;
    const int es = OBF ? 2 : dt_size(oc.dt);
    const int64_t ost = oc.ost;
    char* obase = oc.op + p.tc * ost + c0 * es;
    const int q = lane & 3, tq = (lane >> 4) + 4 * ((lane >> 2) & 3);  // token within 16
    const int32_t olane = (int32_t)(tq * ost) + 4 * q * es;
    const OutRsrc orr = out_rsrc(obase, ost, es, p.nv, !OBF && oc.dt == DT_F32);
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
        *reinterpret_cast<f32x4*>(stage + r16 * os + 4 * g4) = p.o[tb];
        const f32x4 x = *reinterpret_cast<const f32x4*>(stage + tq * os + 4 * q);
        if constexpr (OBF) {  // bf16 outputs known at compile time: one store of four packed values
            typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
            const u32x2 w = __builtin_bit_cast(u32x2, bf16x4{(__bf16)x[0], (__bf16)x[1], (__bf16)x[2], (__bf16)x[3]});
            __builtin_amdgcn_raw_buffer_store_b64(w, orr.lo, (int32_t)(16 * tb * ost) + olane, 0, 0);
        } else {
            out_store4(orr, (int32_t)(16 * tb * ost) + olane, oc.dt, x);
        }
    }
}

// CK: checked row addressing (see chunk_load); without it the loads zero rows past the chunk.
template <typename TIn, typename TG, int DK, int DV, bool CK, bool OBF = false>
struct OutStep {
    using L = Lay<TIn, DK, DV, true>;
    using PR = Prec<TIn>;
    static constexpr int NW = L::NW, DPW = L::DPW, DL = DPW / 4, NDB = DK / 16, NKS = DK / 32;
    static constexpr int NS = PR::NS, NX = PR::NX;
    // q, k, g arrive as LDS tiles (tile_dma) instead of registers, v stays in registers; where the
    // tiles keep the kernel's workgroups per CU (MINB: two at 64, fp16's two V planes excluded)
    static constexpr int RB = DK * 2, TB = CHUNK * RB, FB = 0;
    static constexpr int MINB = (PR::NS == 3 || DK == 128) ? 1 : 2;
    static constexpr bool DMA = tile_dma_inputs<TIn, TG, DK, DV>() && L::BYTES + 3 * TB <= 160 * 1024 / MINB;

    // One chunk: stage 1 (factors, split operands -> LDS), stage 2 (A^T tiles), stage 3 (O, S).
    // after_inputs() runs once stage 1 has consumed `cur` (it may refill those registers);
    // DMA: stage 1 first takes q, k, g from `tiles`, and issue_tiles() runs once every wave has
    // read them (it may refill the tiles).
    // FAST_ONLY: a chunk that needs the token-by-token path returns false right after stage 1
    // (its inputs consumed, the next chunk's loads issued, the pending outputs stored) and the
    // caller finishes it with finish_tokenwise; otherwise both paths are handled here.
    // oc / ad: the walk's output and input addresses (the token-wise path reads rows through them);
    // t_unclamped: the token whose gate stays unclamped (-1: none).
    template <bool FAST_ONLY, typename Hook, typename TileHook>
    __device__ static bool run(const OutCtx& oc, const ChunkAddr& ad, int64_t t_unclamped, int64_t tc, int nv,
                               ChunkIn<TIn, TG, DL>& cur, f32x4 (&S)[NDB], char* smem, const char* tiles,
                               PendingOut& pend, Hook&& after_inputs, TileHook&& issue_tiles) {
        const int lane = threadIdx.x & 63, wave = wave_id(), r16 = lane & 15, g4 = lane >> 4;
        const int tg = lane >> 2, row = lane & 3;
        const int d0 = wave * DPW, c0 = wave * 16;
        const int dl0 = d0 + DL * row;  // first key dim of this lane in stage 1
        char* sQT = smem + L::OFF_QT;
        char* sKT = smem + L::OFF_KT;
        char* sAT = smem + L::OFF_AT;
        char* sVP = smem + L::OFF_VP + wave * NX * L::VPP;
        float* sEM = reinterpret_cast<float*>(smem + L::OFF_FAC);
        float* sEG = sEM + DK;
        int* sFLAG = reinterpret_cast<int*>(smem + L::OFF_FLAG);
        const bool tail_unclamped = t_unclamped == tc + nv - 1;

        // Issue priority: stage 1 (throughput work: factors, splits, the previous chunk's stores) at
        // the base level, stages 2-3 (the MFMA chains that carry the state) one level up, so of the
        // two workgroups on a CU the one in stages 2-3 issues first and the other fills its gaps
        // (config-1 pass 120.9 -> 118.2 us, output kernel 76.1 -> 72.3 us by events, same-box A/B).
        __builtin_amdgcn_s_setprio(0);
        // ---------------- stage 1 -------------------------------------------------------
        if constexpr (DMA) {
            wait_vmem();  // this wave's tile pieces (and v rows) of the chunk have landed ...
            lds_sync();  // ... and every other wave's
            tile_rows<RB, FB>(cur.q, tiles, tg, dl0);
            tile_rows<RB, FB>(cur.k, tiles + TB, tg, dl0);
            tile_rows<RB, FB>(cur.g, tiles + 2 * TB, tg, dl0);
        }
        {
            float G[4][DL], GC[DL], x[4][DL];
            chunk_float<CK>(cur.g, G, tg, nv);
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int i = 0; i < DL; ++i) G[j][i] = min0(G[j][i]);
            chunk_cumsum<DL>(G, GC, lane);
            bool bad = tail_unclamped;
#pragma unroll
            for (int i = 0; i < DL; ++i) bad |= !(GC[i] >= -SPAN_MAX);
            float mh[DL];  // -m log2(e), m = GC / 2
#pragma unroll
            for (int i = 0; i < DL; ++i) mh[i] = -0.5f * LOG2E * GC[i];
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int i = 0; i < DL; ++i) G[j][i] = __builtin_amdgcn_exp2f(fmaf(G[j][i], LOG2E, mh[i]));  // exp(G - m)
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
            // Qt rows
            chunk_float<CK>(cur.q, x, tg, nv);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int i = 0; i < DL; ++i) x[j][i] *= G[j][i];
                lds_put_row<NS, DL>(sQT, L::ROWP, (4 * tg + j) * L::RS + dl0, x[j]);
            }
            // Kt rows (stage 2 reads them as rows, the state update through the transposed read)
            chunk_float<CK>(cur.k, x, tg, nv);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int i = 0; i < DL; ++i) x[j][i] *= __builtin_amdgcn_rcpf(G[j][i]);
                lds_put_row<NS, DL>(sKT, L::ROWP, (4 * tg + j) * L::RS + dl0, x[j]);
            }
            // V rows: tokens 4*tg + j, this wave's columns 4*row .. 4*row+3
            lds_put_v_rows<TIn, NX, CK>(sVP, L::VPP, L::VS, 4 * row, cur.v, tg, nv);
        }
        // The next chunk's loads go out now and fly during stages 2-3, except at (128, 128),
        // where their registers would push the wave past 256 VGPRs: there they go out after stage 3.
        constexpr bool late_refill = DK == 128 && DV == 128 && !DMA;
        if constexpr (!late_refill) after_inputs();
        // The previous chunk's outputs, staged through this wave's slice of the A^T planes
        // (nothing reads them again before this chunk's stage 2).
        if (pend.valid) flush_out<OBF>(oc, c0, pend, reinterpret_cast<float*>(sAT) + wave * 16 * L::OS, L::OS);
        pend.valid = false;
        block_sync<DMA>();
        if constexpr (DMA) issue_tiles();  // every wave has read this chunk's tiles
        __builtin_amdgcn_s_setprio(1);
        bool fast = true;
#pragma unroll
        for (int w = 0; w < NW; ++w) fast = fast && (sFLAG[w] == 0);

        if constexpr (FAST_ONLY) {
            if (!fast) return false;
        }
        if (!FAST_ONLY && !fast) {
            chunk_tokenwise_out<TIn, TG, DK>(ad, oc, t_unclamped, c0, tc, nv, g4, r16, S);
        } else {
            // ---------------- stage 2: causal tiles of A^T -> LDS ----------------------------
            // Wave w owns tiles w, w + NW, ...: all of them are computed together (independent
            // MFMA chains); a wave with one tile fewer recomputes its last tile and skips the store.
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
                // causal mask of a diagonal tile (row = key 4*g4 + j, column = query r16) as factors
                f32x4 diag;
#pragma unroll
                for (int j = 0; j < 4; ++j) diag[j] = (4 * g4 + j > r16) ? 0.f : 1.f;
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    const int i = wave + t * NW;
                    if (i >= 10) continue;
                    const f32x4 m = sb[t] == tb[t] ? diag : f32x4{1.f, 1.f, 1.f, 1.f};
                    const float x[4] = {acc[t][0] * m[0], acc[t][1] * m[1], acc[t][2] * m[2], acc[t][3] * m[3]};
                    lds_put_row<NS, 4>(sAT, L::ATP, (i * 64 + lane) * 4, x);
                }
            }
            block_sync<DMA>();

            // ---------------- stage 3: outputs and state for columns [c0, c0+16) ------------
            Split8<NX> vf[2];
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2) vf[k2] = lds_frag_tr<NX>(sVP, L::VPP, L::VS, 32 * k2, 0, g4, r16);
            f32x4 Ot[4];
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) Ot[tb] = zero4();
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {  // (exp(m) S)^T Qt^T
                const f32x4 e0 = *reinterpret_cast<const f32x4*>(sEM + 32 * ks + 4 * g4);
                const f32x4 e1 = *reinterpret_cast<const f32x4*>(sEM + 32 * ks + 16 + 4 * g4);
                float x[8];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    x[i] = S[2 * ks][i] * e0[i];
                    x[4 + i] = S[2 * ks + 1][i] * e1[i];
                }
                const Split8<NS> sf = split8<NS>(x);
#pragma unroll
                for (int tb = 0; tb < 4; ++tb) {
                    const Split8<NS> qf = lds_frag<NS>(sQT, L::ROWP, L::RS, 16 * tb + r16, 32 * ks, g4);
                    Ot[tb] = mfma_split<NS, NS, NS>(sf, qf, Ot[tb]);
                }
            }
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
                        const __bf16* p = reinterpret_cast<const __bf16*>(sAT + pl * L::ATP);
                        const bf16x4 lo = *reinterpret_cast<const bf16x4*>(p + (i0 * 64 + lane) * 4);
                        const bf16x4 hi = *reinterpret_cast<const bf16x4*>(p + (i1 * 64 + lane) * 4);
                        const __bf16 z = (__bf16)0.f;
                        af.p[pl] = has_hi ? bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]}
                                          : bf16x8{lo[0], lo[1], lo[2], lo[3], z, z, z, z};
                    }
                    Ot[tb] = mfma_split<NX, NS, NS>(vf[k2], af, Ot[tb]);
                }
            }
#pragma unroll
            for (int db = 0; db < NDB; ++db) {  // S <- exp(G_C) S + exp(m) Kt^T V
                f32x4 P = zero4();
#pragma unroll
                for (int k2 = 0; k2 < 2; ++k2) {
                    const Split8<NS> kf = lds_frag_tr<NS>(sKT, L::ROWP, L::RS, 32 * k2, 16 * db, g4, r16);
                    P = mfma_split<NS, NX, NS>(kf, vf[k2], P);
                }
                const f32x4 em = *reinterpret_cast<const f32x4*>(sEM + 16 * db + 4 * g4);
                const f32x4 eg = *reinterpret_cast<const f32x4*>(sEG + 16 * db + 4 * g4);
#pragma unroll
                for (int i = 0; i < 4; ++i) S[db][i] = eg[i] * S[db][i] + em[i] * P[i];
            }
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) pend.o[tb] = Ot[tb];
            pend.tc = tc;
            pend.nv = nv;
            pend.valid = true;
            if constexpr (!L::DEFER) {  // store now, staged through this wave's own V planes
                flush_out<OBF>(oc, c0, pend, reinterpret_cast<float*>(sVP), L::OS);
                pend.valid = false;
            }
        }
        if constexpr (late_refill) after_inputs();
        // the next chunk rewrites LDS (DMA: after the barrier that opens it)
        if constexpr (!DMA) __syncthreads();
        return true;
    }

    // The rest of a chunk that run<true> returned false for.
    template <typename Hook>
    __device__ static void finish_tokenwise(const OutCtx& oc, const ChunkAddr& ad, int64_t t_unclamped, int64_t tc,
                                            int nv, f32x4 (&S)[NDB], Hook&& after_inputs) {
        const int lane = threadIdx.x & 63, r16 = lane & 15, g4 = lane >> 4;
        chunk_tokenwise_out<TIn, TG, DK>(ad, oc, t_unclamped, wave_id() * 16, tc, nv, g4, r16, S);
        constexpr bool late_refill = DK == 128 && DV == 128 && !DMA;
        if constexpr (late_refill) after_inputs();
        block_sync<DMA>();
    }
};

// Outputs of one segment from its carried-in state S (K3).
template <typename TIn, typename TG, int DK, int DV, bool CK, bool OBF>
__device__ void segment_walk(const PrefillParams& a, const Work& wk, int64_t h, f32x4 (&S)[DK / 16], char* smem,
                             char* tiles) {
    using St = OutStep<TIn, TG, DK, DV, CK, OBF>;
    constexpr int DL = St::DL;
    const int lane = threadIdx.x & 63, wave = wave_id(), tg = lane >> 2, row = lane & 3;
    const ChunkAddr ad = chunk_addr<true, TIn, TG>(a, wk, h, tg, wave * St::DPW + DL * row, wave * 16 + 4 * row);
    const int64_t nch = (wk.t_end - wk.t_begin + CHUNK - 1) / CHUNK;
    auto chunk_nv = [&](int64_t c) {
        const int64_t r = wk.t_end - (wk.t_begin + c * CHUNK);
        return (int)(r < CHUNK ? r : CHUNK);
    };
    auto tok = [&](int64_t c) { return wk.t_begin + c * CHUNK; };
    // One register set: stage 1 consumes it and the next chunk's loads refill it at once, so they
    // are in flight during stages 2-3 (registers go to occupancy instead of a second set).
    const OutCtx oc = out_ctx(a, wk, h);
    const int64_t t_unclamped = (a.flags & 1) ? wk.len - 1 : -1;
    ChunkIn<TIn, TG, DL> A;
    // DMA: q, k, g of chunk c go to the tiles (issued once stage 1 of chunk c - 1 has read them),
    // v rows to registers; otherwise every input to registers.
    auto refill = [&](int64_t c1) {
        if constexpr (St::DMA) rows_load<CK>(A.v, chunk_rsrc(ad.v, tok(c1), c1 < nch), ad.v, tok(c1));
        else chunk_load<true, CK>(A, ad, tok(c1), c1 < nch);
    };
    auto tiles_for = [&](int64_t c1) {
        if constexpr (St::DMA)
            if (c1 < nch) chunk_tiles<true, St::RB, St::FB>(tiles, ad, tok(c1), wave, lane);
    };
    tiles_for(0);
    refill(0);
    PendingOut pend;
    pend.valid = false;
    // Chunks take the MFMA path until one needs the token-by-token path (a decay span beyond the
    // factored range, or the unclamped tail); from there a loop that handles both finishes the
    // segment.  The fast loop has no merge with the token-wise code, so its state registers stay put.
    int64_t c = 0;
    for (; c < nch; ++c)
        if (!St::template run<true>(oc, ad, t_unclamped, tok(c), chunk_nv(c), A, S, smem, tiles, pend,
                                    [&] { refill(c + 1); }, [&] { tiles_for(c + 1); }))
            break;
    if (c < nch) {
        St::finish_tokenwise(oc, ad, t_unclamped, tok(c), chunk_nv(c), S, [&] { refill(c + 1); });
        for (++c; c < nch; ++c)
            St::template run<false>(oc, ad, t_unclamped, tok(c), chunk_nv(c), A, S, smem, tiles, pend,
                                    [&] { refill(c + 1); }, [&] { tiles_for(c + 1); });
    }
    if constexpr (St::DMA) lds_sync();  // DMA: no closing barrier after a chunk
    if (pend.valid)  // after the last chunk's closing barrier the A^T planes are free
        flush_out<OBF>(oc, wave * 16, pend, reinterpret_cast<float*>(smem + St::L::OFF_AT) + wave * 16 * St::L::OS,
                       St::L::OS);
}

// ---------------------------------------------------------------------------------------
// Segment-local end state, chunks walked last to first.  With the decay of the later chunks
// (sfx) known, every token's weight exp(sfx + G_C - G_t) = exp(decay from after t to the segment
// end) is at most 1 (or e^{g} of an unclamped tail token), so the state accumulates directly in
// the MFMA accumulators:  L += (k * weight)^T V  - no per-chunk rescale, no overflow guard.
// L tile db holds L[16*db + 4*g4 + i][16*w + r16]; Gseg[i] = summed log-decay of key dim
// d0 + DL*row + i of the segment.
// ---------------------------------------------------------------------------------------
// PREP (VectorisedGLA's prefill, attention.py:425-451): q, k, g arrive as raw projections.  Stage 1
// forms q, k <- RoPE(normalize(elu(x) + 1)) and g <- logsigmoid(g) in fp32, rounds them to the I/O
// dtype, writes them back over the inputs (the reference's in-place pre-processing,
// attention.py:14-79) and uses the rounded k and g for the segment state, so the output kernel that
// follows reads exactly what the reference's scan would.  A row's norm spans the NW waves' dims:
// each wave stores its partial sums of squares and a barrier inside stage 1 separates the stores
// from the reads.
// Pre-processed q, k, g rows of one chunk waiting to be written back (PREP with tiles: a chunk's
// rows go out at the start of the next step, right after its wait for the tiles, so that wait -
// vector memory operations complete in order - never includes stores issued just before it).
template <typename TIn, typename TG, int DL>
struct PrepOut {
    Vec<TIn, DL> q[4], k[4];
    Vec<TG, DL> g[4];
    int64_t tc;
    bool valid;
};

template <bool CK, typename TIn, typename TG, int DL>
__device__ __forceinline__ void prep_out_store(PrepOut<TIn, TG, DL>& po, const ChunkAddr& ad) {
    if (!po.valid) return;
    rows_store<CK>(po.q, chunk_rsrc(ad.q, po.tc, true), ad.q, po.tc);
    rows_store<CK>(po.k, chunk_rsrc(ad.k, po.tc, true), ad.k, po.tc);
    rows_store<CK>(po.g, chunk_rsrc(ad.g, po.tc, true), ad.g, po.tc);
    po.valid = false;
}

template <typename TIn, typename TG, int DK, int DV, bool CK, bool PREP = false>
struct StateStep {
    using L = Lay<TIn, DK, DV, false, PREP>;
    using PR = Prec<TIn>;
    static constexpr int NW = L::NW, DPW = L::DPW, DL = DPW / 4, NDB = DK / 16, NS = PR::NS, NX = PR::NX;
    // Inputs arrive as LDS tiles (tile_dma) where the tiles keep the workgroups per CU the plan
    // assumes (two at 64 x 64; at 128 x 128 the registers already hold one per CU): k, g, v in two
    // tile sets, the next chunk's in flight during this one; PREP: q, k, g, v in one set, the next
    // chunk's issued once every wave has read this one (at the norm-partials barrier).
    static constexpr int RB = DK * 2, TB = CHUNK * RB;
    static constexpr int NT = PREP ? 4 : 6;  // tiles of the kernel
    // unit-index bit that varies within a quad row's stage-1 read (stage1_dim0)
    static constexpr int FB = !PREP ? 0 : (RB == 128 ? 2 : 3);
    static constexpr bool DMA =
        tile_dma_inputs<TIn, TG, DK, DV>() && L::BYTES + NT * TB <= (DK == 128 ? 160 : 80) * 1024;

    // PREP: rc holds this chunk's RoPE table rows; once consumed, the rows of chunk tc_next (the
    // chunk walked after this one) are loaded into it.
    // DMA: the chunk's k, g, v come from `tiles`; issue_next() runs once every wave is past the
    // previous chunk (it may refill the other tile set).
    template <typename Hook, typename TileHook>
    __device__ static void run(const PrefillParams& a, const Work& wk, int64_t tc, int nv,
                               ChunkIn<TIn, TG, DL>& cur, const ChunkAddr& ad, const RopeAddr& rad,
                               RopeIn<DL>& rc, int64_t tc_next, bool next_valid, f32x4 (&Lst)[NDB],
                               float (&Gseg)[DL], char* smem, const char* tiles, PrepOut<TIn, TG, DL>& po,
                               Hook&& after_inputs, TileHook&& issue_next) {
        const int lane = threadIdx.x & 63, wave = wave_id(), r16 = lane & 15, g4 = lane >> 4;
        const int tg = lane >> 2, row = lane & 3;
        const int dl0 = stage1_dim0<DK, DPW, PREP>(wave, row);
        char* sKW = smem + L::OFF_KT;  // exp-weighted k rows
        char* sVP = smem + L::OFF_VP + wave * NX * L::VPP;
        if constexpr (DMA) {
            wait_vmem();  // this wave's tile pieces of the chunk have landed ...
            lds_sync();  // ... and every other wave's; every wave is done with the other set
            if constexpr (PREP) {
                prep_out_store<CK>(po, ad);  // the previous chunk's pre-processed rows
                tile_rows<RB, FB>(cur.q, tiles, tg, dl0);
                tile_rows<RB, FB>(cur.k, tiles + TB, tg, dl0);
                tile_rows<RB, FB>(cur.g, tiles + 2 * TB, tg, dl0);
                tile_rows<RB, FB>(cur.v, tiles + 3 * TB, tg, wave * 16 + 4 * row);
            } else {
                issue_next();
                tile_rows<RB, FB>(cur.k, tiles, tg, dl0);
                tile_rows<RB, FB>(cur.g, tiles + TB, tg, dl0);
                tile_rows<RB, FB>(cur.v, tiles + 2 * TB, tg, wave * 16 + 4 * row);
            }
        }
        if constexpr (PREP) {
            float* sNRM = reinterpret_cast<float*>(smem + L::OFF_NRM);
            float G[4][DL], GC[DL], x[4][DL], y[4][DL];  // g, q, k
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
            norm_partials<DL>(x, sNRM + wave * 64, tg, row);
            norm_partials<DL>(y, sNRM + (NW + wave) * 64, tg, row);
            lds_put_v_rows<TIn, NX, CK>(sVP, L::VPP, L::VS, 4 * row, cur.v, tg, nv);
            block_sync<DMA>();  // every wave's norm partials (and every wave has read the tiles)
            if constexpr (DMA) issue_next();
            if (a.use_rope) {
                rope_rows<DL>(x, rc, row);
                rope_rows<DL>(y, rc, row);
            }
            rope_load<CK>(rc, rad, tc_next, next_valid && a.use_rope != 0);
            Vec<TIn, DL> qo[4], ko[4];
            Vec<TG, DL> go[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float iq = token_inv_norm<NW>(sNRM, 4 * tg + j), ik = token_inv_norm<NW>(sNRM + NW * 64, 4 * tg + j);
#pragma unroll
                for (int i = 0; i < DL; ++i) {
                    x[j][i] *= iq;
                    y[j][i] *= ik;
                }
                vec_pack<TIn, DL>(x[j], qo[j]);
                vec_pack<TIn, DL>(y[j], ko[j]);
                vec_pack<TG, DL>(G[j], go[j]);
            }
            if constexpr (DMA) {  // written back at the start of the next step (or after the walk)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    po.q[j] = qo[j];
                    po.k[j] = ko[j];
                    po.g[j] = go[j];
                }
                po.tc = tc;
                po.valid = true;
            } else {
                rows_store<CK>(qo, chunk_rsrc(ad.q, tc, true), ad.q, tc);
                rows_store<CK>(ko, chunk_rsrc(ad.k, tc, true), ad.k, tc);
                rows_store<CK>(go, chunk_rsrc(ad.g, tc, true), ad.g, tc);
            }
            // the state from the rounded values, as the output kernel will see them
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                vec_float(ko[j], y[j]);
                vec_float(go[j], G[j]);
            }
            float X[4][DL];
            chunk_suffix<DL>(G, X, GC, lane);
            float gs[DL];  // Gseg log2(e)
#pragma unroll
            for (int i = 0; i < DL; ++i) gs[i] = Gseg[i] * LOG2E;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int i = 0; i < DL; ++i) y[j][i] *= __builtin_amdgcn_exp2f(fmaf(X[j][i], LOG2E, gs[i]));
                lds_put_row<NS, DL>(sKW, L::ROWP, (4 * tg + j) * L::RS + dl0, y[j]);
            }
#pragma unroll
            for (int i = 0; i < DL; ++i) Gseg[i] += GC[i];
        } else {
            float G[4][DL], GC[DL], x[4][DL];
            chunk_float<CK>(cur.g, x, tg, nv);
            const bool tail_chunk = (a.flags & 1) && (tc + nv == wk.len);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bool unclamped = tail_chunk && (4 * tg + j == nv - 1);
#pragma unroll
                for (int i = 0; i < DL; ++i) G[j][i] = unclamped ? x[j][i] : min0(x[j][i]);
            }
            float X[4][DL];
            chunk_suffix<DL>(G, X, GC, lane);
            chunk_float<CK>(cur.k, x, tg, nv);
            float gs[DL];  // Gseg log2(e)
#pragma unroll
            for (int i = 0; i < DL; ++i) gs[i] = Gseg[i] * LOG2E;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int i = 0; i < DL; ++i) x[j][i] *= __builtin_amdgcn_exp2f(fmaf(X[j][i], LOG2E, gs[i]));
                lds_put_row<NS, DL>(sKW, L::ROWP, (4 * tg + j) * L::RS + dl0, x[j]);
            }
#pragma unroll
            for (int i = 0; i < DL; ++i) Gseg[i] += GC[i];
            lds_put_v_rows<TIn, NX, CK>(sVP, L::VPP, L::VS, 4 * row, cur.v, tg, nv);
        }
        after_inputs();
        block_sync<DMA>();
        Split8<NX> vf[2];
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) vf[k2] = lds_frag_tr<NX>(sVP, L::VPP, L::VS, 32 * k2, 0, g4, r16);
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2) {
                const Split8<NS> kf = lds_frag_tr<NS>(sKW, L::ROWP, L::RS, 32 * k2, 16 * db, g4, r16);
                Lst[db] = mfma_split<NS, NX, NS>(kf, vf[k2], Lst[db]);
            }
        // the next chunk rewrites LDS (DMA: after the barrier that opens it)
        if constexpr (!DMA) __syncthreads();
    }
};

template <typename TIn, typename TG, int DK, int DV, bool CK, bool PREP = false>
__device__ void segment_state_walk(const PrefillParams& a, const Work& wk, int64_t h, f32x4 (&Lst)[DK / 16],
                                   float (&Gseg)[DK / (DV / 16) / 4], char* smem, char* tiles) {
    using St = StateStep<TIn, TG, DK, DV, CK, PREP>;
    constexpr int DL = St::DL;
    const int lane = threadIdx.x & 63, wave = wave_id(), tg = lane >> 2, row = lane & 3;
    const int dl0 = stage1_dim0<DK, St::DPW, PREP>(wave, row);
    // PREP also reads q (and writes q, k, g back)
    const ChunkAddr ad = chunk_addr<PREP, TIn, TG>(a, wk, h, tg, dl0, wave * 16 + 4 * row);
    RopeAddr rad{};
    if constexpr (PREP) {
        rad.c = tok_addr<float>(a.cs, wk, h, tg, dl0);
        rad.s = tok_addr<float>(a.sn, wk, h, tg, dl0);
    }
    const int64_t nch = (wk.t_end - wk.t_begin + CHUNK - 1) / CHUNK;
    auto chunk_nv = [&](int64_t c) {
        const int64_t r = wk.t_end - (wk.t_begin + c * CHUNK);
        return (int)(r < CHUNK ? r : CHUNK);
    };
    auto tok = [&](int64_t c) { return wk.t_begin + c * CHUNK; };
    ChunkIn<TIn, TG, DL> A, B;
    RopeIn<DL> R;  // PREP: the RoPE table rows of the chunk being walked, loaded one chunk ahead
    PrepOut<TIn, TG, DL> po;
    po.valid = false;
    if constexpr (St::DMA && PREP) {  // one tile set, refilled for the chunk walked next
        auto fill = [&](int64_t c1) {
            if (c1 >= 0) chunk_tiles4<St::RB, St::FB>(tiles, ad, tok(c1), wave, lane);
        };
        rope_load<CK>(R, rad, tok(nch - 1), a.use_rope != 0);
        fill(nch - 1);
        for (int64_t c = nch - 1; c >= 0; --c)
            St::run(a, wk, tok(c), chunk_nv(c), A, ad, rad, R, tok(c - 1), c >= 1, Lst, Gseg, smem, tiles, po, [] {},
                    [&] { fill(c - 1); });
        prep_out_store<CK>(po, ad);
        return;
    }
    if constexpr (St::DMA && !PREP) {
        // tile set 0 holds even steps of the walk (chunks nch-1, nch-3, ...), set 1 odd steps
        char* t0 = tiles;
        char* t1 = tiles + 3 * St::TB;
        auto fill = [&](char* t, int64_t c1) {
            if (c1 >= 0) chunk_tiles<false, St::RB, St::FB>(t, ad, tok(c1), wave, lane);
        };
        fill(t0, nch - 1);
        for (int64_t c = nch - 1; c >= 1; c -= 2) {
            St::run(a, wk, tok(c), chunk_nv(c), A, ad, rad, R, 0, false, Lst, Gseg, smem, t0, po, [] {},
                    [&] { fill(t1, c - 1); });
            St::run(a, wk, tok(c - 1), chunk_nv(c - 1), A, ad, rad, R, 0, false, Lst, Gseg, smem, t1, po, [] {},
                    [&] { fill(t0, c - 2); });
        }
        if (nch & 1) St::run(a, wk, tok(0), chunk_nv(0), A, ad, rad, R, 0, false, Lst, Gseg, smem, t0, po, [] {}, [] {});
        return;
    }
    if constexpr (PREP) rope_load<CK>(R, rad, tok(nch - 1), a.use_rope != 0);
    chunk_load<PREP, CK>(A, ad, tok(nch - 1), true);
    __builtin_amdgcn_sched_barrier(0);  // issue order A, B on every path (see segment_walk)
    chunk_load<PREP, CK>(B, ad, tok(nch - 2), nch > 1);
    // pairs of chunks from the end, then chunk 0 if nch is odd (single-exit loop, as in segment_walk)
    for (int64_t c = nch - 1; c >= 1; c -= 2) {
        St::run(a, wk, tok(c), chunk_nv(c), A, ad, rad, R, tok(c - 1), true, Lst, Gseg, smem, tiles, po,
                [&] { chunk_load<PREP, CK>(A, ad, tok(c - 2), c >= 2); }, [] {});
        St::run(a, wk, tok(c - 1), chunk_nv(c - 1), B, ad, rad, R, tok(c - 2), c >= 2, Lst, Gseg, smem, tiles, po,
                [&] { chunk_load<PREP, CK>(B, ad, tok(c - 3), c >= 3); }, [] {});
    }
    if (nch & 1)
        St::run(a, wk, tok(0), chunk_nv(0), A, ad, rad, R, tok(0), false, Lst, Gseg, smem, tiles, po, [] {}, [] {});
}


// CK: checked row addressing (some sequence length is not a multiple of 4; see chunk_load).
template <typename TIn, typename TG, int DK, int DV, bool CK, bool PREP = false>
__global__ __launch_bounds__(DV * 4, 2) void gla_seg_state_kernel(PrefillParams a) {
    using L = Lay<TIn, DK, DV, false, PREP>;
    constexpr int DL = L::DPW / 4;
    __shared__ __attribute__((aligned(16))) char smem[L::BYTES];
    using St = StateStep<TIn, TG, DK, DV, CK, PREP>;
    __shared__ __attribute__((aligned(16))) char tiles[St::DMA ? St::NT * St::TB : 16];
    const int64_t w = blockIdx.x, h = blockIdx.y;
    Work wk;
    if (!find_work(a, w, wk)) return;
    const int lane = threadIdx.x & 63, wave = wave_id(), r16 = lane & 15, g4 = lane >> 4;
    f32x4 S[DK / 16];
    float Gseg[DL];
#pragma unroll
    for (int db = 0; db < DK / 16; ++db) S[db] = zero4();
#pragma unroll
    for (int i = 0; i < DL; ++i) Gseg[i] = 0.f;
    segment_state_walk<TIn, TG, DK, DV, CK, PREP>(a, wk, h, S, Gseg, smem, tiles);
    float* st = a.ws_state + (w * a.H + h) * (int64_t)DK * DV;
#pragma unroll
    for (int db = 0; db < DK / 16; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) st[state_off(db, i, g4, r16, wave, DV)] = S[db][i];
    if (lane < 4) {  // tg = 0, row = lane: the lane's stage-1 key dims
        float* gs = a.ws_gamma + (w * a.H + h) * (int64_t)DK + stage1_dim0<DK, L::DPW, PREP>(wave, lane);
#pragma unroll
        for (int i = 0; i < DL; ++i) gs[i] = Gseg[i];
    }
}

template <typename TIn, typename TG, int DK, int DV, bool CK, bool OBF>
__global__ __launch_bounds__(DV * 4, (Prec<TIn>::F32 || DK == 128) ? 1 : 2) void gla_seg_output_kernel(PrefillParams a) {
    using L = Lay<TIn, DK, DV, true>;
    __shared__ __attribute__((aligned(16))) char smem[L::BYTES];
    // input tiles: an array of their own, so the compiler knows that reads of smem never wait for
    // the tile DMAs in flight
    using St = OutStep<TIn, TG, DK, DV, CK, OBF>;
    __shared__ __attribute__((aligned(16))) char tiles[St::DMA ? 3 * St::TB : 16];
    const int64_t w = blockIdx.x, h = blockIdx.y;
    Work wk;
    if (!find_work(a, w, wk)) return;
    const int lane = threadIdx.x & 63, wave = wave_id(), r16 = lane & 15, g4 = lane >> 4;
    f32x4 S[DK / 16];
    const float* st = a.ws_state + (w * a.H + h) * (int64_t)DK * DV;
#pragma unroll
    for (int db = 0; db < DK / 16; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) S[db][i] = st[state_off(db, i, g4, r16, wave, DV)];
    segment_walk<TIn, TG, DK, DV, CK, OBF>(a, wk, h, S, smem, tiles);
}

}  // namespace triune
