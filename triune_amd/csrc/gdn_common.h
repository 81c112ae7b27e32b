// gdn_common.h -- device pieces shared by the chunked Gated DeltaNet kernels (per-key-dim gates
// in gdn_chunk.hip, one gate per token and head in gdn_scalar.hip): the segment-map workspace
// layout read by the segment scan and its stores and loads, tile fragments, beta reads and the
// token-by-token update of the per-key-dim kernels (internal to libtriune_hip).
#pragma once

#include "chunk_common.h"

namespace triune {

// Workspace layouts shared by the three segment kernels (head dim D = 16 * NDB, NDB row tiles of
// 16 and NDB / 2 K steps of 32), both chosen so that every lane moves whole 16-byte vectors:
//  - M_p: up to 3 bf16 parts, each stored as the scan's A-operand fragments: element j of lane L
//    for row tile t and K step kk at ((part*NDB + t)*(NDB/2) + kk)*512 + 8L + j;
//  - N_p / S_in[p]: fp32 in MFMA D layout, element i of lane L for column strip c (16 columns)
//    and row tile t at ((c*NDB + t)*64 + L)*4 + i.
template <int D>
constexpr int64_t mslot() { return 3 * D * D; }
constexpr int64_t MSLOT = mslot<64>();

template <int NDB = 4>
__device__ __forceinline__ int64_t dstate_off(int strip, int t, int lane) { return ((strip * NDB + t) * 64 + lane) * 4; }

// Tile fragment from a tile plane set: lane values at (tile, lane) in K slots 0..3 (K=16), or two
// tiles in slots 0..3 / 4..7 (K=32).
template <int NP>
__device__ __forceinline__ Split8<NP> tile_frag(const char* base, int plane_bytes, int i0, int i1, bool has_hi,
                                                int lane) {
    Split8<NP> f;
#pragma unroll
    for (int pl = 0; pl < NP; ++pl) {
        const __bf16* p = reinterpret_cast<const __bf16*>(base + pl * plane_bytes);
        const bf16x4 lo = *reinterpret_cast<const bf16x4*>(p + (i0 * 64 + lane) * 4);
        const __bf16 z = (__bf16)0.f;
        if (has_hi) {
            const bf16x4 hi = *reinterpret_cast<const bf16x4*>(p + (i1 * 64 + lane) * 4);
            f.p[pl] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        } else {
            f.p[pl] = bf16x8{lo[0], lo[1], lo[2], lo[3], z, z, z, z};
        }
    }
    return f;
}

// Slot of the off-diagonal L^T block (sb < tb) in the compact six-tile plane.
__device__ __forceinline__ int lt_index(int sb, int tb) { return (tb - 1) * tb / 2 + sb; }

__device__ __forceinline__ float beta_value(const PrefillParams& a, const Work& wk, int64_t h, int64_t t) {
    const int64_t i = wk.b * a.b_sb + (wk.row0 + t) * a.b_st + h * a.b_sh;
    if (a.beta_dt == DT_F32) return reinterpret_cast<const float*>(a.beta)[i];
    if (a.beta_dt == DT_BF16) return (float)reinterpret_cast<const __bf16*>(a.beta)[i];
    return (float)reinterpret_cast<const _Float16*>(a.beta)[i];
}

// Token-by-token GDN update of one wave's 16 state columns (decay spans beyond the factored form's
// limit).  S tile db holds S[16*db + 4*g4 + i][c0 + r16] (NDB tiles: key dim 16 * NDB); with_v
// false reads V as zero.  BV: beta per value column (BETA_VALUE, fp32 in `kb`) scales u.
template <typename TIn, typename TG, bool OUT, bool BV = false, int NDB>
__device__ void gdn_tokenwise(const PrefillParams& a, const Work& wk, int64_t h, int c0, int64_t tc, int nv, int g4,
                              int r16, bool with_v, f32x4 (&S)[NDB]) {
    for (int t = 0; t < nv; ++t) {
        const int64_t tt = tc + t;
        const float bh = a.beta_kind == BETA_HEAD ? beta_value(a, wk, h, tt) : 1.f;
        // k . S first, then the update one 16-row tile at a time (k read again), so that no
        // per-tile factor array stays live across the whole state (32 rows per lane at D = 128).
        float pred = 0.f;
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            const int d = 16 * db + 4 * g4;
#pragma unroll
            for (int i = 0; i < 4; ++i) pred += (float)tok_row<TIn>(a.k, wk, tt, h, d)[i] * S[db][i];
        }
        pred += __shfl_xor(pred, 16);
        pred += __shfl_xor(pred, 32);
        float u = (with_v ? (float)tok_row<TIn>(a.v, wk, tt, h, c0)[r16] : 0.f) - pred;
        if constexpr (BV) u *= tok_row<float>(a.kb, wk, tt, h, c0)[r16];
        float part = 0.f;
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            const int d = 16 * db + 4 * g4;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float dcy = expf(fminf((float)tok_row<TG>(a.g, wk, tt, h, d)[i], 0.f));
                const float kk = (float)tok_row<TIn>(a.k, wk, tt, h, d)[i];
                const float bk = a.beta_kind == BETA_KEY ? tok_row<float>(a.kb, wk, tt, h, d)[i] : bh;
                const float s = dcy * S[db][i] + bk * kk * u;
                S[db][i] = s;
                if (OUT) part += (float)tok_row<TIn>(a.q, wk, tt, h, d)[i] * s;
            }
        }
        if (OUT) {
            part += __shfl_xor(part, 16);
            part += __shfl_xor(part, 32);
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

// K1 epilogue: the segment map of one (segment w, head h), D = 16 * NDB.  M goes out split into
// NS bf16 parts (the scan's MFMA operands): NS planes of [D][D] per (segment, head), slot stride
// mslot<D>() elements; M[16db + 4g4 + i][16*wave + r16] is element j = 4(wave&1) + (r16&3) of scan
// lane 16(r16>>2) + 4g4 + i for row tile db and K step wave>>1.  N goes out in the D layout of the
// scan.
template <int NS, int NDB>
__device__ __forceinline__ void store_seg_map(const PrefillParams& a, int64_t w, int64_t h, const f32x4 (&M)[NDB],
                                              const f32x4 (&N)[NDB]) {
    constexpr int D = 16 * NDB, NKS = NDB / 2;
    const int lane = threadIdx.x & 63, wave = wave_id(), r16 = lane & 15, g4 = lane >> 4;
    __bf16* dm = reinterpret_cast<__bf16*>(a.ws_m) + (w * a.H + h) * mslot<D>();
    float* dn = a.ws_state + (w * a.H + h) * (int64_t)D * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float m = M[db][i];
            const int sl = 16 * (r16 >> 2) + 4 * g4 + i, j = 4 * (wave & 1) + (r16 & 3);
#pragma unroll
            for (int pl = 0; pl < NS; ++pl) {
                const __bf16 hi = (__bf16)m;
                dm[((pl * NDB + db) * NKS + (wave >> 1)) * 512 + 8 * sl + j] = hi;
                m -= (float)hi;
            }
        }
        *reinterpret_cast<f32x4*>(dn + dstate_off<NDB>(wave, db, lane)) = N[db];
    }
}

// K2 and K3 read the carried-in state S_in[p] of (segment w, head h) from the N slot.
template <int NDB>
__device__ __forceinline__ void load_seg_state(const PrefillParams& a, int64_t w, int64_t h, f32x4 (&S)[NDB]) {
    constexpr int D = 16 * NDB;
    const int lane = threadIdx.x & 63, wave = wave_id();
    const float* st = a.ws_state + (w * a.H + h) * (int64_t)D * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db) S[db] = *reinterpret_cast<const f32x4*>(st + dstate_off<NDB>(wave, db, lane));
}

// The segment map's starting states: M = I restricted to this wave's 16 columns, N = 0.
template <int NDB>
__device__ __forceinline__ void init_seg_map(f32x4 (&M)[NDB], f32x4 (&N)[NDB]) {
    const int lane = threadIdx.x & 63, wave = wave_id(), r16 = lane & 15, g4 = lane >> 4;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            M[db][i] = (16 * db + 4 * g4 + i == 16 * wave + r16) ? 1.f : 0.f;
            N[db][i] = 0.f;
        }
}

}  // namespace triune
