// chunk_common.h -- device pieces shared by the chunked prefill kernels (GLA, Gated DeltaNet):
// segment work assignment, the stage-1 lane mapping and its loads, decay scans, bf16-part LDS
// planes and MFMA fragment reads (internal to libtriune_hip).
#pragma once

#include <type_traits>

#include "kernels.h"

namespace triune {

constexpr int CHUNK = 64;
constexpr float SPAN_MAX = 64.f;
constexpr int PAD = 4;  // row padding (elements) of LDS planes: spreads rows over banks

struct Work {
    int64_t seq, b, row0, t_begin, t_end, len;
    int p;
};

// x is the same in every lane; say so to the compiler (scalar registers, scalar branches).
__device__ __forceinline__ int64_t uniform_i64(int64_t x) {
    const uint64_t u = (uint64_t)x;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)u);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(u >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ bool find_work(const PrefillParams& a, int64_t w, Work& wk) {
    if (!a.varlen) {
        const int64_t seq = w / a.nseg_dense;
        if (seq >= a.n_seqs) return false;
        wk.seq = seq;
        wk.b = seq;
        wk.row0 = 0;
        wk.p = (int)(w - seq * a.nseg_dense);
        wk.len = a.T;
    } else {
        const int64_t total = a.seg_off[a.n_seqs];
        if (w >= total) return false;
        int64_t lo = 0, hi = a.n_seqs - 1;  // largest seq with seg_off[seq] <= w
        while (lo < hi) {
            const int64_t mid = (lo + hi + 1) >> 1;
            if (a.seg_off[mid] <= w) lo = mid;
            else hi = mid - 1;
        }
        wk.seq = lo;
        wk.b = 0;
        wk.row0 = a.cu[lo];
        wk.p = (int)(w - a.seg_off[lo]);
        wk.len = (int64_t)a.cu[lo + 1] - (int64_t)a.cu[lo];
    }
    if (!a.varlen) {  // dense: nseg near-equal segments (chunk counts differ by at most one)
        const int64_t nch = (wk.len + CHUNK - 1) / CHUNK;
        wk.t_begin = (int64_t)wk.p * nch / a.nseg_dense * CHUNK;
        wk.t_end = (int64_t)(wk.p + 1) * nch / a.nseg_dense * CHUNK;
    } else {
        wk.t_begin = (int64_t)wk.p * a.P * CHUNK;
        wk.t_end = wk.t_begin + (int64_t)a.P * CHUNK;
    }
    if (wk.t_end > wk.len) wk.t_end = wk.len;
    // the segment is per workgroup: uniform loop bounds keep the chunk loops scalar
    wk.b = uniform_i64(wk.b);
    wk.row0 = uniform_i64(wk.row0);
    wk.len = uniform_i64(wk.len);
    wk.t_begin = uniform_i64(wk.t_begin);
    wk.t_end = uniform_i64(wk.t_end);
    return wk.t_begin < wk.t_end;
}

// ---------------------------------------------------------------------------------------
// Precision and LDS layout
// ---------------------------------------------------------------------------------------
template <typename TIn>
struct Prec {
    static constexpr bool F32 = std::is_same<TIn, float>::value;
    static constexpr int NS = F32 ? 3 : 2;                                             // parts of derived operands
    static constexpr int NX = F32 ? 3 : (std::is_same<TIn, _Float16>::value ? 2 : 1);  // parts of V
};

// Every LDS operand is stored token-major as NP planes of bf16 parts (x ~= p0 + p1 (+ p2)).
// Fragments whose K index is the token come out of the same planes through the transposed
// read (ds_read_b64_tr_b16), so no operand is stored twice.

// Causal tiles of A^T (key block sb <= query block tb); index i = tb*(tb+1)/2 + sb.
__device__ __forceinline__ void tile_sb_tb(int i, int& sb, int& tb) {
    tb = i >= 6 ? 3 : (i >= 3 ? 2 : (i >= 1 ? 1 : 0));
    sb = i - tb * (tb + 1) / 2;
}
__device__ __forceinline__ int tile_index(int sb, int tb) { return tb * (tb + 1) / 2 + sb; }

// ---- LDS plane access ------------------------------------------------------------------
// Fragment whose lane index is a plane row (token-major plane, K index along the row): lane
// (g4, r16) reads row `row`, elements col0 + 4*g4 + [0,4) into K slots 0..3 and
// col0 + 16 + 4*g4 + [0,4) into slots 4..7, one bf16 part per plane.
template <int NP>
__device__ __forceinline__ Split8<NP> lds_frag(const char* base, int plane_bytes, int rs, int row, int col0, int g4) {
    Split8<NP> f;
#pragma unroll
    for (int pl = 0; pl < NP; ++pl) {
        const __bf16* p = reinterpret_cast<const __bf16*>(base + pl * plane_bytes) + row * rs + col0 + 4 * g4;
        const bf16x4 a = *reinterpret_cast<const bf16x4*>(p);
        const bf16x4 b = *reinterpret_cast<const bf16x4*>(p + 16);
        f.p[pl] = bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    }
    return f;
}

// ds_read_b64_tr_b16: within each 16-lane group, lane m supplies the address of four
// consecutive 16-bit elements M[m][0..3]; lane i receives M[4j + (i >> 2)][i & 3], j = 0..3.
__device__ __forceinline__ bf16x4 lds_read_tr(const __bf16* p) {
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
    const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
    return __builtin_bit_cast(bf16x4, r);
}

// Fragment whose lane index is a plane column (K index down the rows): lane (g4, r16) gets
// column col0 + r16 of rows row0 + 4*g4 + [0,4) (K slots 0..3) and row0 + 16 + 4*g4 + [0,4)
// (slots 4..7).  Lane (g4, m) addresses row row0 + 4*g4 + (m >> 2), columns col0 + 4*(m & 3).
template <int NP>
__device__ __forceinline__ Split8<NP> lds_frag_tr(const char* base, int plane_bytes, int rs, int row0, int col0,
                                                  int g4, int r16) {
    Split8<NP> f;
    const int off = (row0 + 4 * g4 + (r16 >> 2)) * rs + col0 + 4 * (r16 & 3);
#pragma unroll
    for (int pl = 0; pl < NP; ++pl) {
        const __bf16* p = reinterpret_cast<const __bf16*>(base + pl * plane_bytes) + off;
        const bf16x4 a = lds_read_tr(p);
        const bf16x4 b = lds_read_tr(p + 16 * rs);
        f.p[pl] = bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    }
    return f;
}

// N (multiple of 4) consecutive values at element index idx (a multiple of 4), split into NP
// bf16 planes.
template <int NP, int N>
__device__ __forceinline__ void lds_put_row(char* base, int plane_bytes, int idx, const float* x) {
#pragma unroll
    for (int c = 0; c < N; c += 4) {
        float r[4] = {x[c], x[c + 1], x[c + 2], x[c + 3]};
        uint32_t w[NP][2];
        split_pairs<NP, 2>(r, w);
#pragma unroll
        for (int pl = 0; pl < NP; ++pl)
            *reinterpret_cast<uint2*>(reinterpret_cast<__bf16*>(base + pl * plane_bytes) + idx + c) =
                uint2{w[pl][0], w[pl][1]};
    }
}

// ---- global inputs -----------------------------------------------------------------------
// N consecutive elements of T as 32-bit words (N * sizeof(T) is 4, 8, 16 or 32 bytes).
template <typename T, int N>
struct Vec {
    static constexpr int BYTES = N * (int)sizeof(T);
    static constexpr int W = BYTES / 4;
    uint32_t w[W];
};

// Raw buffer load of one Vec at byte offset voff + soff of the resource; bytes at or past the
// resource's num_records read as zero without touching memory.
template <typename T, int N>
__device__ __forceinline__ void vec_load(Vec<T, N>& v, __amdgpu_buffer_rsrc_t r, int voff, int soff) {
    if constexpr (Vec<T, N>::BYTES % 16 == 0) {
#pragma unroll
        for (int i = 0; i < Vec<T, N>::BYTES / 16; ++i) {
            const auto u = __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16 * i, soff, 0);
            v.w[4 * i] = u[0]; v.w[4 * i + 1] = u[1]; v.w[4 * i + 2] = u[2]; v.w[4 * i + 3] = u[3];
        }
    } else if constexpr (Vec<T, N>::BYTES == 8) {
        const auto u = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
        v.w[0] = u[0]; v.w[1] = u[1];
    } else {
        v.w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
    }
}

template <typename T, int N>
__device__ __forceinline__ void vec_float(const Vec<T, N>& v, float* x) {
    if constexpr (std::is_same<T, float>::value) {
#pragma unroll
        for (int i = 0; i < N; ++i) x[i] = __uint_as_float(v.w[i]);
    } else if constexpr (std::is_same<T, __bf16>::value) {
#pragma unroll
        for (int i = 0; i < N / 2; ++i) {
            x[2 * i] = __uint_as_float(v.w[i] << 16);
            x[2 * i + 1] = __uint_as_float(v.w[i] & 0xffff0000u);
        }
    } else {
#pragma unroll
        for (int i = 0; i < N / 2; ++i) {
            const uint32_t u = v.w[i];
            x[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u & 0xffffu));
            x[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u >> 16));
        }
    }
}

template <typename T>
__device__ __forceinline__ const T* tok_row(const TokTensor& x, const Work& wk, int64_t t, int64_t h, int d) {
    return reinterpret_cast<const T*>(x.p) + wk.b * x.sb + (wk.row0 + t) * x.st + h * x.sh + d;
}

__device__ __forceinline__ float lane_value(float x, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

// Addressing of one token-major input under the stage-1 lane mapping.  Each chunk gets a buffer
// resource based at its first row (wave-uniform) whose num_records ends at the tensor's extent,
// so rows past the end read as zero; lanes add a 32-bit offset (token 4*tg, their first column)
// and the scalar offset selects token j of the four.  A resource with num_records 0 turns a
// load into a no-op, which keeps the number of loads per chunk fixed.  The host guarantees
// 64 * token stride + row bytes < 2^31.
struct TokAddr {
    const char* p0;  // token 0 of the sequence, head h (uniform)
    int64_t rem;     // bytes readable from p0 (uniform)
    int32_t st;      // token stride, bytes (uniform)
    int32_t lane;    // 4*tg*st + col*sizeof(T)
};

template <typename T>
__device__ __forceinline__ TokAddr tok_addr(const TokTensor& x, const Work& wk, int64_t h, int tg, int col) {
    TokAddr r;
    const int64_t es = (int64_t)sizeof(T);
    const int64_t base = uniform_i64((wk.b * x.sb + wk.row0 * x.st + h * x.sh) * es);
    r.p0 = reinterpret_cast<const char*>(x.p) + base;
    // readable bytes: to the tensor's extent and at most to the segment's last token
    const int64_t seg = wk.t_end * x.st * es;
    r.rem = x.extent - base < seg ? x.extent - base : seg;
    r.st = (int32_t)(x.st * es);
    r.lane = 4 * tg * r.st + col * (int32_t)es;
    return r;
}

// Token j of a lane's four rows is addressed through the scalar offset (j * st), but the buffer
// range check covers only the vector and instruction offsets: a chunk whose 64 rows reach past
// the tensor's extent (at most the last chunk of a tensor) must take them through the vector
// offset, where the check zeroes every row past the end.
__device__ __forceinline__ bool chunk_edge(const TokAddr& a, int64_t tc) { return (tc + CHUNK) * a.st > a.rem; }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t chunk_rsrc(const TokAddr& a, int64_t tc, bool valid) {
    const int64_t off = tc * a.st;
    int64_t n = a.rem - off;
    n = n < 0 ? 0 : (n > 0x7fffffff ? 0x7fffffff : n);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(a.p0) + off, (short)0, valid ? (int)n : 0,
                                             0x00020000);
}

struct ChunkAddr {
    TokAddr q, k, g, v;
};

template <bool OUT, typename TIn, typename TG>
__device__ __forceinline__ ChunkAddr chunk_addr(const PrefillParams& a, const Work& wk, int64_t h, int tg, int dcol,
                                                int vcol) {
    ChunkAddr c;
    if (OUT) c.q = tok_addr<TIn>(a.q, wk, h, tg, dcol);
    c.k = tok_addr<TIn>(a.k, wk, h, tg, dcol);
    c.g = tok_addr<TG>(a.g, wk, h, tg, dcol);
    c.v = tok_addr<TIn>(a.v, wk, h, tg, vcol);
    return c;
}

// Stage-1 lane mapping: lane = 4*tg + row (tg = lane >> 2, row = lane & 3) holds tokens 4*tg + j
// (j < 4) of key dims d0 + DL*row + i (i < DL, DL = DPW/4) and value columns c0 + 4*row + c
// (c < 4).  The four lanes of a quad read one contiguous 4*DL-element piece of a token row, so
// each quad costs the L1 a single access; a scan over tokens is a serial sum over j, a DPP scan
// over the four tg of each 16-lane row, and a scan over the four rows' totals.
template <typename TIn, typename TG, int DL>
struct ChunkIn {
    Vec<TIn, DL> q[4], k[4];
    Vec<TG, DL> g[4];
    Vec<TIn, 4> v[4];
};

// Inputs of the chunk starting at token tc (valid: false issues the same loads as no-ops).
// In a partial chunk the rows past its end are other tokens of the tensor or zeros; stage 1
// zeroes them.  CK: a chunk may reach past a tensor's extent with rows of a lane's four (some
// sequence length is not a multiple of 4), so such chunks address their rows through the
// checked vector offset (see chunk_edge); without CK every load uses the scalar offset.
// Records end at the segment's last token (tok_addr), so without CK, where every sequence length
// and hence every chunk's row count is a multiple of 4, whole four-row groups past a chunk read as
// zero and stage 1 need not zero them.
template <bool OUT, bool CK = true, typename TIn, typename TG, int DL>
__device__ __forceinline__ void chunk_load(ChunkIn<TIn, TG, DL>& c, const ChunkAddr& ad, int64_t tc, bool valid) {
    __amdgpu_buffer_rsrc_t rq;
    if (OUT) rq = chunk_rsrc(ad.q, tc, valid);
    const __amdgpu_buffer_rsrc_t rk = chunk_rsrc(ad.k, tc, valid), rg = chunk_rsrc(ad.g, tc, valid),
                                 rv = chunk_rsrc(ad.v, tc, valid);
    const bool edge = CK && ((OUT && chunk_edge(ad.q, tc)) || chunk_edge(ad.k, tc) || chunk_edge(ad.g, tc) ||
                             chunk_edge(ad.v, tc));
    if (edge) {  // rows through the checked vector offset (see chunk_edge)
        int lq = ad.q.lane, lk = ad.k.lane, lg = ad.g.lane, lv = ad.v.lane;
        asm volatile("" : "+v"(lq), "+v"(lk), "+v"(lg), "+v"(lv));  // offsets made here, not kept live
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (OUT) vec_load(c.q[j], rq, lq + j * ad.q.st, 0);
            vec_load(c.k[j], rk, lk + j * ad.k.st, 0);
            vec_load(c.g[j], rg, lg + j * ad.g.st, 0);
            vec_load(c.v[j], rv, lv + j * ad.v.st, 0);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (OUT) vec_load(c.q[j], rq, ad.q.lane, j * ad.q.st);
            vec_load(c.k[j], rk, ad.k.lane, j * ad.k.st);
            vec_load(c.g[j], rg, ad.g.lane, j * ad.g.st);
            vec_load(c.v[j], rv, ad.v.lane, j * ad.v.st);
        }
    }
}

// Rows 4*tg + j (j < 4) of one input, as chunk_load takes them.
template <bool CK = true, typename T, int N>
__device__ __forceinline__ void rows_load(Vec<T, N> (&v)[4], __amdgpu_buffer_rsrc_t r, const TokAddr& a, int64_t tc) {
    if (CK && chunk_edge(a, tc)) {
        int l = a.lane;
        asm volatile("" : "+v"(l));
#pragma unroll
        for (int j = 0; j < 4; ++j) vec_load(v[j], r, l + j * a.st, 0);
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) vec_load(v[j], r, a.lane, j * a.st);
    }
}

// N floats into a Vec of T (round to nearest even for 16-bit types).
template <typename T, int N>
__device__ __forceinline__ void vec_pack(const float* x, Vec<T, N>& v) {
    if constexpr (std::is_same<T, float>::value) {
#pragma unroll
        for (int i = 0; i < N; ++i) v.w[i] = __float_as_uint(x[i]);
    } else if constexpr (std::is_same<T, __bf16>::value) {
#pragma unroll
        for (int i = 0; i < N / 2; ++i) v.w[i] = pk_bf16(x[2 * i], x[2 * i + 1]);
    } else {
#pragma unroll
        for (int i = 0; i < N / 2; ++i)
            v.w[i] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x[2 * i]) |
                     ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x[2 * i + 1]) << 16);
    }
}

// Raw buffer store of one Vec (the counterpart of vec_load): bytes at or past the resource's
// num_records (in the vector offset) are dropped.
template <typename T, int N>
__device__ __forceinline__ void vec_store(const Vec<T, N>& v, __amdgpu_buffer_rsrc_t r, int voff, int soff) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    if constexpr (Vec<T, N>::BYTES % 16 == 0) {
#pragma unroll
        for (int i = 0; i < Vec<T, N>::BYTES / 16; ++i)
            __builtin_amdgcn_raw_buffer_store_b128(u32x4{v.w[4 * i], v.w[4 * i + 1], v.w[4 * i + 2], v.w[4 * i + 3]}, r,
                                                   voff + 16 * i, soff, 0);
    } else if constexpr (Vec<T, N>::BYTES == 8) {
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{v.w[0], v.w[1]}, r, voff, soff, 0);
    } else {
        __builtin_amdgcn_raw_buffer_store_b32(v.w[0], r, voff, soff, 0);
    }
}

// Rows 4*tg + j (j < 4) of one tensor written back with rows_load's addressing (edge chunks through
// the checked vector offset), so rows past the resource's records are not written.
template <bool CK = true, typename T, int N>
__device__ __forceinline__ void rows_store(const Vec<T, N> (&v)[4], __amdgpu_buffer_rsrc_t r, const TokAddr& a,
                                           int64_t tc) {
    if (CK && chunk_edge(a, tc)) {
        int l = a.lane;
        asm volatile("" : "+v"(l));
#pragma unroll
        for (int j = 0; j < 4; ++j) vec_store(v[j], r, l + j * a.st, 0);
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) vec_store(v[j], r, a.lane, j * a.st);
    }
}

// x[j][i] = element i of token j, zeroed for tokens at or past nv (partial chunks only).
// ZERO = false: the loads already returned zero past the chunk (chunk_load without CK).
template <bool ZERO = true, typename T, int N>
__device__ __forceinline__ void chunk_float(const Vec<T, N> (&v)[4], float (&x)[4][N], int tg, int nv) {
#pragma unroll
    for (int j = 0; j < 4; ++j) vec_float(v[j], x[j]);
    if (ZERO && nv < CHUNK) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const bool ok = 4 * tg + j < nv;
#pragma unroll
            for (int i = 0; i < N; ++i) x[j][i] = ok ? x[j][i] : 0.f;
        }
    }
}

// ---- chunk tiles loaded straight into LDS (2-byte inputs, rows of RB = 128 or 256 bytes) -----
// A tile holds the 64 rows of one input's chunk with the 16-byte units of each row permuted by
// s = the token group g = (t >> 2) & 7 spread over the unit-index bits other than FB:
//   RB = 128 (D = 64): 32 pair-rows of 256 B; unit u of token t sits at position
//            ((t & 1) * 8 + u) ^ s of pair-row t >> 1;
//   RB = 256 (D = 128): unit u of token t sits at position u ^ s of row t.
// A DMA instruction writes 1 KB in lane order (lane L at +16 L), i.e. whole rows, so every
// instruction fetches whole 128/256-byte rows (the stage-1 register loads fetch 32 bytes of
// sixteen rows each, which keeps the L1's miss tracking full with partial lines).  In a stage-1
// read the 32 lanes of an LDS cycle cover token groups 0..7 (tokens 4*tg + j) and two units of
// each row that differ in bit FB of the unit index (FB = 0 for the plain dim mapping; 2 or 3 for
// the pre-processing one at 64 or 128 dims); s varies the other three bits, so those lanes land on
// 32 distinct 8-byte bank pairs: no bank conflict.
template <int RB>
constexpr int tile_bytes() {
    static_assert(RB == 128 || RB == 256, "tile rows of 128 or 256 bytes");
    return CHUNK * RB;
}

template <int FB>
__device__ __forceinline__ int tile_swz(int g) {
    return (g & ((1 << FB) - 1)) | ((g >> FB) << (FB + 1));
}

template <int RB, int FB>
__device__ __forceinline__ int tile_off(int t, int byte) {
    const int s = tile_swz<FB>((t >> 2) & 7);
    if constexpr (RB == 128)
        return (t >> 1) * 256 + (((((t & 1) << 3) | (byte >> 4)) ^ s) << 4) + (byte & 15);
    else
        return t * 256 + (((byte >> 4) ^ s) << 4) + (byte & 15);
}

// Buffer resource words (raw buffer, stride 0) of `records` bytes from `base`.
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4 raw_rsrc4(const void* base, int records) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    return i32x4{(int)(uint32_t)a, (int)((uint32_t)(a >> 32) & 0xffffu), records, 0x00020000};
}

// 16 bytes at byte offset voff of resource r into LDS at lds + 16 * lane (lds wave-uniform).
// Issued through asm so that the compiler does not track it: it would otherwise wait for every
// tile DMA in flight before transposed LDS reads (ds_read_b64_tr_b16), whose addresses it cannot
// tell apart from the tiles.  Nothing reads a tile before vm_drain and a barrier.  M0 carries
// the LDS address and is restored afterwards; one wait state separates its write from the load.
__device__ __forceinline__ void dma16(const char* lds, int voff, i32x4 r) {
    const uint32_t l = (uint32_t)reinterpret_cast<uintptr_t>(lds);
    uint32_t save;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(save)
        : "s"(l), "v"(voff), "s"(r)
        : "memory");
}

// This wave's two 1 KB pieces of one input's tile (a tile is 8 (RB = 128) or 16 (RB = 256) pieces,
// two per wave of the workgroup): the rows of the resource `r` (based at the chunk's first row,
// token stride st bytes; records end at the segment's last row, so rows past it land as zeros).
// Lane L of a piece fetches the 16 bytes that belong at +16 L.
template <int RB, int FB>
__device__ __forceinline__ void tile_dma(char* tile, i32x4 r, int st, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int m = 2 * wave + i;
        int t, u;
        if constexpr (RB == 128) {             // piece m: pair-rows 4m .. 4m+3
            const int p = 4 * m + (lane >> 4);
            const int val = (lane & 15) ^ tile_swz<FB>((p >> 1) & 7);
            t = 2 * p + (val >> 3);
            u = val & 7;
        } else {                               // piece m: rows 4m .. 4m+3
            t = 4 * m + (lane >> 4);
            u = (lane & 15) ^ tile_swz<FB>(m & 7);
        }
        dma16(tile + m * 1024, t * st + u * 16, r);
    }
}

// Elements [col, col + N) (2-byte T, N * 2 of 4 or 8 bytes, not crossing a 16-byte unit) of
// token t of a tile.
template <int RB, int FB, typename T, int N>
__device__ __forceinline__ void tile_read(Vec<T, N>& v, const char* tile, int t, int col) {
    static_assert(sizeof(T) == 2 && (N == 2 || N == 4), "tile reads of 4 or 8 bytes");
    const char* p = tile + tile_off<RB, FB>(t, col * 2);
    if constexpr (N == 4) {
        const uint2 u = *reinterpret_cast<const uint2*>(p);
        v.w[0] = u.x; v.w[1] = u.y;
    } else {
        v.w[0] = *reinterpret_cast<const uint32_t*>(p);
    }
}

// Rows 4*tg + j (j < 4) of a tile, as rows_load takes them from memory.
template <int RB, int FB, typename T, int N>
__device__ __forceinline__ void tile_rows(Vec<T, N> (&v)[4], const char* tile, int tg, int col) {
#pragma unroll
    for (int j = 0; j < 4; ++j) tile_read<RB, FB>(v[j], tile, 4 * tg + j, col);
}

// Instances whose inputs can arrive as tiles: 2-byte inputs, the gate in the same type, square
// 64 or 128 heads (a tile row per token of each input; two 1 KB pieces per wave).
template <typename TIn, typename TG, int DK, int DV>
constexpr bool tile_dma_inputs() {
    return sizeof(TIn) == 2 && std::is_same<TIn, TG>::value && DK == DV && (DK == 64 || DK == 128);
}

// Workgroup barrier for LDS traffic only: this wave's LDS operations complete, then s_barrier.
// Unlike __syncthreads it has no release fence, which would also wait for every tile DMA in
// flight (they count as LDS stores); the empty asm statements keep the compiler from moving memory
// operations across it.
__device__ __forceinline__ void lds_sync() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt, expcnt unconstrained
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Barrier of a kernel instance: the LDS-only one where tile DMAs may be in flight.
template <bool DMA>
__device__ __forceinline__ void block_sync() {
    if constexpr (DMA) lds_sync();
    else __syncthreads();
}

// This wave's share of the tiles of the chunk at token tc of the N inputs `src` (tile i at
// tiles + i * tile_bytes<RB>()).
template <int RB, int FB, int N>
__device__ __forceinline__ void tiles_from(char* tiles, const TokAddr* const (&src)[N], int64_t tc, int wave,
                                           int lane) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const TokAddr& x = *src[i];
        const int64_t off = tc * x.st;
        int64_t n = x.rem - off;
        n = n < 0 ? 0 : (n > 0x7fffffff ? 0x7fffffff : n);
        tile_dma<RB, FB>(tiles + i * tile_bytes<RB>(), raw_rsrc4(x.p0 + off, (int)n), x.st, wave, lane);
    }
}

// q, k, g (OUT, the output kernel) or k, g, v (the segment-state kernel).
template <bool OUT, int RB, int FB>
__device__ __forceinline__ void chunk_tiles(char* tiles, const ChunkAddr& ad, int64_t tc, int wave, int lane) {
    const TokAddr* const src[3] = {OUT ? &ad.q : &ad.k, OUT ? &ad.k : &ad.g, OUT ? &ad.g : &ad.v};
    tiles_from<RB, FB>(tiles, src, tc, wave, lane);
}

// q, k, g, v (the pre-processing segment-state kernel).
template <int RB, int FB>
__device__ __forceinline__ void chunk_tiles4(char* tiles, const ChunkAddr& ad, int64_t tc, int wave, int lane) {
    const TokAddr* const src[4] = {&ad.q, &ad.k, &ad.g, &ad.v};
    tiles_from<RB, FB>(tiles, src, tc, wave, lane);
}

// min(x, 0) in one instruction (fminf first quiets NaNs with an extra max in IEEE mode).
__device__ __forceinline__ float min0(float x) {
    // min(x, 0) as one integer min: a float with the sign bit set is a negative int32 and keeps
    // its bits; every other float (positive, +0, positive NaN) maps to the bits of +0.0f.
    return __int_as_float(min(__float_as_int(x), 0));
}

// V rows of tokens 4*tg + j (this lane's four columns) into one bf16 plane.  bf16 V is copied
// as loaded (no conversion round trip); rows at or past nv are zeroed.  Other types go through
// the split.
template <typename T, int NX, bool ZERO = true>
__device__ __forceinline__ void lds_put_v_rows(char* base, int plane_bytes, int rs, int col, const Vec<T, 4> (&v)[4],
                                               int tg, int nv) {
    if constexpr (std::is_same<T, __bf16>::value) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const bool ok = !ZERO || nv >= CHUNK || 4 * tg + j < nv;
            *reinterpret_cast<uint2*>(reinterpret_cast<__bf16*>(base) + (4 * tg + j) * rs + col) =
                uint2{ok ? v[j].w[0] : 0u, ok ? v[j].w[1] : 0u};
        }
    } else {
        float vx[4][4];
        chunk_float<ZERO>(v, vx, tg, nv);
#pragma unroll
        for (int j = 0; j < 4; ++j) lds_put_row<NX, 4>(base, plane_bytes, (4 * tg + j) * rs + col, vx[j]);
    }
}

// In place: G[j][i] <- inclusive sum over tokens 0..4*tg+j of the chunk (per key dim i);
// returns the chunk totals in GC[i] (identical across the lanes sharing `row`).
template <int DL>
__device__ __forceinline__ void chunk_cumsum(float (&G)[4][DL], float (&GC)[DL], int lane) {
    float T[DL], I[DL];
#pragma unroll
    for (int i = 0; i < DL; ++i) {
        G[1][i] += G[0][i];
        G[2][i] += G[1][i];
        G[3][i] += G[2][i];
        T[i] = G[3][i];
        I[i] = T[i];
    }
    // the four tg of a 16-lane DPP row sit 4 lanes apart
#pragma unroll
    for (int i = 0; i < DL; ++i) I[i] += row_shr<4>(I[i]);
#pragma unroll
    for (int i = 0; i < DL; ++i) I[i] += row_shr<8>(I[i]);
    // R = this DPP row's total for the lane's `row` (rotations by 4 and 8 sum its four tg); then
    // an inclusive scan of R over the four DPP rows through whole-row swaps: the 16-lane swap
    // gives odd rows their even neighbour and every row its pair's total, the 32-lane swap
    // gives rows 2-3 the total of rows 0-1 and every lane the chunk total.
    const int rr = lane >> 4;
#pragma unroll
    for (int i = 0; i < DL; ++i) {
        float R = T[i] + row_ror<4>(T[i]);
        R += row_ror<8>(R);
        const RowPair p16 = swap16(R);
        const float Q = p16.lo + p16.hi;  // the pair's total (rows 0+1 or 2+3)
        const RowPair p32 = swap32(Q);
        const float P = R + ((rr & 1) ? p16.lo : 0.f) + (rr >= 2 ? p32.lo : 0.f);
        const float E = I[i] - T[i] + (P - R);
#pragma unroll
        for (int j = 0; j < 4; ++j) G[j][i] += E;
        GC[i] = p32.lo + p32.hi;
    }
}

// X[j][i] <- sum of g over the tokens after 4*tg + j in the chunk (exclusive suffix, per key dim
// i), GC[i] <- the chunk total.  Every suffix is summed from the later tokens only, so its
// rounding error scales with the suffix itself, not with the chunk total (a difference of two
// prefix sums loses that accuracy when the total is large).
template <int DL>
__device__ __forceinline__ void chunk_suffix(const float (&g)[4][DL], float (&X)[4][DL], float (&GC)[DL], int lane) {
    float T[DL], Y[DL];
#pragma unroll
    for (int i = 0; i < DL; ++i) {
        X[3][i] = 0.f;
        X[2][i] = g[3][i];
        X[1][i] = X[2][i] + g[2][i];
        X[0][i] = X[1][i] + g[1][i];
        T[i] = X[0][i] + g[0][i];
    }
    // Y = sum of T over the later tg of the same 16-lane DPP row (4 lanes apart)
#pragma unroll
    for (int i = 0; i < DL; ++i) Y[i] = row_shl<4>(T[i]);
#pragma unroll
    for (int i = 0; i < DL; ++i) Y[i] += row_shl<4>(Y[i]);
#pragma unroll
    for (int i = 0; i < DL; ++i) Y[i] += row_shl<8>(Y[i]);
    // Z = this DPP row's total for the lane's `row`; the rows after the lane's own add up through
    // whole-row swaps (even rows take their odd neighbour; rows 0-1 take the total of rows 2-3).
    const int rr = lane >> 4;
#pragma unroll
    for (int i = 0; i < DL; ++i) {
        float Z = T[i] + row_ror<4>(T[i]);
        Z += row_ror<8>(Z);
        const RowPair p16 = swap16(Z);
        const RowPair p32 = swap32(p16.lo + p16.hi);
        const float later_rows = ((rr & 1) ? 0.f : p16.hi) + (rr < 2 ? p32.hi : 0.f);
        const float E = Y[i] + later_rows;
#pragma unroll
        for (int j = 0; j < 4; ++j) X[j][i] += E;
        GC[i] = p32.lo + p32.hi;
    }
}


// S tile db of wave w: element i is S[16*db + 4*g4 + i][16*w + r16].
// Four fp32 values (one D-layout column piece) as a K=16 operand: K slots 0..3, zeros above.
template <int NP>
__device__ __forceinline__ Split8<NP> split_k16(const f32x4& v) {
    const float x[8] = {v[0], v[1], v[2], v[3], 0.f, 0.f, 0.f, 0.f};
    return split8<NP>(x);
}

// Two D-layout tiles stacked along K (rows of tile lo in slots 0..3, of tile hi in 4..7): the
// B operand (or the A operand of the transpose) of a K=32 product.
template <int NP>
__device__ __forceinline__ Split8<NP> split_k32(const f32x4& lo, const f32x4& hi) {
    const float x[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return split8<NP>(x);
}

// ---- chunk outputs ------------------------------------------------------------------------
// Output rows of one chunk for a wave's 16 columns: a buffer resource over rows [0, nv) from
// `base` (row stride ost bytes, 16 columns of es bytes each), so rows past the chunk's end are
// dropped by the hardware, and a second resource that is the same for fp32 and empty otherwise.
struct OutRsrc {
    __amdgpu_buffer_rsrc_t lo, hi;
};

__device__ __forceinline__ OutRsrc out_rsrc(char* base, int64_t ost, int es, int nv, bool f32) {
    const int n = nv > 0 ? (int)((nv - 1) * ost + 16 * es) : 0;
    OutRsrc r;
    r.lo = __builtin_amdgcn_make_buffer_rsrc(base, (short)0, n, 0x00020000);
    r.hi = __builtin_amdgcn_make_buffer_rsrc(base, (short)0, f32 ? n : 0, 0x00020000);
    return r;
}

// Four values of one output row as dtype dt at byte offset voff: always two 8-byte buffer
// stores (the second one lands in the empty resource for 16-bit types), so the number of
// outstanding memory operations never depends on dt or on the chunk length and the wait for the
// next chunk's loads can leave the stores in flight.
__device__ __forceinline__ void out_store4(const OutRsrc& r, int voff, int dt, const f32x4& x) {
    // all three encodings, chosen by selects: no branch between the loads and the stores
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
    const u32x2 b = __builtin_bit_cast(u32x2, bf16x4{(__bf16)x[0], (__bf16)x[1], (__bf16)x[2], (__bf16)x[3]});
    const u32x2 f = __builtin_bit_cast(u32x2, f16x4{(_Float16)x[0], (_Float16)x[1], (_Float16)x[2], (_Float16)x[3]});
    const bool f32 = dt == DT_F32, bf = dt == DT_BF16;
    u32x2 w0, w1;
    w0[0] = f32 ? __float_as_uint(x[0]) : (bf ? b[0] : f[0]);
    w0[1] = f32 ? __float_as_uint(x[1]) : (bf ? b[1] : f[1]);
    w1[0] = __float_as_uint(x[2]);
    w1[1] = __float_as_uint(x[3]);
    __builtin_amdgcn_raw_buffer_store_b64(w0, r.lo, voff, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b64(w1, r.hi, voff + 8, 0, 0);
}

// One output of a (sequence, head) of a [B, T, H, D] tensor: token 0's address and the token
// stride in bytes, made once per workgroup so a chunk loop carries three scalars per output
// instead of its strides.
struct RowsOut {
    char* base;
    int64_t ost;
    int es, dt;
};

__device__ __forceinline__ RowsOut rows_out(void* p, int64_t sb, int64_t st, int64_t sh, int dt, const Work& wk,
                                            int64_t h) {
    RowsOut r;
    r.dt = dt;
    r.es = dt_size(dt);
    r.ost = st * r.es;
    r.base = reinterpret_cast<char*>(p) + uniform_i64((wk.b * sb + wk.row0 * st + h * sh) * r.es);
    return r;
}

// s_waitcnt vmcnt(0) (the LDS and export counters are left free): every vector memory access of
// this wave has completed.  On gfx9 one counter tracks loads and stores, so a later wait for a
// load issued before a burst of stores also waits for those stores; draining the (long since
// returned) prefetch loads right before the burst lets that later wait be skipped.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Wave index within the workgroup as a wave-uniform (scalar) value.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

__device__ __forceinline__ int64_t state_off(int db, int i, int g4, int r16, int wave, int Dv) {
    return (int64_t)(16 * db + 4 * g4 + i) * Dv + 16 * wave + r16;
}

}  // namespace triune
