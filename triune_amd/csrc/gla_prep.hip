// gla_prep.hip -- GLA input pre-processing on gfx950, and the decode step fused with it.
//
// Pre-processing of the reference's VectorisedGLA (triune/model/attention.py:14-79, the
// _fused_qkv_g_prep_inplace_kernel Triton kernel; the unfused form is attention.py:509-528):
//   q, k <- RoPE(normalize(elu(x) + 1))   per (token, head) row of HD elements
//   g    <- logsigmoid(g)
// with normalize(a) = a / sqrt(max(sum(a^2), 1e-12)) and RoPE pairing element d with d + HD/2:
//   out[d]        = a[d] cos[t][d]        - a[d + HD/2] sin[t][d]
//   out[d + HD/2] = a[d + HD/2] cos[t][d + HD/2] + a[d] sin[t][d + HD/2]          (d < HD/2)
// The fused decode step (attention.py:81-179, _fused_qkvg_decode_step_kernel) applies the same
// pre-processing to one token per sequence and then the GLA step with decay sigmoid(g)
// (= exp(logsigmoid(g))):  S <- diag(sigmoid(g)) S + k v^T ,  o = S^T q.
//
// gla_prep_kernel: memory-bound, in place.  A row is covered by HD/8 consecutive lanes holding 8
// elements each (16-byte accesses for 16-bit types); the sum of squares is reduced and the RoPE
// partner exchanged with lane shuffles inside the row's lane group.
// gla_fused_decode_kernel: the decode kernel's layout (256-thread blocks walking (b, h) rows, thread
// = RPT key rows x 4 value columns); every wave forms the two norms itself from one element per
// lane, so no barrier separates the pre-processing from the state update.
#include "kernels.h"
#include "common.h"

namespace triune {

template <typename T>
using V4 = T __attribute__((ext_vector_type(4)));

// Eight consecutive elements as floats / back (16-bit: one 16-byte access; fp32: two).
template <typename T>
__device__ __forceinline__ void ld8(const T* p, float (&x)[8]) {
    const V4<T> a = *reinterpret_cast<const V4<T>*>(p);
    const V4<T> b = *reinterpret_cast<const V4<T>*>(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        x[i] = (float)a[i];
        x[4 + i] = (float)b[i];
    }
}

template <typename T>
__device__ __forceinline__ void st8(T* p, const float (&x)[8]) {
    V4<T> a, b;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        a[i] = (T)x[i];
        b[i] = (T)x[4 + i];
    }
    *reinterpret_cast<V4<T>*>(p) = a;
    *reinterpret_cast<V4<T>*>(p + 4) = b;
}


// Sum over the 64 lanes of a wave, in every lane: DPP inclusive scans of the four 16-lane rows,
// then the rows' last lanes read into scalars (no LDS-routed shuffle on the path).
__device__ __forceinline__ float wave_sum(float x) {
    x = row_inclusive_scan(x);
    const int v = __float_as_int(x);
    return (__int_as_float(__builtin_amdgcn_readlane(v, 15)) + __int_as_float(__builtin_amdgcn_readlane(v, 31))) +
           (__int_as_float(__builtin_amdgcn_readlane(v, 47)) + __int_as_float(__builtin_amdgcn_readlane(v, 63)));
}

// ---------------------------------------------------------------------------------------
// In-place pre-processing of qkv [B, T, 3, H, HD] (q, k; v untouched) and g [B, T, H, HD].
// ---------------------------------------------------------------------------------------
template <int HD, typename TIO, typename TCS>
__global__ __launch_bounds__(256) void gla_prep_kernel(PrepParams a) {
    constexpr int LPR = HD / 8;  // lanes per row
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63;
    const int64_t nrows = a.B * a.T * a.H;
    const int64_t row = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW + lane / LPR;
    const bool ok = row < nrows;
    const int64_t r = ok ? row : nrows - 1;  // past the end: a valid row is read, nothing stored
    const int c = lane % LPR;                 // this lane's 8 elements: 8c .. 8c+7
    const int64_t h = r % a.H, bt = r / a.H, t = bt % a.T, b = bt / a.T;
    TIO* qp = reinterpret_cast<TIO*>(a.qkv) + b * a.qkv_sb + t * a.qkv_st + h * a.qkv_sh + 8 * c;
    TIO* kp = qp + a.qkv_sp;
    TIO* gp = reinterpret_cast<TIO*>(a.g) + b * a.g_sb + t * a.g_st + h * a.g_sh + 8 * c;
    float q[8], k[8], g[8];
    ld8(qp, q);
    ld8(kp, k);
    ld8(gp, g);
    float sq = 0.f, sk = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        q[i] = elu1(q[i]);
        k[i] = elu1(k[i]);
        sq += q[i] * q[i];
        sk += k[i] * k[i];
        g[i] = logsigmoid(g[i]);
    }
#pragma unroll
    for (int m = 1; m < LPR; m <<= 1) {
        sq += __shfl_xor(sq, m);
        sk += __shfl_xor(sk, m);
    }
    const float iq = inv_norm(sq), ik = inv_norm(sk);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        q[i] *= iq;
        k[i] *= ik;
    }
    if (a.use_rope) {
        const TCS* cp = reinterpret_cast<const TCS*>(a.cos) + t * a.cs_st + 8 * c;
        const TCS* sp = reinterpret_cast<const TCS*>(a.sin) + t * a.cs_st + 8 * c;
        float cs[8], sn[8];
        ld8(cp, cs);
        ld8(sp, sn);
        const float sgn = c < LPR / 2 ? -1.f : 1.f;  // first half: a cos - a' sin; second: a cos + a' sin
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float qo = __shfl_xor(q[i], LPR / 2), ko = __shfl_xor(k[i], LPR / 2);
            q[i] = q[i] * cs[i] + sgn * qo * sn[i];
            k[i] = k[i] * cs[i] + sgn * ko * sn[i];
        }
    }
    if (ok) {
        st8(qp, q);
        st8(kp, k);
        st8(gp, g);
    }
}

// ---------------------------------------------------------------------------------------
// Fused decode: qkvg [B, 4, H, HD] (q, k, v, g raw), cos/sin [HD] of the step's position,
// state [B, H, HD, HD] in TS (fp32 or the I/O type), o [B, H, HD].  A block walks rows
// blockIdx.x, + gridDim.x, ... and loads the next row's state while it pre-processes the current
// row's inputs; the loads complete before the current row is stored.  State accesses are buffer
// loads/stores over one row whose record count is 0 without an initial state (loads return 0) or
// without a state output (stores are dropped), so every path issues the same memory operations.
// ---------------------------------------------------------------------------------------
template <int HD>
struct FusedDecodeTiling {
    static constexpr int RPT = HD * HD / (4 * 256) > 4 ? HD * HD / (4 * 256) : 4;  // key rows per thread
    static constexpr int CG = HD / 4;                                            // column groups
    static constexpr int TPB = HD * HD / (4 * RPT);
    static constexpr int WAVES = TPB / 64;
    static constexpr int EPL = HD / 64 > 0 ? HD / 64 : 1;  // norm elements per lane
};

template <int HD, typename TIO, typename TCS, typename TS>
__global__ __launch_bounds__(FusedDecodeTiling<HD>::TPB) void gla_fused_decode_kernel(FusedDecodeParams a, uint32_t rows) {
    using Tl = FusedDecodeTiling<HD>;
    constexpr int RPT = Tl::RPT, CG = Tl::CG, WAVES = Tl::WAVES, EPL = Tl::EPL;
    constexpr int SB = (int)sizeof(TS);
    static_assert(Tl::TPB == 256 || Tl::TPB == 64 || Tl::TPB == 128, "fused decode tiling");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int cg = tid % CG, rg = tid / CG, r0 = rg * RPT;
    const uint32_t H32 = (uint32_t)a.H;
    const int32_t voff = (r0 * HD + 4 * cg) * SB;  // this thread's first state element in a row
    auto row_rsrc = [&](const void* p, int64_t srow, bool on) {
        char* base = reinterpret_cast<char*>(const_cast<void*>(p)) + (on ? srow : 0) * HD * HD * SB;
        return __builtin_amdgcn_make_buffer_rsrc(base, (short)0, on ? HD * HD * SB : 0, 0x00020000);
    };
    // State row of (b, h): row itself, or through the pool's slots (-1: b's slot lies outside the
    // pool, a padded batch row; its buffer resources then hold no records).  The slot index is
    // the same for the whole block and read through the scalar cache (a vector load would need a
    // wait on every load outstanding before the state address is known).
    const int32_t nsr = (int32_t)(a.n_state_rows < INT32_MAX ? a.n_state_rows : INT32_MAX);
    auto state_row = [&](uint32_t row) -> int64_t {
        if (!a.slots) return (int64_t)row;
        const auto* sp = (const __attribute__((address_space(4))) int32_t*)a.slots;
        const int32_t sl = sp[row / H32];
        return (sl >= 0 && sl < nsr) ? (int64_t)sl * a.H + row % H32 : -1;
    };
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    struct Raw {
        u32x4 w[RPT];  // 16-bit states use the first two words
        int64_t srow;
    };
    // `live` false: the loads are issued all the same but over a resource of no records (they read
    // zeros and touch no memory), so every path issues the same loads and waits for the same ones.
    auto fetch = [&](Raw& x, uint32_t row, bool live) {
        x.srow = state_row(row);
        const auto r = row_rsrc(a.state_in, x.srow, live && a.has_init != 0 && x.srow >= 0);
#pragma unroll
        for (int m = 0; m < RPT; ++m) {
            if constexpr (SB == 4) {
                x.w[m] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff + m * HD * SB, 0, 2));
            } else {
                const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, voff + m * HD * SB, 0, 2));
                x.w[m] = u32x4{v[0], v[1], 0u, 0u};
            }
        }
    };
    auto unpack = [&](const u32x4& w) -> f32x4 {
        if constexpr (SB == 4) {
            return __builtin_bit_cast(f32x4, w);
        } else {
            const V4<TS> v = __builtin_bit_cast(V4<TS>, u32x2{w[0], w[1]});
            return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
        }
    };
    const int tbytes = a.use_rope ? HD * (int)sizeof(TCS) : 0;
    const auto rcos = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(a.cos), (short)0, tbytes, 0x00020000);
    const auto rsin = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(a.sin), (short)0, tbytes, 0x00020000);
    auto ld_table4 = [](__amdgpu_buffer_rsrc_t r, int off, float* x) {
        if constexpr (sizeof(TCS) == 4) {
            const f32x4 v = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = v[i];
        } else {
            const V4<TCS> v = __builtin_bit_cast(V4<TCS>, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = (float)v[i];
        }
    };
    auto ld4 = [](const auto* p, float* x) {
        using T = std::remove_const_t<std::remove_pointer_t<decltype(p)>>;
        const V4<T> v = *reinterpret_cast<const V4<T>*>(p);
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = (float)v[i];
    };
    constexpr int PH = HD / 2;
    const float rope = a.use_rope ? 1.f : 0.f;
    // HD <= 64: lane d (mod HD) finishes element d of q and k (HD = 32: lanes 32..63 repeat 0..31,
    // counted once in the norms).  The RoPE entries of element d are the same for every row (one
    // position per step) and loaded once; buffer loads over a table of HD entries, or of none when
    // RoPE is off (they then read zeros and never touch memory, as cos and sin may be null).
    const int d = lane % HD;
    float ce = 0.f, se = 0.f;
    if constexpr (EPL == 1) {
        if constexpr (sizeof(TCS) == 4) {
            ce = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(rcos, d * 4, 0, 0));
            se = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsin, d * 4, 0, 0));
        } else {
            ce = (float)__builtin_bit_cast(TCS, (unsigned short)__builtin_amdgcn_raw_buffer_load_b16(rcos, d * 2, 0, 0));
            se = (float)__builtin_bit_cast(TCS, (unsigned short)__builtin_amdgcn_raw_buffer_load_b16(rsin, d * 2, 0, 0));
        }
    }
    // The row's small inputs for HD <= 64, in their storage type until used: element d of q and k,
    // this thread's key rows of g and its 4 value columns.
    struct Small {
        TIO q, k;
        V4<TIO> g[RPT / 4], v;
    };
    auto row_base = [&](uint32_t row) {
        const int64_t b = row / H32, h = row % H32;
        return reinterpret_cast<const TIO*>(a.qkvg) + b * a.x_sb + h * a.x_sh;
    };
    auto fetch_small = [&](Small& x, uint32_t row) {
        if constexpr (EPL == 1) {
            const TIO* base = row_base(row);
            x.q = base[d];
            x.k = base[a.x_sp + d];
#pragma unroll
            for (int m = 0; m < RPT; m += 4) x.g[m / 4] = *reinterpret_cast<const V4<TIO>*>(base + 3 * a.x_sp + r0 + m);
            x.v = *reinterpret_cast<const V4<TIO>*>(base + 2 * a.x_sp + 4 * cg);
        }
    };
    __shared__ f32x4 red[2][WAVES][CG];
    // One row, its state in `cur` (loaded during the previous row): load its small inputs and
    // pre-process them, issue the next row's state loads into `nxt` (past the last row they read
    // nothing), wait for every load and store of the wave, then update, store and reduce.  The
    // wait keeps a wave's state reads and writes from overlapping: at the config-2 shape
    // (B = 256, H = 6, HD = 64) 9.2 us per step, against 10.1-10.4 us with the next row's
    // reads in flight during this row's stores (issued before or after them).
    auto step = [&](const Raw& cur, Raw& nxt, uint32_t row, int buf) {
        const uint32_t nrow = row + gridDim.x;
        const bool more = nrow < rows;
        Small sc;
        fetch_small(sc, row);
        const int64_t b = row / H32, h = row % H32;
        float qv[RPT], kv[RPT], dv[RPT], vv[4];
        if constexpr (EPL == 1) {
            // ELU+1, norm and RoPE (partner element d +- HD/2 from lane d ^ HD/2) once per element;
            // every thread then gathers its key rows from those lanes.
            const float q1 = elu1((float)sc.q), k1 = elu1((float)sc.k);
            const bool first = lane < HD;
            const float sq = wave_sum(first ? q1 * q1 : 0.f), sk = wave_sum(first ? k1 * k1 : 0.f);
            const float qn = q1 * inv_norm(sq), kn = k1 * inv_norm(sk);
            const float qo = __shfl_xor(qn, PH), ko = __shfl_xor(kn, PH);
            const float c = rope * ce + (1.f - rope), sg = rope * (d < PH ? -se : se);
            const float qr_d = qn * c + sg * qo, kr_d = kn * c + sg * ko;
#pragma unroll
            for (int m = 0; m < RPT; ++m) {
                qv[m] = lane_bcast(qr_d, r0 + m);
                kv[m] = lane_bcast(kr_d, r0 + m);
                dv[m] = sigmoid((float)sc.g[m / 4][m % 4]);
            }
#pragma unroll
            for (int c4 = 0; c4 < 4; ++c4) vv[c4] = (float)sc.v[c4];
        } else {
            // HD = 128 (two elements per lane): each thread forms its key rows and their RoPE
            // partner rows itself; the norm elements, rows, partners, cos/sin and value columns are
            // loaded together at the top of the row.
            const TIO* base = row_base(row);
            const TIO* qr = base;
            const TIO* kr = base + a.x_sp;
            const TIO* vr = base + 2 * a.x_sp;
            const TIO* gr = base + 3 * a.x_sp;
            float qa[EPL], ka[EPL], gg[RPT];
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                qa[e] = (float)qr[lane + 64 * e];
                ka[e] = (float)kr[lane + 64 * e];
            }
            const int rp = r0 < PH ? r0 + PH : r0 - PH;  // partner rows rp .. rp+RPT-1
            float qo[RPT], qp[RPT], ko[RPT], kp[RPT], cs[RPT], sn2[RPT];
#pragma unroll
            for (int m = 0; m < RPT; m += 4) {
                ld4(qr + r0 + m, qo + m);
                ld4(qr + rp + m, qp + m);
                ld4(kr + r0 + m, ko + m);
                ld4(kr + rp + m, kp + m);
                ld4(gr + r0 + m, gg + m);
                ld_table4(rcos, (r0 + m) * (int)sizeof(TCS), cs + m);
                ld_table4(rsin, (r0 + m) * (int)sizeof(TCS), sn2 + m);
            }
            ld4(vr + 4 * cg, vv);
            float sq = 0.f, sk = 0.f;
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const float q1 = elu1(qa[e]), k1 = elu1(ka[e]);
                sq += q1 * q1;
                sk += k1 * k1;
            }
            sq = wave_sum(sq);
            sk = wave_sum(sk);
            const float iq = inv_norm(sq), ik = inv_norm(sk);
            const float sgn = r0 < PH ? -1.f : 1.f;
#pragma unroll
            for (int m = 0; m < RPT; ++m) {
                const float qn = elu1(qo[m]) * iq, kn = elu1(ko[m]) * ik;
                const float qn2 = elu1(qp[m]) * iq, kn2 = elu1(kp[m]) * ik;
                const float c = rope * cs[m] + (1.f - rope), sg = rope * sgn * sn2[m];
                qv[m] = qn * c + sg * qn2;
                kv[m] = kn * c + sg * kn2;
                dv[m] = sigmoid(gg[m]);
            }
        }

        fetch(nxt, more ? nrow : row, more);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        f32x4 y[RPT];
        float o4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < RPT; ++m) {
            const f32x4 s = unpack(cur.w[m]);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                y[m][c] = dv[m] * s[c] + kv[m] * vv[c];
                o4[c] += qv[m] * y[m][c];
            }
        }
        const int64_t sr = cur.srow;
        const auto ro = row_rsrc(a.state_out, sr, a.save_final != 0 && sr >= 0);
#pragma unroll
        for (int m = 0; m < RPT; ++m) {
            if constexpr (SB == 4) {
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, y[m]), ro, voff + m * HD * SB, 0, 2);
            } else {
                const V4<TS> v = V4<TS>{(TS)y[m][0], (TS)y[m][1], (TS)y[m][2], (TS)y[m][3]};
                __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), ro, voff + m * HD * SB, 0, 2);
            }
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) o4[c] = xor_group_sum<CG>(o4[c]);
        if (lane < CG) red[buf][wave][cg] = f32x4{o4[0], o4[1], o4[2], o4[3]};
        // barrier ordering LDS only: the state loads and stores in flight need not complete before it
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        // the readout: threads tid < CG store columns 4*cg .. 4*cg+3; the others issue the same
        // store past the row's records (dropped)
        {
            f32x4 s = red[buf][0][cg];
#pragma unroll
            for (int w = 1; w < WAVES; ++w) s += red[buf][w][cg];
            if (sr < 0) s = zero4();
            const int ob = dt_size(a.o_dt);
            const auto rout = __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<char*>(a.o) + (b * a.o_sb + h * a.o_sh) * ob,
                                                                (short)0, HD * ob, 0x00020000);
            buffer_store4_dt(rout, tid < CG ? 4 * cg * ob : HD * ob, a.o_dt, s);
        }
    };
    // Two state register sets used in turn, so no loaded state is ever copied between registers.
    Raw A, B;
    uint32_t row = blockIdx.x;
    fetch(A, row, true);
    while (row < rows) {
        step(A, B, row, 0);
        row += gridDim.x;
        if (row >= rows) break;
        step(B, A, row, 1);
        row += gridDim.x;
    }
}

// ---------------------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------------------
template <int HD, typename TIO, typename TCS>
static hipError_t launch_prep_t(const PrepParams& a, hipStream_t stream) {
    constexpr int RPB = 4 * (64 / (HD / 8));  // rows per 256-thread block
    const int64_t rows = a.B * a.T * a.H;
    hipLaunchKernelGGL((gla_prep_kernel<HD, TIO, TCS>), dim3((unsigned)((rows + RPB - 1) / RPB)), dim3(256), 0, stream,
                       a);
    return hipGetLastError();
}

template <typename TIO, typename TCS>
static hipError_t launch_prep_hd(const PrepParams& a, int HD, hipStream_t stream) {
    if (HD == 64) return launch_prep_t<64, TIO, TCS>(a, stream);
    if (HD == 128) return launch_prep_t<128, TIO, TCS>(a, stream);
    return launch_prep_t<32, TIO, TCS>(a, stream);
}

template <typename TIO>
static hipError_t launch_prep_cs(const PrepParams& a, int HD, int cs_dt, hipStream_t stream) {
    if (cs_dt == DT_F32) return launch_prep_hd<TIO, float>(a, HD, stream);
    if (cs_dt == DT_BF16) return launch_prep_hd<TIO, __bf16>(a, HD, stream);
    return launch_prep_hd<TIO, _Float16>(a, HD, stream);
}

hipError_t launch_gla_prep(const PrepParams& a, int HD, int io_dt, int cs_dt, hipStream_t stream) {
    if (HD != 32 && HD != 64 && HD != 128) return hipErrorInvalidValue;
    if (io_dt == DT_F32) return launch_prep_cs<float>(a, HD, cs_dt, stream);
    if (io_dt == DT_BF16) return launch_prep_cs<__bf16>(a, HD, cs_dt, stream);
    return launch_prep_cs<_Float16>(a, HD, cs_dt, stream);
}

template <int HD, typename TIO, typename TCS, typename TS>
static hipError_t launch_fdec_t(const FusedDecodeParams& a, hipStream_t stream) {
    const uint32_t rows = (uint32_t)(a.B * a.H);
    const uint32_t blocks = rows < (uint32_t)a.max_blocks ? rows : (uint32_t)a.max_blocks;
    hipLaunchKernelGGL((gla_fused_decode_kernel<HD, TIO, TCS, TS>), dim3(blocks), dim3(FusedDecodeTiling<HD>::TPB), 0,
                       stream, a, rows);
    return hipGetLastError();
}

template <int HD, typename TIO, typename TCS>
static hipError_t launch_fdec_s(const FusedDecodeParams& a, int s_dt, hipStream_t stream) {
    if (s_dt == DT_F32) return launch_fdec_t<HD, TIO, TCS, float>(a, stream);
    return launch_fdec_t<HD, TIO, TCS, TIO>(a, stream);  // state in the I/O type (checked by the caller)
}

template <int HD, typename TIO>
static hipError_t launch_fdec_cs(const FusedDecodeParams& a, int cs_dt, int s_dt, hipStream_t stream) {
    if (cs_dt == DT_F32) return launch_fdec_s<HD, TIO, float>(a, s_dt, stream);
    return launch_fdec_s<HD, TIO, TIO>(a, s_dt, stream);  // tables in the I/O type (checked by the caller)
}

template <typename TIO>
static hipError_t launch_fdec_hd(const FusedDecodeParams& a, int HD, int cs_dt, int s_dt, hipStream_t stream) {
    if (HD == 64) return launch_fdec_cs<64, TIO>(a, cs_dt, s_dt, stream);
    if (HD == 128) return launch_fdec_cs<128, TIO>(a, cs_dt, s_dt, stream);
    return launch_fdec_cs<32, TIO>(a, cs_dt, s_dt, stream);
}

hipError_t launch_gla_fused_decode(const FusedDecodeParams& a, int HD, int io_dt, int cs_dt, int s_dt,
                                   hipStream_t stream) {
    if (HD != 32 && HD != 64 && HD != 128) return hipErrorInvalidValue;
    if (io_dt == DT_F32) return launch_fdec_hd<float>(a, HD, cs_dt, s_dt, stream);
    if (io_dt == DT_BF16) return launch_fdec_hd<__bf16>(a, HD, cs_dt, s_dt, stream);
    return launch_fdec_hd<_Float16>(a, HD, cs_dt, s_dt, stream);
}

}  // namespace triune
