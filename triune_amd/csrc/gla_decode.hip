// gla_decode.hip -- batched O(1) GLA decode step on gfx950.
//
// For each row r = (b, h):   S <- diag(exp(g)) S + k v^T ;   o = S^T q
// with the fp32 state streamed from HBM once (read + write) per step.  Semantics follow the
// reference's T == 1 branch (triune/kernels/fast_gla.py:746-753; no clamp on g), its C
// decode step (csrc/engine/engine.cpp:419-475) and its CUDA decode kernel
// (csrc/kernels/gla.cu:23-75: bf16 q/k/v, fp32 log-gate, fp32 state in place, bf16 out).
//
// Thread layout: a 256-thread block updates one state row (b, h) at a time.  Thread (rg, cg) owns the RPT
// consecutive state rows rg*RPT .. rg*RPT+RPT-1 and columns 4*cg .. 4*cg+3, so a wave streams a
// contiguous RPT*16 rows x 256 B block with float4 accesses and every block has 4 waves in
// flight; the readout is reduced across row groups with lane shuffles inside a wave and LDS
// across the waves.  State accesses are nontemporal: each element is read and written once
// per step.
#include "kernels.h"

namespace triune {

// Four consecutive elements of a 16-bit or fp32 tensor, kept in their storage type until used.
template <typename T>
using Vec4 = T __attribute__((ext_vector_type(4)));

// TIO: dtype of q, k, v; TG: dtype of g.  A block walks rows blockIdx.x, + gridDim.x, ...; the
// next row's state loads are issued before this row's state is stored and its readout reduced,
// so reads of one row overlap the writes of the previous one.  The row's small q/k/g/v loads are
// issued at the top of its iteration (prefetching them as well measured 12% slower).
template <int DK, int DV, int RPT, typename TIO, typename TG>
__global__ __launch_bounds__(DK * DV / (4 * RPT)) void gla_decode_kernel(DecodeParams a, uint32_t rows) {
    constexpr int TPB = DK * DV / (4 * RPT);  // threads per block
    constexpr int CG = DV / 4;                // column groups (float4 columns)
    constexpr int WAVES = TPB / 64;
    static_assert(TPB % 64 == 0 && CG <= 64 && RPT % 4 == 0, "unsupported decode tiling");
    const int tid = threadIdx.x;
    const int cg = tid % CG, rg = tid / CG;
    const int r0 = rg * RPT;
    const int wave = tid / 64;
    const uint32_t H32 = (uint32_t)a.H;  // rows = B * H < 2^31

    struct In {
        f32x4 st[RPT];
        int64_t srow;  // state row (through slots when given)
    };
    struct Small {
        Vec4<TIO> q[RPT / 4], k[RPT / 4], v;
        Vec4<TG> g[RPT / 4];
    };
    // State row of (b, h), or -1 when b's slot lies outside the pool (a padded batch row): such a
    // row reads no state, stores none and outputs zeros.  The row is the same for the whole block.
    auto state_row = [&](uint32_t row) -> int64_t {
        const uint32_t b = row / H32, h = row % H32;
        if (!a.slots) return (int64_t)row;
        const int64_t sl = (int64_t)a.slots[b];
        return (sl >= 0 && sl < a.n_state_rows) ? sl * a.H + h : -1;
    };
    auto fetch = [&](In& x, uint32_t row) {
        x.srow = state_row(row);
        if (x.srow < 0) {
#pragma unroll
            for (int m = 0; m < RPT; ++m) x.st[m] = zero4();
            return;
        }
        const float* sin = a.state_in + x.srow * (int64_t)(DK * DV) + (int64_t)r0 * DV + 4 * cg;
#pragma unroll
        for (int m = 0; m < RPT; ++m)
            x.st[m] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(sin + m * DV));
    };
    auto fetch_small = [&](Small& x, uint32_t row) {
        const int64_t b = row / H32, h = row % H32;
        const TIO* q = reinterpret_cast<const TIO*>(a.q) + b * a.q_sb + h * a.q_sh + r0;
        const TIO* k = reinterpret_cast<const TIO*>(a.k) + b * a.k_sb + h * a.k_sh + r0;
        const TG* g = reinterpret_cast<const TG*>(a.g) + b * a.g_sb + h * a.g_sh + r0;
        const Vec4<TIO>* qp = reinterpret_cast<const Vec4<TIO>*>(q);
        const Vec4<TIO>* kp = reinterpret_cast<const Vec4<TIO>*>(k);
        const Vec4<TG>* gp = reinterpret_cast<const Vec4<TG>*>(g);
#pragma unroll
        for (int i = 0; i < RPT / 4; ++i) {
            x.q[i] = qp[i];
            x.k[i] = kp[i];
            x.g[i] = gp[i];
        }
        const TIO* v = reinterpret_cast<const TIO*>(a.v) + b * a.v_sb + h * a.v_sh + 4 * cg;
        x.v = *reinterpret_cast<const Vec4<TIO>*>(v);
    };
    __shared__ f32x4 red[2][WAVES][CG];
    uint32_t row = blockIdx.x;
    In cur;
    fetch(cur, row);
    for (int buf = 0; row < rows; row += gridDim.x, buf ^= 1) {
        Small sm;
        fetch_small(sm, row);
        f32x4 y[RPT];
        float o4[4] = {0.f, 0.f, 0.f, 0.f};
        float vv[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) vv[c] = (float)sm.v[c];
#pragma unroll
        for (int m = 0; m < RPT; ++m) {
            const float d = expf((float)sm.g[m / 4][m % 4]);
            const float km = (float)sm.k[m / 4][m % 4], qm = (float)sm.q[m / 4][m % 4];
            y[m] = cur.st[m];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                y[m][c] = d * y[m][c] + km * vv[c];
                o4[c] += qm * y[m][c];
            }
        }
        const int64_t srow = cur.srow;
        const uint32_t nrow = row + gridDim.x;
        if (nrow < rows) fetch(cur, nrow);
        if (srow >= 0) {
            float* sout = a.state_out + srow * (int64_t)(DK * DV) + (int64_t)r0 * DV + 4 * cg;
#pragma unroll
            for (int m = 0; m < RPT; ++m) __builtin_nontemporal_store(y[m], reinterpret_cast<f32x4*>(sout + m * DV));
        }
        // reduce over the row groups of a wave (lanes tid ^ CG*2^k share a column group) ...
#pragma unroll
        for (int c = 0; c < 4; ++c) o4[c] = xor_group_sum<CG>(o4[c]);
        // ... then across the waves (double-buffered: the next row's writes follow a barrier)
        if ((tid % 64) < CG) red[buf][wave][cg] = f32x4{o4[0], o4[1], o4[2], o4[3]};
        __syncthreads();
        if (tid < CG) {
            f32x4 s = red[buf][0][cg];
#pragma unroll
            for (int w = 1; w < WAVES; ++w) s += red[buf][w][cg];
            if (srow < 0) s = zero4();
            const int64_t b = row / H32, h = row % H32;
            const int64_t off = b * a.o_sb + h * a.o_sh + 4 * cg;
            store4_dt(reinterpret_cast<char*>(a.o) + off * dt_size(a.o_dt), a.o_dt, s[0], s[1], s[2], s[3]);
        }
    }
}

template <int DK, int DV, typename TIO, typename TG>
static hipError_t launch_decode_t(const DecodeParams& a, int max_blocks, hipStream_t stream) {
    constexpr int RPT = (DK * DV / (4 * 256)) > 4 ? (DK * DV / (4 * 256)) : 4;
    constexpr int TPB = DK * DV / (4 * RPT);
    const uint32_t rows = (uint32_t)(a.B * a.H);
    const uint32_t blocks = rows < (uint32_t)max_blocks ? rows : (uint32_t)max_blocks;
    hipLaunchKernelGGL((gla_decode_kernel<DK, DV, RPT, TIO, TG>), dim3(blocks), dim3(TPB), 0, stream, a, rows);
    return hipGetLastError();
}

template <int DK, int DV, typename TIO>
static hipError_t launch_decode_g(const DecodeParams& a, int mb, hipStream_t stream) {
    if (a.g_dt == DT_F32) return launch_decode_t<DK, DV, TIO, float>(a, mb, stream);
    if (a.g_dt == DT_BF16) return launch_decode_t<DK, DV, TIO, __bf16>(a, mb, stream);
    return launch_decode_t<DK, DV, TIO, _Float16>(a, mb, stream);
}

template <int DK, int DV>
static hipError_t launch_decode_io(const DecodeParams& a, int mb, hipStream_t stream) {
    if (a.io_dt == DT_F32) return launch_decode_g<DK, DV, float>(a, mb, stream);
    if (a.io_dt == DT_BF16) return launch_decode_g<DK, DV, __bf16>(a, mb, stream);
    return launch_decode_g<DK, DV, _Float16>(a, mb, stream);
}

// Supported (Dk, Dv): (32,32), (64,64), (128,128), (64,128), (128,64).  Returns
// hipErrorInvalidValue for other shapes.  max_blocks caps the grid (blocks then walk several
// rows); four blocks per CU measured best for the 16 KB rows of (64, 64).
hipError_t launch_gla_decode(const DecodeParams& a, int Dk, int Dv, int max_blocks, hipStream_t stream) {
    const int mb = max_blocks > 0 ? max_blocks : 1;
    if (Dk == 64 && Dv == 64) return launch_decode_io<64, 64>(a, mb, stream);
    if (Dk == 128 && Dv == 128) return launch_decode_io<128, 128>(a, mb, stream);
    if (Dk == 32 && Dv == 32) return launch_decode_io<32, 32>(a, mb, stream);
    if (Dk == 64 && Dv == 128) return launch_decode_io<64, 128>(a, mb, stream);
    if (Dk == 128 && Dv == 64) return launch_decode_io<128, 64>(a, mb, stream);
    return hipErrorInvalidValue;
}

}  // namespace triune
