// gla_decode.hip -- batched O(1) GLA decode step on gfx950.
//
// For each row r = (b, h):   S <- diag(exp(g)) S + k v^T ;   o = S^T q
// with the fp32 state streamed from HBM once (read + write) per step.  Semantics follow the
// reference's T == 1 branch (triune/kernels/fast_gla.py:746-753; no clamp on g), its C
// decode step (csrc/engine/engine.cpp:419-475) and its CUDA decode kernel
// (csrc/kernels/gla.cu:23-75: bf16 q/k/v, fp32 log-gate, fp32 state in place, bf16 out).
//
// Thread layout: one state row (b, h) per 256-thread block.  Thread (rg, cg) owns the RPT
// consecutive state rows rg*RPT .. rg*RPT+RPT-1 and columns 4*cg .. 4*cg+3, so a wave streams a
// contiguous RPT*16 rows x 256 B block with float4 accesses and every block has 4 waves in
// flight; the readout is reduced across row groups with lane shuffles inside a wave and LDS
// across the waves.  State accesses are nontemporal: each element is read and written once
// per step.
#include "kernels.h"

namespace triune {

__device__ __forceinline__ void load_small(const void* base, int dt, int64_t off, float* x, int n) {
    // n (4 or a multiple of 8) consecutive elements at element offset off
    const char* p = reinterpret_cast<const char*>(base) + off * dt_size(dt);
    if (n % 8 == 0) {
        for (int c = 0; c < n; c += 8) {
            float y[8];
            load8_dt(p + c * dt_size(dt), dt, true, y);
#pragma unroll
            for (int j = 0; j < 8; ++j) x[c + j] = y[j];
        }
        return;
    }
    if (dt == DT_F32) {
        float4 t = *reinterpret_cast<const float4*>(p);
        x[0] = t.x; x[1] = t.y; x[2] = t.z; x[3] = t.w;
    } else if (dt == DT_BF16) {
        bf16x4 t = *reinterpret_cast<const bf16x4*>(p);
        x[0] = (float)t[0]; x[1] = (float)t[1]; x[2] = (float)t[2]; x[3] = (float)t[3];
    } else {
        typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
        f16x4 t = *reinterpret_cast<const f16x4*>(p);
        x[0] = (float)t[0]; x[1] = (float)t[1]; x[2] = (float)t[2]; x[3] = (float)t[3];
    }
}

template <int DK, int DV, int RPT>
__global__ __launch_bounds__(DK * DV / (4 * RPT)) void gla_decode_kernel(DecodeParams a) {
    constexpr int TPB = DK * DV / (4 * RPT);  // threads per block (one state row)
    constexpr int CG = DV / 4;                // column groups (float4 columns)
    constexpr int WAVES = TPB / 64;
    static_assert(TPB % 64 == 0 && CG <= 64 && (RPT == 4 || RPT % 8 == 0), "unsupported decode tiling");
    const int tid = threadIdx.x;
    const int64_t row = blockIdx.x;
    const int64_t b = row / a.H, h = row % a.H;
    const int cg = tid % CG, rg = tid / CG;
    const int r0 = rg * RPT;

    float qv[RPT], kv[RPT], gv[RPT], vv[4];
    load_small(a.q, a.io_dt, b * a.q_sb + h * a.q_sh + r0, qv, RPT);
    load_small(a.k, a.io_dt, b * a.k_sb + h * a.k_sh + r0, kv, RPT);
    load_small(a.g, a.g_dt, b * a.g_sb + h * a.g_sh + r0, gv, RPT);
    load_small(a.v, a.io_dt, b * a.v_sb + h * a.v_sh + 4 * cg, vv, 4);
    const int64_t srow = a.slots ? (int64_t)a.slots[b] * a.H + h : row;
    const float* sin = a.state_in + srow * (int64_t)(DK * DV) + (int64_t)r0 * DV + 4 * cg;
    float* sout = a.state_out + srow * (int64_t)(DK * DV) + (int64_t)r0 * DV + 4 * cg;
    f32x4 st[RPT];
#pragma unroll
    for (int m = 0; m < RPT; ++m) st[m] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(sin + m * DV));
    float o4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < RPT; ++m) {
        const float d = expf(gv[m]);
        f32x4 s = st[m];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            s[c] = d * s[c] + kv[m] * vv[c];
            o4[c] += qv[m] * s[c];
        }
        __builtin_nontemporal_store(s, reinterpret_cast<f32x4*>(sout + m * DV));
    }
    // reduce over the row groups of a wave (lanes tid ^ CG*2^k share a column group) ...
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int sh = CG; sh < 64; sh <<= 1) o4[c] += __shfl_xor(o4[c], sh);
    // ... then across the four waves
    __shared__ f32x4 red[WAVES][CG];
    const int wave = tid / 64;
    if ((tid % 64) < CG) red[wave][cg] = f32x4{o4[0], o4[1], o4[2], o4[3]};
    __syncthreads();
    if (tid < CG) {
        f32x4 s = red[0][cg];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) s += red[w][cg];
        const int64_t off = b * a.o_sb + h * a.o_sh + 4 * cg;
        store4_dt(reinterpret_cast<char*>(a.o) + off * dt_size(a.o_dt), a.o_dt, s[0], s[1], s[2], s[3]);
    }
}

template <int DK, int DV>
static hipError_t launch_decode_t(const DecodeParams& a, hipStream_t stream) {
    constexpr int RPT = (DK * DV / (4 * 256)) > 4 ? (DK * DV / (4 * 256)) : 4;
    constexpr int TPB = DK * DV / (4 * RPT);
    dim3 grid((unsigned)(a.B * a.H));
    hipLaunchKernelGGL((gla_decode_kernel<DK, DV, RPT>), grid, dim3(TPB), 0, stream, a);
    return hipGetLastError();
}

// Supported (Dk, Dv): (32,32), (64,64), (128,128), (64,128), (128,64).  Returns
// hipErrorInvalidValue for other shapes.
hipError_t launch_gla_decode(const DecodeParams& a, int Dk, int Dv, hipStream_t stream) {
    if (Dk == 64 && Dv == 64) return launch_decode_t<64, 64>(a, stream);
    if (Dk == 128 && Dv == 128) return launch_decode_t<128, 128>(a, stream);
    if (Dk == 32 && Dv == 32) return launch_decode_t<32, 32>(a, stream);
    if (Dk == 64 && Dv == 128) return launch_decode_t<64, 128>(a, stream);
    if (Dk == 128 && Dv == 64) return launch_decode_t<128, 64>(a, stream);
    return hipErrorInvalidValue;
}

}  // namespace triune
