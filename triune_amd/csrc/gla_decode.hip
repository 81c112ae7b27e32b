// gla_decode.hip -- batched O(1) GLA decode step on gfx950.
//
// For each row r = (b, h):   S <- diag(exp(g)) S + k v^T ;   o = S^T q
// with the fp32 state streamed from HBM once (read + write) per step.  Semantics follow the
// reference's T == 1 branch (triune/kernels/fast_gla.py:746-753; no clamp on g), its C
// decode step (csrc/engine/engine.cpp:419-475) and its CUDA decode kernel
// (csrc/kernels/gla.cu:23-75: bf16 q/k/v, fp32 log-gate, fp32 state in place, bf16 out).
//
// Thread layout: TPB threads per row; thread (rg, cg) owns state rows 16*rg + m (m < RPT)
// and columns 4*cg .. 4*cg+3, so each wave-wide float4 access touches whole 256-byte
// (Dv=64) row segments.  q/k/g for a thread's rows are two 16-byte loads each; the readout
// is reduced across row groups with lane shuffles (and LDS when a row spans several waves).
#include "kernels.h"

namespace triune {

__device__ __forceinline__ void load_rows(const void* base, int dt, int64_t off, float* x, int n) {
    // n consecutive elements (n multiple of 8) starting at element offset off
    for (int c = 0; c < n; c += 8) {
        float y[8];
        load8_dt(reinterpret_cast<const char*>(base) + (off + c) * dt_size(dt), dt, true, y);
#pragma unroll
        for (int j = 0; j < 8; ++j) x[c + j] = y[j];
    }
}

template <int DK, int DV, int TPB>
__global__ __launch_bounds__(256) void gla_decode_kernel(DecodeParams a) {
    constexpr int CG = DV / 4;         // column groups
    constexpr int RG = TPB / CG;       // row groups
    constexpr int RPT = DK / RG;       // rows per thread
    constexpr int ROWS_PER_BLOCK = 256 / TPB;
    static_assert(RPT % 8 == 0, "rows per thread must be a multiple of 8");
    const int tid = threadIdx.x % TPB;
    const int64_t row = (int64_t)blockIdx.x * ROWS_PER_BLOCK + threadIdx.x / TPB;
    const bool active = row < a.B * a.H;
    const int64_t b = active ? row / a.H : 0, h = active ? row % a.H : 0;
    const int cg = tid % CG, rg = tid / CG;
    const int r0 = rg * RPT;

    float o4[4] = {0.f, 0.f, 0.f, 0.f};
    if (active) {
        float qv[RPT], kv[RPT], gv[RPT], vv[4];
        load_rows(a.q, a.io_dt, b * a.q_sb + h * a.q_sh + r0, qv, RPT);
        load_rows(a.k, a.io_dt, b * a.k_sb + h * a.k_sh + r0, kv, RPT);
        load_rows(a.g, a.g_dt, b * a.g_sb + h * a.g_sh + r0, gv, RPT);
        {
            const int64_t off = b * a.v_sb + h * a.v_sh + 4 * cg;
            if (a.io_dt == DT_F32) {
                float4 t = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(a.v) + off);
                vv[0] = t.x; vv[1] = t.y; vv[2] = t.z; vv[3] = t.w;
            } else if (a.io_dt == DT_BF16) {
                bf16x4 t = *reinterpret_cast<const bf16x4*>(reinterpret_cast<const __bf16*>(a.v) + off);
                vv[0] = (float)t[0]; vv[1] = (float)t[1]; vv[2] = (float)t[2]; vv[3] = (float)t[3];
            } else {
                typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
                f16x4 t = *reinterpret_cast<const f16x4*>(reinterpret_cast<const _Float16*>(a.v) + off);
                vv[0] = (float)t[0]; vv[1] = (float)t[1]; vv[2] = (float)t[2]; vv[3] = (float)t[3];
            }
        }
        const int64_t srow = a.slots ? (int64_t)a.slots[b] * a.H + h : row;
        const float* sin = a.state_in + srow * (int64_t)(DK * DV) + (int64_t)r0 * DV + 4 * cg;
        float* sout = a.state_out + srow * (int64_t)(DK * DV) + (int64_t)r0 * DV + 4 * cg;
        float4 st[RPT];
#pragma unroll
        for (int m = 0; m < RPT; ++m) st[m] = *reinterpret_cast<const float4*>(sin + m * DV);
#pragma unroll
        for (int m = 0; m < RPT; ++m) {
            const float d = expf(gv[m]);
            float4 s = st[m];
            s.x = d * s.x + kv[m] * vv[0];
            s.y = d * s.y + kv[m] * vv[1];
            s.z = d * s.z + kv[m] * vv[2];
            s.w = d * s.w + kv[m] * vv[3];
            st[m] = s;
            o4[0] += qv[m] * s.x;
            o4[1] += qv[m] * s.y;
            o4[2] += qv[m] * s.z;
            o4[3] += qv[m] * s.w;
        }
#pragma unroll
        for (int m = 0; m < RPT; ++m) *reinterpret_cast<float4*>(sout + m * DV) = st[m];
    }
    // reduce the readout over row groups: lanes tid and tid ^ (CG * 2^k) share a column group
    constexpr int IN_WAVE = (64 / CG) < RG ? (64 / CG) : RG;  // row groups inside one wave
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int sh = CG; sh < CG * IN_WAVE; sh <<= 1) o4[c] += __shfl_xor(o4[c], sh);
    constexpr int WAVES = TPB / 64;  // waves per row (>1 only when a row spans several waves)
    if constexpr (WAVES > 1) {
        __shared__ float red[ROWS_PER_BLOCK][WAVES][CG][4];
        const int wave = tid / 64;
        if ((tid % 64) < CG) {
#pragma unroll
            for (int c = 0; c < 4; ++c) red[threadIdx.x / TPB][wave][cg][c] = o4[c];
        }
        __syncthreads();
        if (tid < CG) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                float s = 0.f;
#pragma unroll
                for (int w = 0; w < WAVES; ++w) s += red[threadIdx.x / TPB][w][cg][c];
                o4[c] = s;
            }
        }
    }
    if (active && tid < CG) {
        const int64_t off = b * a.o_sb + h * a.o_sh + 4 * cg;
        char* op = reinterpret_cast<char*>(a.o) + off * dt_size(a.o_dt);
        store4_dt(op, a.o_dt, o4[0], o4[1], o4[2], o4[3]);
    }
}

template <int DK, int DV, int TPB>
static hipError_t launch_decode_t(const DecodeParams& a, hipStream_t stream) {
    constexpr int ROWS_PER_BLOCK = 256 / TPB;
    const int64_t rows = a.B * a.H;
    dim3 grid((unsigned)((rows + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK));
    hipLaunchKernelGGL((gla_decode_kernel<DK, DV, TPB>), grid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

// Supported (Dk, Dv): (32,32), (64,64), (128,128), (64,128), (128,64).  Returns
// hipErrorInvalidValue for other shapes.
hipError_t launch_gla_decode(const DecodeParams& a, int Dk, int Dv, hipStream_t stream) {
    if (Dk == 64 && Dv == 64) return launch_decode_t<64, 64, 64>(a, stream);
    if (Dk == 128 && Dv == 128) return launch_decode_t<128, 128, 256>(a, stream);
    if (Dk == 32 && Dv == 32) return launch_decode_t<32, 32, 32>(a, stream);
    if (Dk == 64 && Dv == 128) return launch_decode_t<64, 128, 128>(a, stream);
    if (Dk == 128 && Dv == 64) return launch_decode_t<128, 64, 128>(a, stream);
    return hipErrorInvalidValue;
}

}  // namespace triune
