// gla_prefill.hip -- instances and host launchers of the chunked GLA prefill (gla_prefill.h):
// raw q/k/g inputs, dense and varlen, and the varlen plan kernel.
#include "gla_prefill.h"

#include <hip/hip_ext.h>

namespace triune {

// K0 (varlen): segment offsets from cu_seqlens, one thread block.
__global__ __launch_bounds__(256) void gla_varlen_plan_kernel(const int32_t* cu, int64_t n_seqs, int P,
                                                               int32_t* seg_off) {
    __shared__ int32_t part[256];
    int32_t base = 0;
    if (threadIdx.x == 0) seg_off[0] = 0;
    for (int64_t s0 = 0; s0 < n_seqs; s0 += 256) {
        const int64_t s = s0 + threadIdx.x;
        int32_t n = 0;
        if (s < n_seqs) {
            int64_t len = (int64_t)cu[s + 1] - (int64_t)cu[s];
            if (len < 0) len = 0;
            const int64_t chunks = (len + CHUNK - 1) / CHUNK;
            n = (int32_t)((chunks + P - 1) / P);
        }
        part[threadIdx.x] = n;
        __syncthreads();
        for (int off = 1; off < 256; off <<= 1) {
            const int32_t add = threadIdx.x >= off ? part[threadIdx.x - off] : 0;
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
bool prefill_shape_supported(int Dk, int Dv) {
    return (Dk == 32 && Dv == 32) || (Dk == 64 && Dv == 64) || (Dk == 128 && Dv == 128) || (Dk == 128 && Dv == 64);
}

// fp32 I/O keeps three bf16 parts of every LDS operand: at (128, 128) they exceed the 160 KB LDS,
// so that pair is served as two 64-column halves by the caller.
bool prefill_dtype_supported(int Dk, int Dv, int io_dt) {
    return prefill_shape_supported(Dk, Dv) && !(io_dt == DT_F32 && Dk == 128 && Dv == 128);
}

// ev0 / ev1 (output kernel only): events stamped with the kernel's own start and end
// (hipExtLaunchKernel), or null.
template <typename TIn, typename TG, bool CK>
static hipError_t launch_seg_ck(const PrefillParams& a, int64_t n_work, bool with_out, hipStream_t stream,
                                hipEvent_t ev0, hipEvent_t ev1) {
    const dim3 grid((unsigned)n_work, (unsigned)a.H);
    const dim3 block((unsigned)(a.Dv * 4));
    constexpr bool OBF_ok = std::is_same<TIn, __bf16>::value;
    const bool obf = OBF_ok && a.o_dt == DT_BF16;
    auto out = [&](auto kern) {
        if (ev0 || ev1) hipExtLaunchKernelGGL(kern, grid, block, 0, stream, ev0, ev1, 0, a);
        else hipLaunchKernelGGL(kern, grid, block, 0, stream, a);
    };
#define TRIUNE_SEG_CASE(DK_, DV_)                                                                       \
    if (a.Dk == DK_ && a.Dv == DV_) {                                                                   \
        if (with_out && obf) out(gla_seg_output_kernel<TIn, TG, DK_, DV_, CK, OBF_ok>);                  \
        else if (with_out) out(gla_seg_output_kernel<TIn, TG, DK_, DV_, CK, false>);                     \
        else hipLaunchKernelGGL((gla_seg_state_kernel<TIn, TG, DK_, DV_, CK>), grid, block, 0, stream, a); \
        return hipGetLastError();                                                                       \
    }
    TRIUNE_SEG_CASE(64, 64)
    if constexpr (!Prec<TIn>::F32) {
        TRIUNE_SEG_CASE(128, 128)
    }
    TRIUNE_SEG_CASE(32, 32)
    TRIUNE_SEG_CASE(128, 64)
#undef TRIUNE_SEG_CASE
    return hipErrorInvalidValue;
}

// Unchecked row addressing only when every sequence is a whole number of four-row groups (dense
// with T % 4 == 0): then no chunk reaches past a tensor's extent with part of a group.
template <typename TIn, typename TG>
static hipError_t launch_seg_t(const PrefillParams& a, int64_t n_work, bool with_out, hipStream_t stream,
                               hipEvent_t ev0, hipEvent_t ev1) {
    if (!a.varlen && a.T % 4 == 0) return launch_seg_ck<TIn, TG, false>(a, n_work, with_out, stream, ev0, ev1);
    return launch_seg_ck<TIn, TG, true>(a, n_work, with_out, stream, ev0, ev1);
}

static hipError_t launch_seg(const PrefillParams& a, int64_t n_work, int io_dt, bool with_out, hipStream_t stream,
                             hipEvent_t ev0 = nullptr, hipEvent_t ev1 = nullptr) {
    const bool g32 = a.g_dt == DT_F32;
    if (io_dt == DT_BF16) {
        if (g32) return launch_seg_t<__bf16, float>(a, n_work, with_out, stream, ev0, ev1);
        if (a.g_dt == DT_BF16) return launch_seg_t<__bf16, __bf16>(a, n_work, with_out, stream, ev0, ev1);
    } else if (io_dt == DT_F16) {
        if (g32) return launch_seg_t<_Float16, float>(a, n_work, with_out, stream, ev0, ev1);
        if (a.g_dt == DT_F16) return launch_seg_t<_Float16, _Float16>(a, n_work, with_out, stream, ev0, ev1);
    } else if (io_dt == DT_F32 && g32) {
        return launch_seg_t<float, float>(a, n_work, with_out, stream, ev0, ev1);
    }
    return hipErrorInvalidValue;
}

// Resident workgroups per CU of the output kernel for (Dk, Dv) on the instance that runs (ck:
// checked row addressing, see launch_seg_t; bf16 I/O instance: the other dtypes use at least as
// much LDS, so this is an upper bound that only costs balance).
int gla_seg_output_blocks_per_cu(int Dk, int Dv, bool ck) {
    int nb = 0;
    hipError_t e = hipErrorInvalidValue;
#define TRIUNE_OCC_CASE(DK_, DV_)                                                                             \
    if (Dk == DK_ && Dv == DV_)                                                                               \
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(                                                     \
            &nb,                                                                                              \
            ck ? reinterpret_cast<const void*>(gla_seg_output_kernel<__bf16, __bf16, DK_, DV_, true, false>)         \
               : reinterpret_cast<const void*>(gla_seg_output_kernel<__bf16, __bf16, DK_, DV_, false, false>),       \
            DV_ * 4, 0);
    TRIUNE_OCC_CASE(64, 64)
    TRIUNE_OCC_CASE(128, 128)
    TRIUNE_OCC_CASE(32, 32)
    TRIUNE_OCC_CASE(128, 64)
#undef TRIUNE_OCC_CASE
    return (e == hipSuccess && nb > 0) ? nb : 1;
}

hipError_t launch_gla_seg_state(const PrefillParams& a, int64_t n_work, int io_dt, hipStream_t stream) {
    return launch_seg(a, n_work, io_dt, false, stream);
}

hipError_t launch_gla_seg_output(const PrefillParams& a, int64_t n_work, int io_dt, hipStream_t stream, hipEvent_t ev0,
                                 hipEvent_t ev1) {
    return launch_seg(a, n_work, io_dt, true, stream, ev0, ev1);
}

hipError_t launch_gla_varlen_plan(const int32_t* cu, int64_t n_seqs, int P, int32_t* seg_off, hipStream_t stream) {
    hipLaunchKernelGGL(gla_varlen_plan_kernel, dim3(1), dim3(256), 0, stream, cu, n_seqs, P, seg_off);
    return hipGetLastError();
}

}  // namespace triune
