// gla_prefill_prep.hip -- the segment-state kernel with VectorisedGLA's input pre-processing
// (gla_prefill.h, PREP instances of gla_seg_state_kernel): q, k, g arrive as raw projections; the
// kernel writes RoPE(normalize(elu(x) + 1)) of q and k and logsigmoid(g) back over them while it
// forms the segment states, and the plain output kernel then reads the processed tensors
// (reference: triune/model/attention.py:14-79, the in-place prep kernel, then the scan launched at
// :443-451; here the prep kernel's separate pass is gone).  Dense [B, T, H, D] inputs, Dk = Dv = D
// in {32, 64, 128}, bf16 or fp16 I/O, g in the I/O dtype, fp32 RoPE tables.
#include "gla_prefill.h"

namespace triune {

template <typename TIn, bool CK>
static hipError_t launch_prep_ck(const PrefillParams& a, int64_t n_work, hipStream_t stream) {
    const dim3 grid((unsigned)n_work, (unsigned)a.H);
    const dim3 block((unsigned)(a.Dv * 4));
#define TRIUNE_PREP_CASE(D_)                                                                                 \
    if (a.Dk == D_ && a.Dv == D_) {                                                                          \
        hipLaunchKernelGGL((gla_seg_state_kernel<TIn, TIn, D_, D_, CK, true>), grid, block, 0, stream, a);   \
        return hipGetLastError();                                                                            \
    }
    TRIUNE_PREP_CASE(64)
    TRIUNE_PREP_CASE(128)
    TRIUNE_PREP_CASE(32)
#undef TRIUNE_PREP_CASE
    return hipErrorInvalidValue;
}

bool prefill_prep_supported(int D, int io_dt) {
    return (D == 32 || D == 64 || D == 128) && (io_dt == DT_BF16 || io_dt == DT_F16);
}

// Unchecked row addressing only when T is a whole number of four-row groups (as for the raw path).
hipError_t launch_gla_prep_seg_state(const PrefillParams& a, int64_t n_work, int io_dt, hipStream_t stream) {
    const bool ck = a.T % 4 != 0;
    if (io_dt == DT_BF16)
        return ck ? launch_prep_ck<__bf16, true>(a, n_work, stream) : launch_prep_ck<__bf16, false>(a, n_work, stream);
    if (io_dt == DT_F16)
        return ck ? launch_prep_ck<_Float16, true>(a, n_work, stream) : launch_prep_ck<_Float16, false>(a, n_work, stream);
    return hipErrorInvalidValue;
}

}  // namespace triune
