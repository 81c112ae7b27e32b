// abi.hip -- extern "C" entry points of libtriune_hip.so (declared in include/triune_hip.h).
// Argument validation, workspace layout and the launch sequence of each operator.
#include "../../include/triune_hip.h"
#include "kernels.h"

#include <atomic>
#include <initializer_list>
#include <map>
#include <mutex>

using namespace triune;

namespace {

constexpr size_t kAlign = 256;

size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

bool dtype_ok(int dt) { return dt == TRIUNE_DT_F32 || dt == TRIUNE_DT_BF16 || dt == TRIUNE_DT_F16; }

// 16-byte vector access of 8 elements (16-bit) or 2x4 elements (fp32) needs every row start
// 16-byte aligned: base pointer aligned and strides a multiple of 16 bytes.
bool vec_ok(const void* p, int dt, const int64_t* st, int n) {
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return false;
    const int64_t m = dt == TRIUNE_DT_F32 ? 4 : 8;
    for (int i = 0; i < n; ++i)
        if (st[i] % m != 0) return false;
    return true;
}

// 8-byte access of 4 elements (16-bit) or 16-byte (fp32).
bool vec4_ok(const void* p, int dt, const int64_t* st, int n) {
    if (reinterpret_cast<uintptr_t>(p) % (dt == TRIUNE_DT_F32 ? 16 : 8) != 0) return false;
    for (int i = 0; i < n; ++i)
        if (st[i] % 4 != 0) return false;
    return true;
}

// Per-device query caches: fixed arrays (no host allocation on any call path); 0 = not queried
// yet.  Concurrent first queries store the same value.
constexpr int kMaxDevices = 64;

int current_device() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return -1;
    return dev;
}

// Compute units of the current device, queried once per device (MI355X: 256).
int device_cus() {
    static std::atomic<int> cache[kMaxDevices];
    const int dev = current_device();
    if (dev >= 0) {
        const int c = cache[dev].load(std::memory_order_relaxed);
        if (c > 0) return c;
    }
    int ncu = 0;
    if (dev < 0 || hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || ncu <= 0)
        ncu = 256;  // MI355X
    if (dev >= 0) cache[dev].store(ncu, std::memory_order_relaxed);
    return ncu;
}

// Grid cap of the fused decode step, in workgroups per CU: at the config-2 shape (B = 256,
// H = 6, HD = 64: 1536 rows) 9.2 us per step at 5, 9.9 at 4, 9.7 at 4.5, 11.0 at 5.5 and
// 10.6 at 6.  The plain and Gated DeltaNet decode steps measured best at 4.
constexpr int kFusedDecodeBlocksPerCU = 5;

// Resident (segment, head) workgroups the device holds at once: CUs x output-kernel occupancy
// of the instance that runs (ck: checked row addressing, used unless every sequence length is a
// multiple of 4).  Queried once per device and cached (host-side runtime queries only; nothing
// is enqueued).
int64_t resident_slots(int Dk, int Dv, bool ck) {
    static std::atomic<int64_t> cache[kMaxDevices][4][2];
    const int pair = Dk == 32 ? 0 : (Dk == 64 ? 1 : (Dv == 64 ? 2 : 3));  // (32,32) (64,64) (128,64) (128,128)
    const int dev = current_device();
    if (dev >= 0) {
        const int64_t c = cache[dev][pair][ck].load(std::memory_order_relaxed);
        if (c > 0) return c;
    }
    const int64_t slots = (int64_t)device_cus() * gla_seg_output_blocks_per_cu(Dk, Dv, ck);
    if (dev >= 0) cache[dev][pair][ck].store(slots, std::memory_order_relaxed);
    return slots;
}

// Segments per sequence (dense): fill the resident workgroup slots once with near-equal
// segments; never more segments than chunks.  flags bits 8..15 force a chunk count instead.
int64_t dense_segments(int64_t B, int64_t H, int64_t nchunks, int Dk, int Dv, int flags, bool ck) {
    const int forced = (flags >> TRIUNE_FLAG_SEG_SHIFT) & 0xff;
    if (forced > 0) return (nchunks + forced - 1) / forced;
    int64_t nseg = resident_slots(Dk, Dv, ck) / (B * H);
    if (nseg < 1) nseg = 1;
    if (nseg > nchunks) nseg = nchunks;
    return nseg;
}

// Chunks per segment (varlen): about eight resident rounds of workgroups.  Sequence lengths
// vary, so segments sized for a single round leave the longest walks (up to a whole sequence)
// on the critical path; at config 4 (32 sequences of 128..8192 tokens, D = 128) one round
// (111 chunks per segment) took 3.2 ms and eight rounds (14) 2.1 ms, with 4..32 all within 10 %.
int varlen_seg_chunks(int64_t chunk_jobs, int Dk, int Dv, int flags) {
    const int forced = (flags >> TRIUNE_FLAG_SEG_SHIFT) & 0xff;
    if (forced > 0) return forced;
    const int64_t slots = resident_slots(Dk, Dv, true) * 8;  // varlen runs the checked instances
    int64_t p = (chunk_jobs + slots - 1) / slots;
    if (p < 4) p = 4;
    if (p > 255) p = 255;
    return (int)p;
}

bool prefill_shape_ok(int Dk, int Dv) { return prefill_shape_supported(Dk, Dv); }

// The prefill kernels address the 64 rows of a chunk as a uniform base plus a 32-bit per-lane
// byte offset: 64 token strides plus one row must stay below 2^31 bytes.  Their loads read a
// (sequence, head) only up to t_end token strides past its first row, which covers every row of
// the sequence only when rows do not overlap: the token stride must be at least the row width
// (a tensor broadcast along tokens, stride 0, is copied by the caller).
bool tok_strides_ok(const int64_t* st3_q, int io_dtype, int g_dtype, int o_dtype, int Dk, int Dv) {
    auto ok = [](int64_t st, int dt, int D) {
        const int64_t es = dt == TRIUNE_DT_F32 ? 4 : 2;
        return st >= D && (64 * st + D) * es < ((int64_t)1 << 31);
    };
    return ok(st3_q[1], io_dtype, Dk) && ok(st3_q[4], io_dtype, Dk) && ok(st3_q[7], io_dtype, Dv) &&
           ok(st3_q[10], g_dtype, Dk) && ok(st3_q[13], o_dtype, Dv);
}

bool gate_dtype_ok(int io_dtype, int g_dtype) { return g_dtype == io_dtype || g_dtype == TRIUNE_DT_F32; }

struct PrefillPlan {
    int P;
    int64_t nseg, n_work;
    size_t off_segoff, off_state, off_gamma, total;
};

PrefillPlan plan_dense(int64_t B, int64_t T, int64_t H, int Dk, int Dv, int flags) {
    PrefillPlan p{};
    const int64_t nchunks = (T + 63) / 64;
    p.nseg = dense_segments(B, H, nchunks, Dk, Dv, flags, T % 4 != 0);
    p.P = (int)((nchunks + p.nseg - 1) / p.nseg);
    p.n_work = B * p.nseg;
    p.off_segoff = 0;
    p.off_state = 0;
    p.off_gamma = align_up((size_t)p.n_work * H * Dk * Dv * sizeof(float));
    p.total = p.off_gamma + align_up((size_t)p.n_work * H * Dk * sizeof(float));
    return p;
}

PrefillPlan plan_varlen(int64_t n_seqs, int64_t total_tokens, int64_t H, int Dk, int Dv, int flags) {
    PrefillPlan p{};
    const int64_t nchunks = (total_tokens + 63) / 64 + n_seqs;
    p.P = varlen_seg_chunks(H * nchunks, Dk, Dv, flags);
    p.n_work = (total_tokens + 64 * (int64_t)p.P - 1) / (64 * (int64_t)p.P) + n_seqs;
    p.nseg = 0;
    p.off_segoff = 0;
    p.off_state = align_up((size_t)(n_seqs + 1) * sizeof(int32_t));
    p.off_gamma = p.off_state + align_up((size_t)p.n_work * H * Dk * Dv * sizeof(float));
    p.total = p.off_gamma + align_up((size_t)p.n_work * H * Dk * sizeof(float));
    return p;
}

// Backward workspace: the forward's segment plan and workspaces, then the segment maps R (later
// the gradient at each segment's end), the segment end states and every chunk's starting state.
struct BwdPlan {
    PrefillPlan f;
    int64_t nchunks;
    size_t off_r, off_send, off_chunk, total;
};

BwdPlan plan_bwd(int64_t B, int64_t T, int64_t H, int D, int flags) {
    BwdPlan p{};
    p.f = plan_dense(B, T, H, D, D, flags);
    p.nchunks = (T + 63) / 64;
    const size_t dd = (size_t)D * D * sizeof(float);
    p.off_r = p.f.total;
    p.off_send = p.off_r + align_up((size_t)p.f.n_work * H * dd);
    p.off_chunk = p.off_send + align_up((size_t)p.f.n_work * H * dd);
    p.total = p.off_chunk + align_up((size_t)B * H * p.nchunks * dd);
    return p;
}

int launch_status(hipError_t e) { return e == hipSuccess ? TRIUNE_OK : TRIUNE_ERR_LAUNCH; }

int dense_launch(PrefillParams& a, const PrefillPlan& pl, const float* s0, float* s_final, int io_dtype, bool prep,
                 hipStream_t st);

// Events armed by triune_hip_set_output_kernel_events for this host thread (null: disarmed).
struct OutputEvents {
    hipEvent_t begin = nullptr, end = nullptr;
};
thread_local OutputEvents g_output_events;

// The GLA output kernel; armed events ride on its dispatch (hipExtLaunchKernel), the tightest
// placement HIP offers: on MI355X they still read about 4 us above the kernel trace's duration
// (the dispatch latency), against 4-7 us for markers recorded around the launch.
int launch_output_timed(const PrefillParams& a, int64_t n_work, int io_dtype, hipStream_t st) {
    const OutputEvents ev = g_output_events;
    return launch_status(launch_gla_seg_output(a, n_work, io_dtype, st, ev.begin, ev.end));
}

}  // namespace

extern "C" {

int triune_hip_abi_version(void) { return TRIUNE_HIP_ABI_VERSION; }

int triune_hip_set_output_kernel_events(void* begin, void* end) {
    if ((begin == nullptr) != (end == nullptr)) return TRIUNE_ERR_NULL;
    g_output_events.begin = reinterpret_cast<hipEvent_t>(begin);
    g_output_events.end = reinterpret_cast<hipEvent_t>(end);
    return TRIUNE_OK;
}

const char* triune_hip_error_string(int code) {
    switch (code) {
        case TRIUNE_OK: return "ok";
        case TRIUNE_ERR_NULL: return "a required pointer is NULL";
        case TRIUNE_ERR_SHAPE: return "unsupported or inconsistent sizes";
        case TRIUNE_ERR_DTYPE: return "unsupported dtype code";
        case TRIUNE_ERR_LAYOUT: return "stride or alignment requirement not met";
        case TRIUNE_ERR_WORKSPACE: return "workspace missing or too small";
        case TRIUNE_ERR_LAUNCH: return "HIP kernel launch failed";
        case TRIUNE_ERR_SCRATCH:
            return "problem exceeds the static scratch of the allocation-free entry point "
                   "(use the entry point that takes a workspace)";
        case TRIUNE_ERR_MEMORY: return "a pointer is not device memory of the current device";
        default: return "unknown error";
    }
}

int triune_hip_gla_decode_step(const void* q, const void* k, const void* v, const void* g, int io_dtype,
                               int g_dtype, const int64_t* strides, const float* state_in, float* state_out,
                               const int32_t* slots, int64_t n_state_rows, void* o, int o_dtype, int64_t B,
                               int64_t H, int Dk, int Dv, void* stream) {
    if (!q || !k || !v || !g || !strides || !state_in || !state_out || !o) return TRIUNE_ERR_NULL;
    if (!dtype_ok(io_dtype) || !dtype_ok(g_dtype) || !dtype_ok(o_dtype)) return TRIUNE_ERR_DTYPE;
    if (B < 0 || H <= 0 || n_state_rows < 0) return TRIUNE_ERR_SHAPE;
    if (!slots && n_state_rows < B) return TRIUNE_ERR_SHAPE;  // row b of the state for batch b
    if (!((Dk == 32 && Dv == 32) || (Dk == 64 && Dv == 64) || (Dk == 128 && Dv == 128) ||
          (Dk == 64 && Dv == 128) || (Dk == 128 && Dv == 64)))
        return TRIUNE_ERR_SHAPE;
    if (B > 0x7fffffff / H) return TRIUNE_ERR_SHAPE;  // rows (b, h) are indexed in 32 bits
    if (B == 0) return TRIUNE_OK;
    if (!vec_ok(q, io_dtype, strides + 0, 2) || !vec_ok(k, io_dtype, strides + 2, 2) ||
        !vec4_ok(v, io_dtype, strides + 4, 2) || !vec_ok(g, g_dtype, strides + 6, 2) ||
        !vec4_ok(o, o_dtype, strides + 8, 2) || reinterpret_cast<uintptr_t>(state_in) % 16 ||
        reinterpret_cast<uintptr_t>(state_out) % 16)
        return TRIUNE_ERR_LAYOUT;
    DecodeParams a{};
    a.q = q; a.k = k; a.v = v; a.g = g;
    a.io_dt = io_dtype; a.g_dt = g_dtype; a.o_dt = o_dtype;
    a.q_sb = strides[0]; a.q_sh = strides[1];
    a.k_sb = strides[2]; a.k_sh = strides[3];
    a.v_sb = strides[4]; a.v_sh = strides[5];
    a.g_sb = strides[6]; a.g_sh = strides[7];
    a.o_sb = strides[8]; a.o_sh = strides[9];
    a.state_in = state_in; a.state_out = state_out; a.slots = slots; a.n_state_rows = n_state_rows;
    a.o = o; a.B = B; a.H = H;
    return launch_status(launch_gla_decode(a, Dk, Dv, 4 * device_cus(), (hipStream_t)stream));
}

// ---- the reference's own native decode signatures, on device pointers -----------------------
static thread_local int g_last_error = TRIUNE_OK;

int triune_hip_last_error(void) { return g_last_error; }

// The twins' callers hand over pointers whose memory space the reference's own functions never had
// to ask about: its C step (engine.cpp:419-475) works on host memory, reached from
// triune/ops/_c_bridge.py:259-294 with CPU tensors only.  A GPU kernel given pageable host memory
// takes a memory fault (this pool runs without XNACK), so each twin first asks the runtime where
// every pointer lives and launches only when all of them are device memory of the current device.
// A failed query (an unknown pointer, or no device) leaves an error in the runtime's last-error
// slot; it is cleared here so that the caller's next HIP call does not report it.
}  // extern "C"

namespace {

bool on_current_device(std::initializer_list<const void*> ptrs) {
    const int dev = current_device();
    if (dev < 0) {
        (void)hipGetLastError();
        return false;
    }
    for (const void* p : ptrs) {
        if (!p) return false;
        hipPointerAttribute_t at{};
        if (hipPointerGetAttributes(&at, p) != hipSuccess) {
            (void)hipGetLastError();
            return false;
        }
        if (at.type != hipMemoryTypeDevice || at.device != dev) return false;
    }
    return true;
}

}  // namespace

extern "C" {

void launch_gla_decode_step(const void* Q, const void* K, const void* V, const float* G, float* State, void* Out,
                            int B, int H, int HD, void* stream) {
    if (!Q || !K || !V || !G || !State || !Out) {
        g_last_error = TRIUNE_ERR_NULL;
        return;
    }
    if (B < 0 || H <= 0 || (HD != 32 && HD != 64 && HD != 128)) {
        g_last_error = TRIUNE_ERR_SHAPE;
        return;
    }
    if (B > 0 && !on_current_device({Q, K, V, G, State, Out})) {
        g_last_error = TRIUNE_ERR_MEMORY;
        return;
    }
    const int64_t row = HD, bat = (int64_t)H * HD;  // contiguous [B, 1, H, HD]
    const int64_t st[10] = {bat, row, bat, row, bat, row, bat, row, bat, row};
    g_last_error = triune_hip_gla_decode_step(Q, K, V, G, TRIUNE_DT_BF16, TRIUNE_DT_F32, st, State, State, nullptr,
                                              B, Out, TRIUNE_DT_BF16, B, H, HD, HD, stream);
}

void triune_gla_recurrent_step_f32(const float* q, const float* k, const float* v, const float* g, float* state,
                                   float* out, int batch_heads, int head_dim) {
    if (!q || !k || !v || !g || !state || !out) {
        g_last_error = TRIUNE_ERR_NULL;
        return;
    }
    if (batch_heads < 0 || (head_dim != 32 && head_dim != 64 && head_dim != 128)) {
        g_last_error = TRIUNE_ERR_SHAPE;
        return;
    }
    if (batch_heads > 0 && !on_current_device({q, k, v, g, state, out})) {
        g_last_error = TRIUNE_ERR_MEMORY;
        return;
    }
    const int64_t row = head_dim;  // contiguous [batch_heads, head_dim] rows: one head per row
    const int64_t st[10] = {row, row, row, row, row, row, row, row, row, row};
    g_last_error = triune_hip_gla_decode_step(q, k, v, g, TRIUNE_DT_F32, TRIUNE_DT_F32, st, state, state, nullptr,
                                              batch_heads, out, TRIUNE_DT_F32, batch_heads, 1, head_dim, head_dim,
                                              nullptr);
}

size_t triune_hip_gla_prefill_workspace_size(int64_t B, int64_t T, int64_t H, int Dk, int Dv, int flags) {
    if (B <= 0 || T <= 0 || H <= 0 || !prefill_shape_ok(Dk, Dv)) return 0;
    return plan_dense(B, T, H, Dk, Dv, flags).total;
}

// extent: bytes from p to one past the last element of a [nb, nt, H, D] view (nb, nt >= 1).
static void fill_tok(TokTensor& t, const void* p, const int64_t* st3, int64_t nb, int64_t nt, int64_t H, int D,
                     int dt) {
    t.p = p; t.sb = st3[0]; t.st = st3[1]; t.sh = st3[2];
    const int64_t es = dt == TRIUNE_DT_F32 ? 4 : 2;
    t.extent = ((nb - 1) * t.sb + (nt - 1) * t.st + (H - 1) * t.sh + D) * es;
}

int triune_hip_gla_prefill(const void* q, const void* k, const void* v, const void* g, int io_dtype, int g_dtype,
                           const int64_t* strides, const float* s0, void* o, int o_dtype, float* s_final,
                           int64_t B, int64_t T, int64_t H, int Dk, int Dv, int flags, void* workspace,
                           size_t workspace_bytes, void* stream) {
    if (!q || !k || !v || !g || !o || !strides) return TRIUNE_ERR_NULL;
    if (!dtype_ok(io_dtype) || !dtype_ok(g_dtype) || !dtype_ok(o_dtype)) return TRIUNE_ERR_DTYPE;
    if (!gate_dtype_ok(io_dtype, g_dtype)) return TRIUNE_ERR_DTYPE;
    if (B < 0 || T < 0 || H <= 0 || !prefill_dtype_supported(Dk, Dv, io_dtype)) return TRIUNE_ERR_SHAPE;
    if (!vec_ok(q, io_dtype, strides + 0, 3) || !vec_ok(k, io_dtype, strides + 3, 3) ||
        !vec_ok(v, io_dtype, strides + 6, 3) || !vec_ok(g, g_dtype, strides + 9, 3) ||
        !vec_ok(o, o_dtype, strides + 12, 3) || reinterpret_cast<uintptr_t>(s0) % 16 ||
        reinterpret_cast<uintptr_t>(s_final) % 16 || !tok_strides_ok(strides, io_dtype, g_dtype, o_dtype, Dk, Dv))
        return TRIUNE_ERR_LAYOUT;
    hipStream_t st = (hipStream_t)stream;
    if (B == 0) return TRIUNE_OK;
    if (T == 0) {
        if (!s_final) return TRIUNE_OK;
        ScanParams sc{};  // N = 0: fin = init (or zero)
        sc.kv = s_final; sc.kv_dt = DT_F32; sc.dec = s_final; sc.dec_dt = DT_F32;
        sc.init = s0; sc.i_so = H * (int64_t)Dk * Dv; sc.i_sh = (int64_t)Dk * Dv;
        sc.fin = s_final; sc.fin_dt = DT_F32; sc.f_so = sc.i_so; sc.f_sh = sc.i_sh;
        sc.n_outer = B; sc.H = H; sc.Dk = Dk; sc.Dv = Dv; sc.N = 0;
        return launch_status(launch_recurrent_scan(sc, st));
    }
    const PrefillPlan pl = plan_dense(B, T, H, Dk, Dv, flags);
    if (!workspace || workspace_bytes < pl.total) return TRIUNE_ERR_WORKSPACE;
    char* ws = reinterpret_cast<char*>(workspace);
    if (reinterpret_cast<uintptr_t>(ws) % 16) return TRIUNE_ERR_LAYOUT;

    PrefillParams a{};
    fill_tok(a.q, q, strides + 0, B, T, H, Dk, io_dtype);
    fill_tok(a.k, k, strides + 3, B, T, H, Dk, io_dtype);
    fill_tok(a.v, v, strides + 6, B, T, H, Dv, io_dtype);
    fill_tok(a.g, g, strides + 9, B, T, H, Dk, g_dtype);
    a.o = o; a.o_sb = strides[12]; a.o_st = strides[13]; a.o_sh = strides[14];
    a.g_dt = g_dtype; a.o_dt = o_dtype;
    a.s0 = s0;
    a.ws_state = reinterpret_cast<float*>(ws + pl.off_state);
    a.ws_gamma = reinterpret_cast<float*>(ws + pl.off_gamma);
    a.n_seqs = B; a.H = H; a.T = T; a.Dk = Dk; a.Dv = Dv;
    a.P = pl.P; a.nseg_dense = (int)pl.nseg; a.varlen = 0; a.flags = flags & 0xff;
    return dense_launch(a, pl, s0, s_final, io_dtype, false, st);
}

}  // extern "C"

namespace {

// The dense launch sequence on a filled parameter block: segment states, the carry scan over the
// segments (initial and final states), outputs.  prep: the segment-state kernel first
// pre-processes q, k, g in place (the output kernel then reads the processed tensors).
int dense_launch(PrefillParams& a, const PrefillPlan& pl, const float* s0, float* s_final, int io_dtype, bool prep,
                 hipStream_t st) {
    const int64_t H = a.H, B = a.n_seqs;
    const int Dk = a.Dk, Dv = a.Dv;
    hipError_t e = prep ? launch_gla_prep_seg_state(a, pl.n_work, io_dtype, st)
                        : launch_gla_seg_state(a, pl.n_work, io_dtype, st);
    if (e != hipSuccess) return TRIUNE_ERR_LAUNCH;

    const int64_t DD = (int64_t)Dk * Dv;
    ScanParams sc{};
    sc.kv = a.ws_state; sc.kv_dt = DT_F32;
    sc.kv_so = pl.nseg * H * DD; sc.kv_sh = DD; sc.kv_sn = H * DD;
    sc.dec = a.ws_gamma; sc.dec_dt = DT_F32; sc.dec_is_log = 1;
    sc.d_so = pl.nseg * H * Dk; sc.d_sh = Dk; sc.d_sn = H * Dk;
    sc.init = s0; sc.i_so = H * DD; sc.i_sh = DD;
    sc.s_all = a.ws_state; sc.sa_dt = DT_F32;
    sc.sa_so = sc.kv_so; sc.sa_sh = sc.kv_sh; sc.sa_sn = sc.kv_sn;
    sc.fin = s_final; sc.fin_dt = DT_F32; sc.f_so = H * DD; sc.f_sh = DD;
    sc.n_outer = B; sc.H = H; sc.Dk = Dk; sc.Dv = Dv; sc.N = pl.nseg;
    e = launch_recurrent_scan(sc, st);
    if (e != hipSuccess) return TRIUNE_ERR_LAUNCH;

    return launch_output_timed(a, pl.n_work, io_dtype, st);
}

}  // namespace

extern "C" {

int triune_hip_gla_prefill_prep(const void* q, const void* k, const void* v, const void* g, int io_dtype,
                                const int64_t* strides, const float* cos, const float* sin, int64_t cs_stride,
                                int use_rope, const float* s0, void* o, int o_dtype, float* s_final, int64_t B,
                                int64_t T, int64_t H, int D, void* workspace, size_t workspace_bytes, void* stream) {
    if (!q || !k || !v || !g || !o || !strides || (use_rope && (!cos || !sin))) return TRIUNE_ERR_NULL;
    if (!dtype_ok(io_dtype) || !dtype_ok(o_dtype)) return TRIUNE_ERR_DTYPE;
    if (!prefill_prep_supported(D, io_dtype)) return io_dtype == TRIUNE_DT_F32 ? TRIUNE_ERR_DTYPE : TRIUNE_ERR_SHAPE;
    if (B < 0 || T < 0 || H <= 0) return TRIUNE_ERR_SHAPE;
    if (!vec_ok(q, io_dtype, strides + 0, 3) || !vec_ok(k, io_dtype, strides + 3, 3) ||
        !vec_ok(v, io_dtype, strides + 6, 3) || !vec_ok(g, io_dtype, strides + 9, 3) ||
        !vec_ok(o, o_dtype, strides + 12, 3) || reinterpret_cast<uintptr_t>(s0) % 16 ||
        reinterpret_cast<uintptr_t>(s_final) % 16 || !tok_strides_ok(strides, io_dtype, io_dtype, o_dtype, D, D))
        return TRIUNE_ERR_LAYOUT;
    if (use_rope && (!vec_ok(cos, TRIUNE_DT_F32, &cs_stride, 1) || !vec_ok(sin, TRIUNE_DT_F32, &cs_stride, 1) ||
                     cs_stride < D || (64 * cs_stride + D) * 4 >= ((int64_t)1 << 31)))
        return TRIUNE_ERR_LAYOUT;
    hipStream_t st = (hipStream_t)stream;
    if (B == 0) return TRIUNE_OK;
    if (T == 0) {
        if (!s_final) return TRIUNE_OK;
        ScanParams sc{};  // N = 0: fin = init (or zero)
        sc.kv = s_final; sc.kv_dt = DT_F32; sc.dec = s_final; sc.dec_dt = DT_F32;
        sc.init = s0; sc.i_so = H * (int64_t)D * D; sc.i_sh = (int64_t)D * D;
        sc.fin = s_final; sc.fin_dt = DT_F32; sc.f_so = sc.i_so; sc.f_sh = sc.i_sh;
        sc.n_outer = B; sc.H = H; sc.Dk = D; sc.Dv = D; sc.N = 0;
        return launch_status(launch_recurrent_scan(sc, st));
    }
    const PrefillPlan pl = plan_dense(B, T, H, D, D, 0);
    if (!workspace || workspace_bytes < pl.total) return TRIUNE_ERR_WORKSPACE;
    char* ws = reinterpret_cast<char*>(workspace);
    if (reinterpret_cast<uintptr_t>(ws) % 16) return TRIUNE_ERR_LAYOUT;

    PrefillParams a{};
    fill_tok(a.q, q, strides + 0, B, T, H, D, io_dtype);
    fill_tok(a.k, k, strides + 3, B, T, H, D, io_dtype);
    fill_tok(a.v, v, strides + 6, B, T, H, D, io_dtype);
    fill_tok(a.g, g, strides + 9, B, T, H, D, io_dtype);
    a.o = o; a.o_sb = strides[12]; a.o_st = strides[13]; a.o_sh = strides[14];
    a.g_dt = io_dtype; a.o_dt = o_dtype;
    a.s0 = s0;
    a.ws_state = reinterpret_cast<float*>(ws + pl.off_state);
    a.ws_gamma = reinterpret_cast<float*>(ws + pl.off_gamma);
    a.n_seqs = B; a.H = H; a.T = T; a.Dk = D; a.Dv = D;
    a.P = pl.P; a.nseg_dense = (int)pl.nseg; a.varlen = 0; a.flags = 0;
    a.use_rope = use_rope ? 1 : 0;
    if (use_rope) {  // [T, D] tables shared by every sequence and head (batch and head strides 0)
        const int64_t cst[3] = {0, cs_stride, 0};
        fill_tok(a.cs, cos, cst, 1, T, 1, D, TRIUNE_DT_F32);
        fill_tok(a.sn, sin, cst, 1, T, 1, D, TRIUNE_DT_F32);
    }
    return dense_launch(a, pl, s0, s_final, io_dtype, true, st);
}

}  // extern "C"

namespace {

// Single-launch prefill plan: one workgroup per two 64-token chunks; each XCD runs the chunk pairs
// of ceil(B * H / 8) (sequence, head) pairs, which must all be resident at once on its CUs (a
// workgroup waits for the earlier chunk pairs of its (sequence, head)).  The fold reads every
// earlier pair's map, so pairs per sequence stay at most gla_onepass_max_pairs() (32).
constexpr size_t kOnePassHdrBytes = 64;

int64_t onepass_pairs(int64_t T) { return ((T + 63) / 64 + 1) / 2; }

int onepass_slots_per_xcd() {
    static std::atomic<int> cache[kMaxDevices];
    const int dev = current_device();
    if (dev >= 0) {
        const int c = cache[dev].load(std::memory_order_relaxed);
        if (c > 0) return c;
    }
    const int slots = device_cus() / 8 * gla_onepass_blocks_per_cu();
    if (dev >= 0 && slots > 0) cache[dev].store(slots, std::memory_order_relaxed);
    return slots;
}

bool onepass_fits(int64_t B, int64_t T, int64_t H, int D) {
    if (B <= 0 || T <= 0 || H <= 0 || D != 64) return false;
    const int64_t np = onepass_pairs(T), bh = B * H;
    if (np > gla_onepass_max_pairs() || bh > 0x7fffffff / np) return false;
    return (bh + 7) / 8 * np <= onepass_slots_per_xcd();
}

size_t onepass_ws_bytes(int64_t B, int64_t T, int64_t H, int D) {
    const int64_t n = B * H * onepass_pairs(T);
    return align_up((size_t)n * D * D * sizeof(float)) + align_up((size_t)n * D * sizeof(float));
}

size_t onepass_ctrl_bytes(int64_t B, int64_t T, int64_t H) {
    return kOnePassHdrBytes + align_up((size_t)(B * H * onepass_pairs(T)) * sizeof(uint64_t));
}

}  // namespace

extern "C" {

int triune_hip_gla_prefill_onepass_supported(int64_t B, int64_t T, int64_t H, int D, int io_dtype, int g_dtype,
                                             int prep, int flags) {
    if (!gla_onepass_dtypes_ok(io_dtype, g_dtype, prep != 0)) return 0;
    if ((flags & ~TRIUNE_FLAG_TAIL_UNCLAMPED) != 0 || (prep && flags != 0)) return 0;
    return onepass_fits(B, T, H, D) ? 1 : 0;
}

size_t triune_hip_gla_prefill_onepass_workspace_size(int64_t B, int64_t T, int64_t H, int D) {
    if (B <= 0 || T <= 0 || H <= 0 || D != 64) return 0;
    return onepass_ws_bytes(B, T, H, D);
}

size_t triune_hip_gla_prefill_onepass_ctrl_size(int64_t B, int64_t T, int64_t H, int D) {
    if (B <= 0 || T <= 0 || H <= 0 || D != 64) return 0;
    return onepass_ctrl_bytes(B, T, H);
}

int triune_hip_gla_prefill_onepass(const void* q, const void* k, const void* v, const void* g, int io_dtype,
                                   int g_dtype, const int64_t* strides, const float* cos, const float* sin,
                                   int64_t cs_stride, int prep, int use_rope, const float* s0, void* o, int o_dtype,
                                   float* s_final, int64_t B, int64_t T, int64_t H, int D, int flags, void* workspace,
                                   size_t workspace_bytes, void* ctrl, size_t ctrl_bytes, void* stream) {
    if (!q || !k || !v || !g || !o || !strides || (prep && use_rope && (!cos || !sin))) return TRIUNE_ERR_NULL;
    if (!dtype_ok(io_dtype) || !dtype_ok(g_dtype) || !dtype_ok(o_dtype)) return TRIUNE_ERR_DTYPE;
    if (!gla_onepass_dtypes_ok(io_dtype, g_dtype, prep != 0)) return TRIUNE_ERR_DTYPE;
    if (B < 0 || T < 0 || H <= 0 || D != 64) return TRIUNE_ERR_SHAPE;
    if ((flags & ~TRIUNE_FLAG_TAIL_UNCLAMPED) != 0 || (prep && flags != 0)) return TRIUNE_ERR_SHAPE;
    if (!vec_ok(q, io_dtype, strides + 0, 3) || !vec_ok(k, io_dtype, strides + 3, 3) ||
        !vec_ok(v, io_dtype, strides + 6, 3) || !vec_ok(g, g_dtype, strides + 9, 3) ||
        !vec_ok(o, o_dtype, strides + 12, 3) || reinterpret_cast<uintptr_t>(s0) % 16 ||
        reinterpret_cast<uintptr_t>(s_final) % 16 || !tok_strides_ok(strides, io_dtype, g_dtype, o_dtype, D, D))
        return TRIUNE_ERR_LAYOUT;
    if (prep && use_rope &&
        (!vec_ok(cos, TRIUNE_DT_F32, &cs_stride, 1) || !vec_ok(sin, TRIUNE_DT_F32, &cs_stride, 1) || cs_stride < D ||
         (64 * cs_stride + D) * 4 >= ((int64_t)1 << 31)))
        return TRIUNE_ERR_LAYOUT;
    if (B == 0 || T == 0) return TRIUNE_ERR_SHAPE;  // nothing for a chunk kernel: the caller's other paths
    if (!onepass_fits(B, T, H, D)) return TRIUNE_ERR_SHAPE;
    if (!workspace || workspace_bytes < onepass_ws_bytes(B, T, H, D)) return TRIUNE_ERR_WORKSPACE;
    if (!ctrl || ctrl_bytes < onepass_ctrl_bytes(B, T, H)) return TRIUNE_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(workspace) % 16 || reinterpret_cast<uintptr_t>(ctrl) % 16)
        return TRIUNE_ERR_LAYOUT;
    const int64_t nch = (T + 63) / 64, npair = onepass_pairs(T), n = B * H * npair;
    char* ws = reinterpret_cast<char*>(workspace);
    PrefillParams a{};
    fill_tok(a.q, q, strides + 0, B, T, H, D, io_dtype);
    fill_tok(a.k, k, strides + 3, B, T, H, D, io_dtype);
    fill_tok(a.v, v, strides + 6, B, T, H, D, io_dtype);
    fill_tok(a.g, g, strides + 9, B, T, H, D, g_dtype);
    a.o = o; a.o_sb = strides[12]; a.o_st = strides[13]; a.o_sh = strides[14];
    a.g_dt = g_dtype; a.o_dt = o_dtype;
    a.s0 = s0;
    a.seq_final = s_final;
    a.ws_state = reinterpret_cast<float*>(ws);
    a.ws_gamma = reinterpret_cast<float*>(ws + align_up((size_t)n * D * D * sizeof(float)));
    a.n_seqs = B; a.H = H; a.T = T; a.Dk = D; a.Dv = D;
    a.P = 1; a.nseg_dense = (int)nch; a.varlen = 0; a.flags = flags & TRIUNE_FLAG_TAIL_UNCLAMPED;
    a.use_rope = prep && use_rope ? 1 : 0;
    if (a.use_rope) {  // [T, D] tables shared by every sequence and head (batch and head strides 0)
        const int64_t cst[3] = {0, cs_stride, 0};
        fill_tok(a.cs, cos, cst, 1, T, 1, D, TRIUNE_DT_F32);
        fill_tok(a.sn, sin, cst, 1, T, 1, D, TRIUNE_DT_F32);
    }
    OnePassCtl c{};
    c.hdr = reinterpret_cast<uint32_t*>(ctrl);
    c.flags = reinterpret_cast<uint64_t*>(reinterpret_cast<char*>(ctrl) + kOnePassHdrBytes);
    c.nch = nch;
    c.npair = npair;
    c.nh8 = (B * H + 7) / 8;
    const OutputEvents ev = g_output_events;  // the measurement hook: the one kernel's start and end
    return launch_status(launch_gla_onepass(a, c, io_dtype, prep != 0, (hipStream_t)stream, ev.begin, ev.end));
}

}  // extern "C"

namespace {

// Allocation-free prefill: the workspace of triune_hip_gla_prefill lives in this file-scope
// device array instead of a caller buffer.  Each GPU holds its own copy until the process ends;
// host code must use the address hipGetSymbolAddress returns for the current device (the
// array's name is a host-side stand-in), fetched once per device on its first call.
constexpr size_t kScratchBytes = (size_t)TRIUNE_GLA_PREFILL_SCRATCH_BYTES;
static __device__ __align__(256) char scratch[kScratchBytes];

// The scratch address on the current device (which must own `stream`), or nullptr.
void* scratch_for(void* stream) {
    static std::atomic<void*> ptrs[kMaxDevices];
    const int dev = current_device();
    if (dev < 0) return nullptr;
    if (stream) {
        hipDevice_t sdev = -1;
        if (hipStreamGetDevice((hipStream_t)stream, &sdev) != hipSuccess || sdev != dev) return nullptr;
    }
    void* p = ptrs[dev].load(std::memory_order_acquire);
    if (p) return p;
    void* q = nullptr;
    if (hipGetSymbolAddress(&q, HIP_SYMBOL(scratch)) != hipSuccess || !q) return nullptr;
    ptrs[dev].store(q, std::memory_order_release);
    return q;
}

}  // namespace

extern "C" {

size_t triune_hip_gla_prefill_noalloc_max_bytes(void) { return kScratchBytes; }

int triune_hip_gla_prefill_noalloc(const void* q, const void* k, const void* v, const void* g, int io_dtype,
                                   int g_dtype, const int64_t* strides, const float* s0, void* o, int o_dtype,
                                   float* s_final, int64_t B, int64_t T, int64_t H, int Dk, int Dv, int flags,
                                   void* stream) {
    // the checks that need no workspace run first, with the same codes as the allocating entry
    if (!q || !k || !v || !g || !o || !strides) return TRIUNE_ERR_NULL;
    if (B < 0 || T < 0 || H <= 0 || !prefill_shape_ok(Dk, Dv)) return TRIUNE_ERR_SHAPE;
    size_t need = 0;
    if (B > 0 && T > 0) {
        need = plan_dense(B, T, H, Dk, Dv, flags).total;
        if (need > kScratchBytes) return TRIUNE_ERR_SCRATCH;
    }
    void* ws = need ? scratch_for(stream) : nullptr;
    if (need && !ws) return TRIUNE_ERR_LAUNCH;
    return triune_hip_gla_prefill(q, k, v, g, io_dtype, g_dtype, strides, s0, o, o_dtype, s_final, B, T, H, Dk, Dv,
                                  flags, ws, need ? kScratchBytes : 0, stream);
}

size_t triune_hip_gla_prefill_bwd_workspace_size(int64_t B, int64_t T, int64_t H, int Dk, int Dv, int flags) {
    if (B <= 0 || T <= 0 || H <= 0 || Dk != Dv || !gla_bwd_supported(Dk, TRIUNE_DT_BF16)) return 0;
    return plan_bwd(B, T, H, Dk, flags).total;
}

int triune_hip_gla_prefill_bwd(const void* q, const void* k, const void* v, const void* g, int io_dtype, int g_dtype,
                               const void* dout, const int64_t* strides, const float* s0, const float* ds_final,
                               void* dq, void* dk, void* dv, int d_dtype, void* dg, int dg_dtype, float* ds0,
                               int64_t B, int64_t T, int64_t H, int Dk, int Dv, int flags, void* workspace,
                               size_t workspace_bytes, void* stream) {
    if (!q || !k || !v || !g || !dout || !strides || !dq || !dk || !dv || !dg) return TRIUNE_ERR_NULL;
    if (!dtype_ok(io_dtype) || !dtype_ok(g_dtype) || !dtype_ok(d_dtype) || !dtype_ok(dg_dtype)) return TRIUNE_ERR_DTYPE;
    if (!gate_dtype_ok(io_dtype, g_dtype)) return TRIUNE_ERR_DTYPE;
    if ((flags & TRIUNE_FLAG_BWD_ACC_QKG) && (d_dtype != TRIUNE_DT_F32 || dg_dtype != TRIUNE_DT_F32))
        return TRIUNE_ERR_DTYPE;
    if ((flags & TRIUNE_FLAG_BWD_ACC_V) && d_dtype != TRIUNE_DT_F32) return TRIUNE_ERR_DTYPE;
    if (B < 0 || T < 0 || H <= 0 || Dk != Dv || !gla_bwd_supported(Dk, io_dtype)) return TRIUNE_ERR_SHAPE;
    const int64_t* st = strides;  // q, k, v, g, dout, dq, dk, dv, dg: (batch, token, head) each
    auto rows_ok = [&](int i, int dt, int D) {  // as tok_strides_ok: rows at least D apart
        const int64_t es = dt == TRIUNE_DT_F32 ? 4 : 2;
        return st[3 * i + 1] >= D && (64 * st[3 * i + 1] + D) * es < ((int64_t)1 << 31);
    };
    if (!vec_ok(q, io_dtype, st + 0, 3) || !vec_ok(k, io_dtype, st + 3, 3) || !vec_ok(v, io_dtype, st + 6, 3) ||
        !vec_ok(g, g_dtype, st + 9, 3) || !vec_ok(dout, io_dtype, st + 12, 3) || !vec4_ok(dq, d_dtype, st + 15, 3) ||
        !vec4_ok(dk, d_dtype, st + 18, 3) || !vec4_ok(dv, d_dtype, st + 21, 3) || !vec4_ok(dg, dg_dtype, st + 24, 3) ||
        reinterpret_cast<uintptr_t>(s0) % 16 || reinterpret_cast<uintptr_t>(ds_final) % 16 ||
        reinterpret_cast<uintptr_t>(ds0) % 16)
        return TRIUNE_ERR_LAYOUT;
    if (!rows_ok(0, io_dtype, Dk) || !rows_ok(1, io_dtype, Dk) || !rows_ok(2, io_dtype, Dv) || !rows_ok(3, g_dtype, Dk) ||
        !rows_ok(4, io_dtype, Dv) || !rows_ok(5, d_dtype, Dk) || !rows_ok(6, d_dtype, Dk) || !rows_ok(7, d_dtype, Dv) ||
        !rows_ok(8, dg_dtype, Dk))
        return TRIUNE_ERR_LAYOUT;
    hipStream_t hs = (hipStream_t)stream;
    const int64_t D = Dk, DD = (int64_t)Dk * Dv;
    if (B == 0) return TRIUNE_OK;
    if (T == 0) {  // dS0 = dS_final (or zero)
        if (!ds0) return TRIUNE_OK;
        ScanParams sc{};
        sc.kv = ds0; sc.kv_dt = DT_F32; sc.dec = ds0; sc.dec_dt = DT_F32;
        sc.init = ds_final; sc.i_so = H * DD; sc.i_sh = DD;
        sc.fin = ds0; sc.fin_dt = DT_F32; sc.f_so = sc.i_so; sc.f_sh = sc.i_sh;
        sc.n_outer = B; sc.H = H; sc.Dk = Dk; sc.Dv = Dv; sc.N = 0;
        return launch_status(launch_recurrent_scan(sc, hs));
    }
    const BwdPlan pl = plan_bwd(B, T, H, Dk, flags);
    if (!workspace || workspace_bytes < pl.total) return TRIUNE_ERR_WORKSPACE;
    char* ws = reinterpret_cast<char*>(workspace);
    if (reinterpret_cast<uintptr_t>(ws) % 16) return TRIUNE_ERR_LAYOUT;

    BwdParams a{};
    PrefillParams& f = a.f;
    fill_tok(f.q, q, st + 0, B, T, H, Dk, io_dtype);
    fill_tok(f.k, k, st + 3, B, T, H, Dk, io_dtype);
    fill_tok(f.v, v, st + 6, B, T, H, Dv, io_dtype);
    fill_tok(f.g, g, st + 9, B, T, H, Dk, g_dtype);
    f.g_dt = g_dtype; f.o_dt = d_dtype;
    f.s0 = s0;
    f.ws_state = reinterpret_cast<float*>(ws + pl.f.off_state);
    f.ws_gamma = reinterpret_cast<float*>(ws + pl.f.off_gamma);
    f.n_seqs = B; f.H = H; f.T = T; f.Dk = Dk; f.Dv = Dv;
    f.P = pl.f.P; f.nseg_dense = (int)pl.f.nseg; f.varlen = 0; f.flags = flags & TRIUNE_FLAG_TAIL_UNCLAMPED;
    fill_tok(a.dout, dout, st + 12, B, T, H, Dv, io_dtype);
    a.dq = dq; a.dq_sb = st[15]; a.dq_st = st[16]; a.dq_sh = st[17];
    a.dk = dk; a.dk_sb = st[18]; a.dk_st = st[19]; a.dk_sh = st[20];
    a.dv = dv; a.dv_sb = st[21]; a.dv_st = st[22]; a.dv_sh = st[23];
    a.dg = dg; a.dg_sb = st[24]; a.dg_st = st[25]; a.dg_sh = st[26];
    a.d_dt = d_dtype; a.dg_dt = dg_dtype;
    a.acc = ((flags & TRIUNE_FLAG_BWD_ACC_QKG) ? 1 : 0) | ((flags & TRIUNE_FLAG_BWD_ACC_V) ? 2 : 0);
    a.ws_r = reinterpret_cast<float*>(ws + pl.off_r);
    a.ws_send = reinterpret_cast<float*>(ws + pl.off_send);
    a.ws_chunk = reinterpret_cast<float*>(ws + pl.off_chunk);
    a.nchunks = pl.nchunks;
    const int64_t nseg = pl.f.nseg;

    // forward: segment-local states, then the carried-in state of every segment
    if (launch_gla_seg_state(f, pl.f.n_work, io_dtype, hs) != hipSuccess) return TRIUNE_ERR_LAUNCH;
    ScanParams sc{};
    sc.kv = f.ws_state; sc.kv_dt = DT_F32;
    sc.kv_so = nseg * H * DD; sc.kv_sh = DD; sc.kv_sn = H * DD;
    sc.dec = f.ws_gamma; sc.dec_dt = DT_F32; sc.dec_is_log = 1;
    sc.d_so = nseg * H * D; sc.d_sh = D; sc.d_sn = H * D;
    sc.init = s0; sc.i_so = H * DD; sc.i_sh = DD;
    sc.s_all = f.ws_state; sc.sa_dt = DT_F32; sc.sa_so = sc.kv_so; sc.sa_sh = sc.kv_sh; sc.sa_sn = sc.kv_sn;
    sc.fin = nullptr; sc.fin_dt = DT_F32;
    sc.n_outer = B; sc.H = H; sc.Dk = Dk; sc.Dv = Dv; sc.N = nseg;
    if (launch_recurrent_scan(sc, hs) != hipSuccess) return TRIUNE_ERR_LAUNCH;
    // chunk starting states, segment end states, segment maps R
    if (launch_gla_bwd_state(a, pl.f.n_work, io_dtype, hs) != hipSuccess) return TRIUNE_ERR_LAUNCH;
    // the same scan over the segments in reverse order: the gradient reaching each segment's end
    // (in place of R, starting from dS_final) and dS0
    ScanParams rv{};
    rv.kv = a.ws_r + (nseg - 1) * H * DD; rv.kv_dt = DT_F32;
    rv.kv_so = nseg * H * DD; rv.kv_sh = DD; rv.kv_sn = -H * DD;
    rv.dec = f.ws_gamma + (nseg - 1) * H * D; rv.dec_dt = DT_F32; rv.dec_is_log = 1;
    rv.d_so = nseg * H * D; rv.d_sh = D; rv.d_sn = -H * D;
    rv.init = ds_final; rv.i_so = H * DD; rv.i_sh = DD;
    rv.s_all = a.ws_r + (nseg - 1) * H * DD; rv.sa_dt = DT_F32; rv.sa_so = rv.kv_so; rv.sa_sh = rv.kv_sh; rv.sa_sn = rv.kv_sn;
    rv.fin = ds0; rv.fin_dt = DT_F32; rv.f_so = H * DD; rv.f_sh = DD;
    rv.n_outer = B; rv.H = H; rv.Dk = Dk; rv.Dv = Dv; rv.N = nseg;
    if (launch_recurrent_scan(rv, hs) != hipSuccess) return TRIUNE_ERR_LAUNCH;
    return launch_status(launch_gla_bwd_chunk(a, pl.f.n_work, io_dtype, hs));
}

size_t triune_hip_gla_prefill_varlen_workspace_size(int64_t n_seqs, int64_t total_tokens, int64_t H, int Dk,
                                                    int Dv, int flags) {
    if (n_seqs <= 0 || total_tokens < 0 || H <= 0 || !prefill_shape_ok(Dk, Dv)) return 0;
    return plan_varlen(n_seqs, total_tokens, H, Dk, Dv, flags).total;
}

// Packed ragged prefill; with `slots`, sequence i's initial and final states are row slots[i] of
// s0 / s_final (which may be one pool updated in place).
static int varlen_impl(const void* q, const void* k, const void* v, const void* g, int io_dtype, int g_dtype,
                       const int64_t* strides, const int32_t* cu_seqlens, int64_t n_seqs, int64_t total_tokens,
                       const float* s0, void* o, int o_dtype, float* s_final, const int32_t* slots, int64_t n_slots,
                       int64_t H, int Dk, int Dv, int flags, void* workspace, size_t workspace_bytes, void* stream) {
    if (!q || !k || !v || !g || !o || !strides || !cu_seqlens) return TRIUNE_ERR_NULL;
    if (!dtype_ok(io_dtype) || !dtype_ok(g_dtype) || !dtype_ok(o_dtype)) return TRIUNE_ERR_DTYPE;
    if (!gate_dtype_ok(io_dtype, g_dtype)) return TRIUNE_ERR_DTYPE;
    if (n_seqs <= 0 || total_tokens < 0 || H <= 0 || !prefill_dtype_supported(Dk, Dv, io_dtype))
        return TRIUNE_ERR_SHAPE;
    // (token, head) strides; the batch stride is unused (single packed batch)
    const int64_t st3[15] = {0, strides[0], strides[1], 0, strides[2], strides[3], 0, strides[4], strides[5],
                             0, strides[6], strides[7], 0, strides[8], strides[9]};
    if (!vec_ok(q, io_dtype, st3 + 1, 2) || !vec_ok(k, io_dtype, st3 + 4, 2) || !vec_ok(v, io_dtype, st3 + 7, 2) ||
        !vec_ok(g, g_dtype, st3 + 10, 2) || !vec_ok(o, o_dtype, st3 + 13, 2) ||
        reinterpret_cast<uintptr_t>(s0) % 16 || reinterpret_cast<uintptr_t>(s_final) % 16 ||
        !tok_strides_ok(st3, io_dtype, g_dtype, o_dtype, Dk, Dv))
        return TRIUNE_ERR_LAYOUT;
    const PrefillPlan pl = plan_varlen(n_seqs, total_tokens, H, Dk, Dv, flags);
    if (!workspace || workspace_bytes < pl.total) return TRIUNE_ERR_WORKSPACE;
    char* ws = reinterpret_cast<char*>(workspace);
    if (reinterpret_cast<uintptr_t>(ws) % 16) return TRIUNE_ERR_LAYOUT;
    hipStream_t st = (hipStream_t)stream;

    PrefillParams a{};
    const int64_t nt = total_tokens > 0 ? total_tokens : 1;
    fill_tok(a.q, q, st3 + 0, 1, nt, H, Dk, io_dtype);
    fill_tok(a.k, k, st3 + 3, 1, nt, H, Dk, io_dtype);
    fill_tok(a.v, v, st3 + 6, 1, nt, H, Dv, io_dtype);
    fill_tok(a.g, g, st3 + 9, 1, nt, H, Dk, g_dtype);
    a.o = o; a.o_sb = 0; a.o_st = st3[13]; a.o_sh = st3[14];
    a.g_dt = g_dtype; a.o_dt = o_dtype;
    a.s0 = s0;
    int32_t* seg_off = reinterpret_cast<int32_t*>(ws + pl.off_segoff);
    a.ws_state = reinterpret_cast<float*>(ws + pl.off_state);
    a.ws_gamma = reinterpret_cast<float*>(ws + pl.off_gamma);
    a.n_seqs = n_seqs; a.H = H; a.T = 0; a.Dk = Dk; a.Dv = Dv;
    a.P = pl.P; a.nseg_dense = 1; a.varlen = 1; a.cu = cu_seqlens; a.seg_off = seg_off;
    a.flags = flags & 0xff & ~TRIUNE_FLAG_TAIL_UNCLAMPED;

    hipError_t e = launch_gla_varlen_plan(cu_seqlens, n_seqs, pl.P, seg_off, st);
    if (e != hipSuccess) return TRIUNE_ERR_LAUNCH;
    if (pl.n_work > 0) {
        e = launch_gla_seg_state(a, pl.n_work, io_dtype, st);
        if (e != hipSuccess) return TRIUNE_ERR_LAUNCH;
    }
    const int64_t DD = (int64_t)Dk * Dv;
    ScanParams sc{};
    sc.kv = a.ws_state; sc.kv_dt = DT_F32;
    sc.kv_so = 0; sc.kv_sh = DD; sc.kv_sn = H * DD;
    sc.dec = a.ws_gamma; sc.dec_dt = DT_F32; sc.dec_is_log = 1;
    sc.d_so = 0; sc.d_sh = Dk; sc.d_sn = H * Dk;
    sc.init = s0; sc.i_so = H * DD; sc.i_sh = DD;
    sc.s_all = a.ws_state; sc.sa_dt = DT_F32;
    sc.sa_so = 0; sc.sa_sh = DD; sc.sa_sn = H * DD;
    sc.fin = s_final; sc.fin_dt = DT_F32; sc.f_so = H * DD; sc.f_sh = DD;
    sc.n_outer = n_seqs; sc.H = H; sc.Dk = Dk; sc.Dv = Dv; sc.seg_off = seg_off;
    sc.slots = slots; sc.n_slots = n_slots;
    e = launch_recurrent_scan(sc, st);
    if (e != hipSuccess) return TRIUNE_ERR_LAUNCH;
    if (pl.n_work > 0) return launch_output_timed(a, pl.n_work, io_dtype, st);
    return TRIUNE_OK;
}

int triune_hip_gla_prefill_varlen(const void* q, const void* k, const void* v, const void* g, int io_dtype,
                                  int g_dtype, const int64_t* strides, const int32_t* cu_seqlens, int64_t n_seqs,
                                  int64_t total_tokens, const float* s0, void* o, int o_dtype, float* s_final,
                                  int64_t H, int Dk, int Dv, int flags, void* workspace, size_t workspace_bytes,
                                  void* stream) {
    return varlen_impl(q, k, v, g, io_dtype, g_dtype, strides, cu_seqlens, n_seqs, total_tokens, s0, o, o_dtype,
                       s_final, nullptr, 0, H, Dk, Dv, flags, workspace, workspace_bytes, stream);
}

int triune_hip_gla_prefill_varlen_pool(const void* q, const void* k, const void* v, const void* g, int io_dtype,
                                       int g_dtype, const int64_t* strides, const int32_t* cu_seqlens,
                                       int64_t n_seqs, int64_t total_tokens, const int32_t* slots, float* pool,
                                       int64_t n_slots, void* o, int o_dtype, int64_t H, int Dk, int Dv, int flags,
                                       void* workspace, size_t workspace_bytes, void* stream) {
    if (!slots || !pool) return TRIUNE_ERR_NULL;
    if (n_slots <= 0) return TRIUNE_ERR_SHAPE;
    return varlen_impl(q, k, v, g, io_dtype, g_dtype, strides, cu_seqlens, n_seqs, total_tokens, pool, o, o_dtype,
                       pool, slots, n_slots, H, Dk, Dv, flags, workspace, workspace_bytes, stream);
}

int triune_hip_recurrent_scan_fwd(const void* kv, int kv_dtype, const void* decay, int decay_dtype, const void* init,
                                  int init_dtype, void* s_all, void* fin, int out_dtype, int64_t B, int64_t H,
                                  int64_t N, int Dk, int Dv, void* stream) {
    if (!kv || !decay || !s_all || !fin) return TRIUNE_ERR_NULL;
    if (!dtype_ok(kv_dtype) || !dtype_ok(decay_dtype) || !dtype_ok(out_dtype) || (init && !dtype_ok(init_dtype)))
        return TRIUNE_ERR_DTYPE;
    if (B < 0 || H < 0 || N < 0 || Dk <= 0 || Dv <= 0 || Dv % 4 != 0) return TRIUNE_ERR_SHAPE;
    auto al = [](int dt) -> uintptr_t { return dt == TRIUNE_DT_F32 ? 16 : 8; };
    if (reinterpret_cast<uintptr_t>(kv) % al(kv_dtype) || reinterpret_cast<uintptr_t>(s_all) % al(out_dtype) ||
        reinterpret_cast<uintptr_t>(fin) % al(out_dtype) || (init && reinterpret_cast<uintptr_t>(init) % al(init_dtype)))
        return TRIUNE_ERR_LAYOUT;
    if (B == 0 || H == 0) return TRIUNE_OK;
    const int64_t DD = (int64_t)Dk * Dv;
    ScanParams sc{};
    sc.kv = kv; sc.kv_dt = kv_dtype;
    sc.kv_so = H * N * DD; sc.kv_sh = N * DD; sc.kv_sn = DD;
    sc.dec = decay; sc.dec_dt = decay_dtype; sc.dec_is_log = 0;
    sc.d_so = H * N * Dk; sc.d_sh = N * Dk; sc.d_sn = Dk;
    sc.init = nullptr; sc.init_any = init; sc.init_dt = init_dtype; sc.i_so = H * DD; sc.i_sh = DD;
    sc.s_all = s_all; sc.sa_dt = out_dtype; sc.sa_so = sc.kv_so; sc.sa_sh = sc.kv_sh; sc.sa_sn = sc.kv_sn;
    sc.fin = fin; sc.fin_dt = out_dtype; sc.f_so = H * DD; sc.f_sh = DD;
    sc.n_outer = B; sc.H = H; sc.Dk = Dk; sc.Dv = Dv; sc.N = N;
    return launch_status(launch_recurrent_scan(sc, (hipStream_t)stream));
}

int triune_hip_recurrent_scan_bwd(const void* d_s_all, int d_s_all_dtype, const void* d_fin, int d_fin_dtype,
                                  const void* decay, int decay_dtype, const float* s_all, void* d_kv, void* d_decay,
                                  void* d_init, int out_dtype, int64_t B, int64_t H, int64_t N, int Dk, int Dv,
                                  void* stream) {
    if (!decay || !d_kv || !d_decay || !d_init || (N > 0 && !s_all)) return TRIUNE_ERR_NULL;
    if (!dtype_ok(decay_dtype) || !dtype_ok(out_dtype) || (d_s_all && !dtype_ok(d_s_all_dtype)) ||
        (d_fin && !dtype_ok(d_fin_dtype)))
        return TRIUNE_ERR_DTYPE;
    if (B < 0 || H < 0 || N < 0 || Dk <= 0 || Dv <= 0 || Dv % 4 != 0 || Dv > 256) return TRIUNE_ERR_SHAPE;
    auto al = [](int dt) -> uintptr_t { return dt == TRIUNE_DT_F32 ? 16 : 8; };
    auto mis = [](const void* p, uintptr_t m) { return reinterpret_cast<uintptr_t>(p) % m != 0; };
    if ((d_s_all && mis(d_s_all, al(d_s_all_dtype))) || (d_fin && mis(d_fin, al(d_fin_dtype))) || mis(s_all, 16) ||
        mis(d_kv, al(out_dtype)) || mis(d_init, al(out_dtype)))
        return TRIUNE_ERR_LAYOUT;
    if (B == 0 || H == 0) return TRIUNE_OK;
    ScanBwdParams a{};
    a.d_s_all = d_s_all; a.dsa_dt = d_s_all_dtype;
    a.d_fin = d_fin; a.df_dt = d_fin_dtype;
    a.dec = decay; a.dec_dt = decay_dtype;
    a.s_all = s_all; a.d_kv = d_kv; a.d_dec = d_decay; a.d_init = d_init; a.out_dt = out_dtype;
    a.n_outer = B; a.H = H; a.N = N; a.Dk = Dk; a.Dv = Dv;
    return launch_status(launch_recurrent_scan_bwd(a, (hipStream_t)stream));
}

int triune_hip_gdn_prefill(const void* q, const void* k, const void* v, const void* g, int io_dtype, int g_dtype,
                           const void* beta, int beta_dtype, int beta_kind, const int64_t* strides, const float* s0,
                           void* o, int o_dtype, float* s_final, int64_t B, int64_t T, int64_t H, int Dk, int Dv,
                           void* stream) {
    if (!q || !k || !v || !g || !o || !strides) return TRIUNE_ERR_NULL;
    if (beta_kind < TRIUNE_BETA_NONE || beta_kind > TRIUNE_BETA_VALUE) return TRIUNE_ERR_SHAPE;
    if (beta_kind != TRIUNE_BETA_NONE && !beta) return TRIUNE_ERR_NULL;
    if (!dtype_ok(io_dtype) || !dtype_ok(g_dtype) || !dtype_ok(o_dtype) ||
        (beta_kind != TRIUNE_BETA_NONE && !dtype_ok(beta_dtype)))
        return TRIUNE_ERR_DTYPE;
    if (B < 0 || T < 0 || H <= 0) return TRIUNE_ERR_SHAPE;
    if (!((Dk == 32 && Dv == 32) || (Dk == 64 && Dv == 64) || (Dk == 128 && Dv == 128))) return TRIUNE_ERR_SHAPE;
    if (!vec_ok(q, io_dtype, strides + 0, 3) || !vec_ok(k, io_dtype, strides + 3, 3) ||
        !vec_ok(g, g_dtype, strides + 9, 3) || reinterpret_cast<uintptr_t>(s0) % 16 ||
        reinterpret_cast<uintptr_t>(s_final) % 16)
        return TRIUNE_ERR_LAYOUT;
    if (B == 0) return TRIUNE_OK;
    GdnParams a{};
    a.q = q; a.k = k; a.v = v; a.g = g; a.beta = beta;
    a.io_dt = io_dtype; a.g_dt = g_dtype; a.beta_dt = beta_dtype; a.o_dt = o_dtype; a.beta_kind = beta_kind;
    a.q_sb = strides[0]; a.q_st = strides[1]; a.q_sh = strides[2];
    a.k_sb = strides[3]; a.k_st = strides[4]; a.k_sh = strides[5];
    a.v_sb = strides[6]; a.v_st = strides[7]; a.v_sh = strides[8];
    a.g_sb = strides[9]; a.g_st = strides[10]; a.g_sh = strides[11];
    a.b_sb = strides[12]; a.b_st = strides[13]; a.b_sh = strides[14];
    a.o_sb = strides[15]; a.o_st = strides[16]; a.o_sh = strides[17];
    a.o = o; a.s0 = s0; a.s_final = s_final;
    a.B = B; a.T = T; a.H = H;
    // A single token of many rows: the decode step (float4 state streaming) where the rows allow
    // vector loads (q, k, g, v rows aligned, beta fp32 and aligned); else the token-serial kernel.
    const bool vec_beta = beta_kind == TRIUNE_BETA_KEY || beta_kind == TRIUNE_BETA_VALUE;
    if (T == 1 && Dk == Dv && (Dk == 64 || Dk == 128) && gate_dtype_ok(io_dtype, g_dtype) &&
        vec_ok(v, io_dtype, strides + 6, 3) && vec4_ok(o, o_dtype, strides + 15, 3) &&
        (beta_kind == TRIUNE_BETA_NONE || beta_dtype == TRIUNE_DT_F32) &&
        (beta_kind != TRIUNE_BETA_HEAD || reinterpret_cast<uintptr_t>(beta) % 4 == 0) &&
        (!vec_beta || vec_ok(beta, TRIUNE_DT_F32, strides + 12, 3)))
        return launch_status(launch_gdn_decode(a, Dk, 4 * device_cus(), (hipStream_t)stream));
    return launch_status(launch_gdn_tokenwise(a, Dk, Dv, (hipStream_t)stream));
}

// Gated DeltaNet backward: checkpoints every L tokens, per-slice partial sums.  Where one wave per
// (b, h, 8 value columns) leaves resident slots free (six one-wave gradient workgroups of about
// 25 KB of LDS per CU at L = 512 / D), the tokens are cut into segments walked in parallel (not for
// beta per value column): the gradient kernel's NB segments (at most 16), each of up to four
// segments of the lighter kernels (4 from 3 gradient segments, 2 from 8, 1 from 16: at most 30
// light segments per sequence, so the serial carries over the segment maps stay short).  With
// more than two waves per CU (NB < 3) the sequence stays one segment.
struct GdnBwdPlan {
    int64_t nc, nsl, nq, nseg, segc, bsegc, bsegr;
    int L;
    size_t off_part, off_bh, off_seg, total;
};

static GdnBwdPlan plan_gdn_bwd(int64_t B, int64_t T, int64_t H, int D, int beta_kind) {
    GdnBwdPlan p{};
    p.nsl = gdn_bwd_col_slices(D);
    const int64_t waves = B * H * p.nsl, cus = device_cus();
    p.nseg = beta_kind != TRIUNE_BETA_VALUE && waves > 0 ? 6 * cus / waves : 1;
    if (p.nseg > 16) p.nseg = 16;  // each carry step is a D x D map product, walked serially
    // two segments at 4-token sub-chunks (D = 128, 768 waves) ran no faster than one at 8 tokens
    // and wrote twice the checkpoints: segment from three up
    if (p.nseg < 3) p.nseg = 1;
    p.L = p.nseg >= 2 ? 512 / D : gdn_bwd_chunk_tokens(D, waves, cus);
    p.nc = T > 0 ? (T + p.L - 1) / p.L : 0;
    if (p.nseg > p.nc) p.nseg = p.nc;
    if (p.nseg < 2) p.nseg = 1;
    p.bsegc = p.nseg > 1 ? (p.nc + p.nseg - 1) / p.nseg : p.nc;  // sub-chunks per gradient-kernel segment
    const int64_t rmax = p.nseg >= 16 ? 1 : (p.nseg >= 8 ? 2 : 4);
    p.bsegr = p.bsegc < rmax ? p.bsegc : rmax;
    if (p.nseg < 2) p.bsegr = 1;
    p.segc = (p.bsegc + p.bsegr - 1) / p.bsegr;
    p.bsegc = p.segc * p.bsegr;
    p.nseg = p.nc > 0 ? (p.nc + p.segc - 1) / p.segc : 1;
    p.nq = beta_kind == TRIUNE_BETA_KEY ? 4 : 3;
    const int64_t n = B * T * H;
    p.off_part = align_up((size_t)(B * H * p.nc) * D * D * sizeof(float));
    p.off_bh = p.off_part + align_up((size_t)(p.nq * p.nsl * n) * D * sizeof(float));
    p.off_seg = p.off_bh + align_up((size_t)(beta_kind == TRIUNE_BETA_HEAD ? p.nsl * n : 0) * sizeof(float));
    p.total = p.off_seg + (p.nseg > 1 ? 4 * align_up((size_t)(B * H * p.nseg) * D * D * sizeof(float)) : 0);
    return p;
}

size_t triune_hip_gdn_bwd_workspace_size(int64_t B, int64_t T, int64_t H, int Dk, int Dv, int beta_kind) {
    if (B < 0 || T < 0 || H <= 0 || Dk != Dv || (Dk != 64 && Dk != 128)) return 0;
    const size_t t = plan_gdn_bwd(B, T, H, Dk, beta_kind).total;
    return t > 0 ? t : 16;
}

int triune_hip_gdn_bwd(const void* q, const void* k, const void* v, const void* g, int io_dtype, int g_dtype,
                       const void* beta, int beta_dtype, int beta_kind, const int64_t* strides, const float* s0,
                       const void* dout, int dout_dtype, const float* ds_final, void* dq, void* dk, void* dv,
                       void* dg, void* dbeta, float* ds0, int64_t B, int64_t T, int64_t H, int Dk, int Dv,
                       void* workspace, size_t workspace_bytes, void* stream) {
    if (!q || !k || !v || !g || !strides || !dq || !dk || !dv || !dg) return TRIUNE_ERR_NULL;
    if (beta_kind < TRIUNE_BETA_NONE || beta_kind > TRIUNE_BETA_VALUE) return TRIUNE_ERR_SHAPE;
    if (beta_kind != TRIUNE_BETA_NONE && (!beta || !dbeta)) return TRIUNE_ERR_NULL;
    if (!dtype_ok(io_dtype) || !dtype_ok(g_dtype) || (dout && !dtype_ok(dout_dtype)) ||
        (beta_kind != TRIUNE_BETA_NONE && !dtype_ok(beta_dtype)))
        return TRIUNE_ERR_DTYPE;
    if (B < 0 || T < 0 || H <= 0 || Dk != Dv || (Dk != 64 && Dk != 128)) return TRIUNE_ERR_SHAPE;
    const int D = Dk;
    const bool vec_beta = beta_kind == TRIUNE_BETA_KEY || beta_kind == TRIUNE_BETA_VALUE;
    if (!vec_ok(q, io_dtype, strides + 0, 3) || !vec_ok(k, io_dtype, strides + 3, 3) ||
        !vec_ok(v, io_dtype, strides + 6, 3) || !vec_ok(g, g_dtype, strides + 9, 3) ||
        (vec_beta && !vec_ok(beta, beta_dtype, strides + 12, 3)) ||
        (dout && !vec_ok(dout, dout_dtype, strides + 15, 3)) || reinterpret_cast<uintptr_t>(s0) % 16 ||
        reinterpret_cast<uintptr_t>(ds_final) % 16 || reinterpret_cast<uintptr_t>(ds0) % 16)
        return TRIUNE_ERR_LAYOUT;
    if (B == 0) return TRIUNE_OK;
    const GdnBwdPlan pl = plan_gdn_bwd(B, T, H, D, beta_kind);
    hipStream_t st = (hipStream_t)stream;
    if (T == 0) {  // no tokens: the gradient of the initial state is that of the final state
        if (!ds0) return TRIUNE_OK;
        return launch_status(launch_gdn_slice_sum(ds_final, 1, 0, B * H * (int64_t)D * D, ds0, DT_F32, st));
    }
    if (!workspace || workspace_bytes < pl.total) return TRIUNE_ERR_WORKSPACE;
    char* ws = reinterpret_cast<char*>(workspace);
    if (reinterpret_cast<uintptr_t>(ws) % 16) return TRIUNE_ERR_LAYOUT;
    GdnBwdParams p{};
    GdnParams& a = p.f;
    a.q = q; a.k = k; a.v = v; a.g = g; a.beta = beta;
    a.io_dt = io_dtype; a.g_dt = g_dtype; a.beta_dt = beta_dtype; a.beta_kind = beta_kind;
    a.q_sb = strides[0]; a.q_st = strides[1]; a.q_sh = strides[2];
    a.k_sb = strides[3]; a.k_st = strides[4]; a.k_sh = strides[5];
    a.v_sb = strides[6]; a.v_st = strides[7]; a.v_sh = strides[8];
    a.g_sb = strides[9]; a.g_st = strides[10]; a.g_sh = strides[11];
    a.b_sb = strides[12]; a.b_st = strides[13]; a.b_sh = strides[14];
    a.s0 = s0;
    a.B = B; a.T = T; a.H = H;
    p.dout = dout; p.do_dt = dout_dtype; p.do_sb = strides[15]; p.do_st = strides[16]; p.do_sh = strides[17];
    p.dsf = ds_final;
    p.ckpt = reinterpret_cast<float*>(ws);
    p.part = reinterpret_cast<float*>(ws + pl.off_part);
    p.part_bh = reinterpret_cast<float*>(ws + pl.off_bh);
    p.dv = dv;
    p.dbeta_v = beta_kind == TRIUNE_BETA_VALUE ? dbeta : nullptr;
    p.dbeta_dt = beta_dtype;
    p.ds0 = ds0;
    p.nc = pl.nc;
    p.L = pl.L;
    p.nseg = pl.nseg;
    p.segc = pl.segc;
    p.bsegc = pl.bsegc;
    p.bsegr = pl.bsegr;
    if (pl.nseg > 1) {
        const size_t seg_bytes = align_up((size_t)(B * H * pl.nseg) * D * D * sizeof(float));
        p.seg_m = reinterpret_cast<float*>(ws + pl.off_seg);
        p.seg_n = reinterpret_cast<float*>(ws + pl.off_seg + seg_bytes);
        p.seg_dl = reinterpret_cast<float*>(ws + pl.off_seg + 2 * seg_bytes);
        p.seg_de = reinterpret_cast<float*>(ws + pl.off_seg + 3 * seg_bytes);
    }
    if (launch_gdn_bwd(p, D, st) != hipSuccess) return TRIUNE_ERR_LAUNCH;
    const int64_t n = B * T * H * D;
    if (launch_gdn_slice_sum(p.part, (int)pl.nsl, n, n, dq, io_dtype, st) != hipSuccess ||
        launch_gdn_slice_sum(p.part + pl.nsl * n, (int)pl.nsl, n, n, dk, io_dtype, st) != hipSuccess ||
        launch_gdn_slice_sum(p.part + 2 * pl.nsl * n, (int)pl.nsl, n, n, dg, g_dtype, st) != hipSuccess)
        return TRIUNE_ERR_LAUNCH;
    if (beta_kind == TRIUNE_BETA_KEY &&
        launch_gdn_slice_sum(p.part + 3 * pl.nsl * n, (int)pl.nsl, n, n, dbeta, beta_dtype, st) != hipSuccess)
        return TRIUNE_ERR_LAUNCH;
    if (beta_kind == TRIUNE_BETA_HEAD &&
        launch_gdn_slice_sum(p.part_bh, (int)pl.nsl, B * T * H, B * T * H, dbeta, beta_dtype, st) != hipSuccess)
        return TRIUNE_ERR_LAUNCH;
    return TRIUNE_OK;
}

}  // extern "C"

namespace {

// Chunked GDN: segments per sequence fill the resident output-kernel slots once (for I/O dtype
// io_dt; bf16 holds the most workgroups per CU, so its plan bounds the workspace of every dtype).
// D: head dim (Dk = Dv), 64 or 128; the workspace holds D x D fp32 states and M maps per segment.
struct GdnPlan {
    int64_t nseg, n_work;
    size_t off_m, off_spare, total;
};

// sg: the scalar-gate kernels (gdn_scalar.hip, D = 64), whose output kernel has its own occupancy.
GdnPlan plan_gdn(int64_t B, int64_t T, int64_t H, int io_dt, bool sg, int D) {
    static std::mutex mu;
    static std::map<int, int64_t> slots_cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = -1;
    int64_t slots;
    const bool ck = T % 4 != 0;  // the instance the launch picks (launch_gdn_t, launch_sg_t)
    {
        std::lock_guard<std::mutex> lock(mu);
        const int key = 32 * dev + 8 * io_dt + (D == 128 ? 4 : 0) + (sg ? 2 : 0) + (ck ? 1 : 0);
        auto it = slots_cache.find(key);
        if (it == slots_cache.end()) {
            int ncu = 0;
            if (dev < 0 || hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
                ncu <= 0)
                ncu = 256;
            const int per_cu = sg ? gdn_sg_seg_out_blocks_per_cu(io_dt, ck) : gdn_seg_out_blocks_per_cu(io_dt, ck, D);
            it = slots_cache.emplace(key, (int64_t)ncu * per_cu).first;
        }
        slots = it->second;
    }
    GdnPlan p{};
    const int64_t nchunks = (T + 63) / 64;
    const size_t dd = (size_t)D * D;
    p.nseg = slots / (B * H);
    if (p.nseg < 1) p.nseg = 1;
    if (p.nseg > nchunks) p.nseg = nchunks;
    p.n_work = B * p.nseg;
    p.off_m = align_up((size_t)p.n_work * H * dd * sizeof(float));
    p.off_spare = p.off_m + align_up((size_t)p.n_work * H * 3 * dd * 2);  // up to 3 bf16 parts of M
    p.total = p.off_spare + align_up((size_t)B * H * dd * sizeof(float));
    return p;
}

}  // namespace

extern "C" {

size_t triune_hip_gdn_prefill_chunked_workspace_size(int64_t B, int64_t T, int64_t H, int Dk, int Dv) {
    if (B <= 0 || T <= 0 || H <= 0 || Dk != Dv || (Dk != 64 && Dk != 128)) return 0;
    return plan_gdn(B, T, H, TRIUNE_DT_BF16, false, Dk).total;
}

size_t triune_hip_gdn_prefill_scalar_decay_workspace_size(int64_t B, int64_t T, int64_t H, int Dk, int Dv) {
    if (B <= 0 || T <= 0 || H <= 0 || Dk != 64 || Dv != 64) return 0;
    return plan_gdn(B, T, H, TRIUNE_DT_BF16, true, 64).total;
}

}  // extern "C"

namespace {

// The chunked GDN forward for both gate forms.  sg: g holds one log-decay per (token, head),
// element (b, t, h) at strides[9..11] (any non-negative strides, element-aligned); otherwise
// g is [B, T, H, Dk] like q and k.
int gdn_chunked_impl(const void* q, const void* k, const void* v, const void* g, int io_dtype, int g_dtype,
                     const void* beta, int beta_dtype, int beta_kind, const int64_t* strides, const float* s0, void* o,
                     int o_dtype, float* s_final, int64_t B, int64_t T, int64_t H, int Dk, int Dv, void* workspace,
                     size_t workspace_bytes, void* stream, bool sg) {
    if (!q || !k || !v || !g || !o || !strides) return TRIUNE_ERR_NULL;
    // beta per key dim or per value dim: fp32 rows of Dk (= Dv) values, read by the per-dim kernels
    const bool vec_beta = beta_kind == TRIUNE_BETA_KEY || beta_kind == TRIUNE_BETA_VALUE;
    if (beta_kind != TRIUNE_BETA_NONE && beta_kind != TRIUNE_BETA_HEAD && (sg || !vec_beta)) return TRIUNE_ERR_SHAPE;
    if (beta_kind != TRIUNE_BETA_NONE && !beta) return TRIUNE_ERR_NULL;
    if (!dtype_ok(io_dtype) || !dtype_ok(g_dtype) || !dtype_ok(o_dtype) || !gate_dtype_ok(io_dtype, g_dtype) ||
        (beta_kind != TRIUNE_BETA_NONE && !dtype_ok(beta_dtype)) ||
        (vec_beta && beta_dtype != TRIUNE_DT_F32))
        return TRIUNE_ERR_DTYPE;
    if (B < 0 || T < 0 || H <= 0 || Dk != Dv || (Dk != 64 && (sg || Dk != 128))) return TRIUNE_ERR_SHAPE;
    if (Dk == 128 && io_dtype == TRIUNE_DT_F32) return TRIUNE_ERR_DTYPE;  // fp32 planes exceed LDS at D = 128
    const bool g_ok = sg ? (reinterpret_cast<uintptr_t>(g) % (g_dtype == TRIUNE_DT_F32 ? 4 : 2) == 0 &&
                            strides[9] >= 0 && strides[10] >= 0 && strides[11] >= 0)
                         : vec_ok(g, g_dtype, strides + 9, 3);
    if (!vec_ok(q, io_dtype, strides + 0, 3) || !vec_ok(k, io_dtype, strides + 3, 3) ||
        !vec_ok(v, io_dtype, strides + 6, 3) || !g_ok || !vec_ok(o, o_dtype, strides + 15, 3) ||
        reinterpret_cast<uintptr_t>(s0) % 16 || reinterpret_cast<uintptr_t>(s_final) % 16 ||
        (vec_beta &&
         (!vec_ok(beta, TRIUNE_DT_F32, strides + 12, 3) || strides[13] < Dk || (64 * strides[13] + Dk) * 4 >= ((int64_t)1 << 31))))
        return TRIUNE_ERR_LAYOUT;
    // o strides sit at 15..17 here (beta takes 12..14); tok_strides_ok reads o's token stride at 13.
    // A scalar gate is read one element per token, so its token stride has no lower bound.
    const int64_t ost[15] = {strides[0], strides[1], strides[2], strides[3], strides[4], strides[5],
                             strides[6], strides[7], strides[8], strides[9], sg ? (int64_t)Dk : strides[10],
                             strides[11], strides[15], strides[16], strides[17]};
    if (!tok_strides_ok(ost, io_dtype, g_dtype, o_dtype, Dk, Dv)) return TRIUNE_ERR_LAYOUT;
    hipStream_t st = (hipStream_t)stream;
    if (B == 0) return TRIUNE_OK;
    if (T == 0) {
        if (!s_final) return TRIUNE_OK;
        ScanParams sc{};  // N = 0: fin = init (or zero)
        sc.kv = s_final; sc.kv_dt = DT_F32; sc.dec = s_final; sc.dec_dt = DT_F32;
        sc.init = s0; sc.i_so = H * (int64_t)Dk * Dv; sc.i_sh = (int64_t)Dk * Dv;
        sc.fin = s_final; sc.fin_dt = DT_F32; sc.f_so = sc.i_so; sc.f_sh = sc.i_sh;
        sc.n_outer = B; sc.H = H; sc.Dk = Dk; sc.Dv = Dv; sc.N = 0;
        return launch_status(launch_recurrent_scan(sc, st));
    }
    const GdnPlan pl = plan_gdn(B, T, H, io_dtype, sg, Dk);
    if (!workspace || workspace_bytes < pl.total) return TRIUNE_ERR_WORKSPACE;
    char* ws = reinterpret_cast<char*>(workspace);
    if (reinterpret_cast<uintptr_t>(ws) % 16) return TRIUNE_ERR_LAYOUT;

    PrefillParams a{};
    fill_tok(a.q, q, strides + 0, B, T, H, Dk, io_dtype);
    fill_tok(a.k, k, strides + 3, B, T, H, Dk, io_dtype);
    fill_tok(a.v, v, strides + 6, B, T, H, Dv, io_dtype);
    fill_tok(a.g, g, strides + 9, B, T, H, sg ? 1 : Dk, g_dtype);
    a.o = o; a.o_sb = strides[15]; a.o_st = strides[16]; a.o_sh = strides[17];
    a.g_dt = g_dtype; a.o_dt = o_dtype;
    a.s0 = s0;
    a.ws_state = reinterpret_cast<float*>(ws);
    a.ws_m = reinterpret_cast<float*>(ws + pl.off_m);
    a.ws_spare = reinterpret_cast<float*>(ws + pl.off_spare);
    a.n_seqs = B; a.H = H; a.T = T; a.Dk = Dk; a.Dv = Dv;
    a.P = 0; a.nseg_dense = (int)pl.nseg; a.varlen = 0; a.flags = 0;
    a.beta = beta; a.beta_dt = beta_dtype; a.beta_kind = beta_kind;
    a.b_sb = strides[12]; a.b_st = strides[13]; a.b_sh = strides[14];
    if (vec_beta) fill_tok(a.kb, beta, strides + 12, B, T, H, Dk, TRIUNE_DT_F32);

    if (beta_kind == TRIUNE_BETA_VALUE) {
        // beta per value column: every column has its own segment map, so each sequence is one
        // segment, walked by the output kernel alone (it writes the final state)
        a.nseg_dense = 1;
        a.gdn_whole = 1;
        a.seq_final = s_final;
        return launch_status(launch_gdn_seg_out(a, B, io_dtype, st));
    }
    hipError_t e = sg ? launch_gdn_sg_seg_mn(a, pl.n_work, io_dtype, st) : launch_gdn_seg_mn(a, pl.n_work, io_dtype, st);
    if (e != hipSuccess) return TRIUNE_ERR_LAUNCH;
    e = launch_gdn_seg_scan(a, s_final, io_dtype, st);
    if (e != hipSuccess) return TRIUNE_ERR_LAUNCH;
    return launch_status(sg ? launch_gdn_sg_seg_out(a, pl.n_work, io_dtype, st)
                            : launch_gdn_seg_out(a, pl.n_work, io_dtype, st));
}

}  // namespace

extern "C" {

int triune_hip_gdn_prefill_chunked(const void* q, const void* k, const void* v, const void* g, int io_dtype,
                                   int g_dtype, const void* beta, int beta_dtype, int beta_kind,
                                   const int64_t* strides, const float* s0, void* o, int o_dtype, float* s_final,
                                   int64_t B, int64_t T, int64_t H, int Dk, int Dv, void* workspace,
                                   size_t workspace_bytes, void* stream) {
    return gdn_chunked_impl(q, k, v, g, io_dtype, g_dtype, beta, beta_dtype, beta_kind, strides, s0, o, o_dtype,
                            s_final, B, T, H, Dk, Dv, workspace, workspace_bytes, stream, false);
}

int triune_hip_gdn_prefill_scalar_decay(const void* q, const void* k, const void* v, const void* g, int io_dtype,
                                        int g_dtype, const void* beta, int beta_dtype, int beta_kind,
                                        const int64_t* strides, const float* s0, void* o, int o_dtype,
                                        float* s_final, int64_t B, int64_t T, int64_t H, int Dk, int Dv,
                                        void* workspace, size_t workspace_bytes, void* stream) {
    return gdn_chunked_impl(q, k, v, g, io_dtype, g_dtype, beta, beta_dtype, beta_kind, strides, s0, o, o_dtype,
                            s_final, B, T, H, Dk, Dv, workspace, workspace_bytes, stream, true);
}

int triune_hip_gla_qkvg_prep(void* qkv, void* g, int io_dtype, const int64_t* strides, const void* cos,
                             const void* sin, int cs_dtype, int64_t cs_stride, int use_rope, int64_t B, int64_t T,
                             int64_t H, int HD, void* stream) {
    if (!qkv || !g || !strides || (use_rope && (!cos || !sin))) return TRIUNE_ERR_NULL;
    if (!dtype_ok(io_dtype) || (use_rope && !dtype_ok(cs_dtype))) return TRIUNE_ERR_DTYPE;
    if (B < 0 || T < 0 || H <= 0 || (HD != 32 && HD != 64 && HD != 128)) return TRIUNE_ERR_SHAPE;
    const int64_t rows = B * T * H;
    if (rows > (int64_t)16 * 0x7fffffff) return TRIUNE_ERR_SHAPE;  // grid: ceil(rows / rows-per-block >= 16) blocks
    if (rows == 0) return TRIUNE_OK;
    // qkv strides (b, t, part, h) and g strides (b, t, h), elements; rows of 8-element vectors
    if (!vec_ok(qkv, io_dtype, strides + 0, 4) || !vec_ok(g, io_dtype, strides + 4, 3)) return TRIUNE_ERR_LAYOUT;
    if (use_rope && (!vec_ok(cos, cs_dtype, &cs_stride, 1) || !vec_ok(sin, cs_dtype, &cs_stride, 1)))
        return TRIUNE_ERR_LAYOUT;
    PrepParams a{};
    a.qkv = qkv; a.qkv_sb = strides[0]; a.qkv_st = strides[1]; a.qkv_sp = strides[2]; a.qkv_sh = strides[3];
    a.g = g; a.g_sb = strides[4]; a.g_st = strides[5]; a.g_sh = strides[6];
    a.cos = cos; a.sin = sin; a.cs_st = cs_stride; a.use_rope = use_rope ? 1 : 0;
    a.B = B; a.T = T; a.H = H;
    return launch_status(launch_gla_prep(a, HD, io_dtype, use_rope ? cs_dtype : TRIUNE_DT_F32, (hipStream_t)stream));
}

int triune_hip_gla_fused_decode_step(const void* qkvg, int io_dtype, const int64_t* strides, const void* cos,
                                     const void* sin, int cs_dtype, int use_rope, const void* state_in,
                                     void* state_out, int state_dtype, void* o, int o_dtype,
                                     const int64_t* o_strides, int64_t B, int64_t H, int HD, void* stream) {
    if (!qkvg || !strides || !o || !o_strides || (use_rope && (!cos || !sin))) return TRIUNE_ERR_NULL;
    if (!dtype_ok(io_dtype) || !dtype_ok(o_dtype) || !dtype_ok(state_dtype)) return TRIUNE_ERR_DTYPE;
    if (state_dtype != TRIUNE_DT_F32 && state_dtype != io_dtype) return TRIUNE_ERR_DTYPE;
    if (use_rope && cs_dtype != TRIUNE_DT_F32 && cs_dtype != io_dtype) return TRIUNE_ERR_DTYPE;
    if (B < 0 || H <= 0 || (HD != 32 && HD != 64 && HD != 128)) return TRIUNE_ERR_SHAPE;
    if (B > 0x7fffffff / H) return TRIUNE_ERR_SHAPE;  // one block per (b, h)
    if (B == 0) return TRIUNE_OK;
    const int sal = state_dtype == TRIUNE_DT_F32 ? 16 : 8;
    if (reinterpret_cast<uintptr_t>(state_in) % sal || reinterpret_cast<uintptr_t>(state_out) % sal ||
        !vec4_ok(o, o_dtype, o_strides, 2) || !vec4_ok(qkvg, io_dtype, strides, 3))
        return TRIUNE_ERR_LAYOUT;
    if (use_rope && (!vec4_ok(cos, cs_dtype, strides, 0) || !vec4_ok(sin, cs_dtype, strides, 0)))
        return TRIUNE_ERR_LAYOUT;
    FusedDecodeParams a{};
    a.qkvg = qkvg; a.x_sb = strides[0]; a.x_sp = strides[1]; a.x_sh = strides[2];
    a.cos = cos; a.sin = sin; a.use_rope = use_rope ? 1 : 0;
    a.has_init = state_in != nullptr; a.save_final = state_out != nullptr;
    a.state_in = state_in; a.state_out = state_out;
    a.o = o; a.o_dt = o_dtype; a.o_sb = o_strides[0]; a.o_sh = o_strides[1];
    a.B = B; a.H = H; a.max_blocks = kFusedDecodeBlocksPerCU * device_cus();
    return launch_status(
        launch_gla_fused_decode(a, HD, io_dtype, use_rope ? cs_dtype : TRIUNE_DT_F32, state_dtype, (hipStream_t)stream));
}

int triune_hip_gla_fused_decode_step_slots(const void* qkvg, int io_dtype, const int64_t* strides, const void* cos,
                                           const void* sin, int cs_dtype, int use_rope, void* state_pool,
                                           int state_dtype, const int32_t* slots, int64_t n_slots, void* o,
                                           int o_dtype, const int64_t* o_strides, int64_t B, int64_t H, int HD,
                                           void* stream) {
    if (!qkvg || !strides || !o || !o_strides || !state_pool || !slots || (use_rope && (!cos || !sin)))
        return TRIUNE_ERR_NULL;
    if (!dtype_ok(io_dtype) || !dtype_ok(o_dtype) || !dtype_ok(state_dtype)) return TRIUNE_ERR_DTYPE;
    if (state_dtype != TRIUNE_DT_F32 && state_dtype != io_dtype) return TRIUNE_ERR_DTYPE;
    if (use_rope && cs_dtype != TRIUNE_DT_F32 && cs_dtype != io_dtype) return TRIUNE_ERR_DTYPE;
    if (B < 0 || H <= 0 || n_slots < 0 || (HD != 32 && HD != 64 && HD != 128)) return TRIUNE_ERR_SHAPE;
    if (B > 0x7fffffff / H || n_slots > 0x7fffffff / H) return TRIUNE_ERR_SHAPE;
    if (B == 0) return TRIUNE_OK;
    const int sal = state_dtype == TRIUNE_DT_F32 ? 16 : 8;
    if (reinterpret_cast<uintptr_t>(state_pool) % sal || reinterpret_cast<uintptr_t>(slots) % 4 ||
        !vec4_ok(o, o_dtype, o_strides, 2) || !vec4_ok(qkvg, io_dtype, strides, 3))
        return TRIUNE_ERR_LAYOUT;
    if (use_rope && (!vec4_ok(cos, cs_dtype, strides, 0) || !vec4_ok(sin, cs_dtype, strides, 0)))
        return TRIUNE_ERR_LAYOUT;
    FusedDecodeParams a{};
    a.qkvg = qkvg; a.x_sb = strides[0]; a.x_sp = strides[1]; a.x_sh = strides[2];
    a.cos = cos; a.sin = sin; a.use_rope = use_rope ? 1 : 0;
    a.has_init = 1; a.save_final = 1;
    a.state_in = state_pool; a.state_out = state_pool;
    a.slots = slots; a.n_state_rows = n_slots;
    a.o = o; a.o_dt = o_dtype; a.o_sb = o_strides[0]; a.o_sh = o_strides[1];
    a.B = B; a.H = H; a.max_blocks = kFusedDecodeBlocksPerCU * device_cus();
    return launch_status(
        launch_gla_fused_decode(a, HD, io_dtype, use_rope ? cs_dtype : TRIUNE_DT_F32, state_dtype, (hipStream_t)stream));
}

}  // extern "C"
