/*
 * triune_hip.h -- C ABI of libtriune_hip.so, the MI355X (gfx950) implementation of the
 * reference's gated-linear-attention inference path.
 *
 * Conventions (shared by every entry point):
 *   - Every pointer argument named q, k, v, g, beta, o, kv, decay, s_all, fin, state*, s0,
 *     s_final, cu_seqlens, slots, workspace is a DEVICE pointer; `strides` arrays are HOST
 *     arrays read during the call.  The library never allocates or frees device memory.
 *   - Token tensors use the reference layout [B, T, H, D] (varlen: [N_tok, H, D]) with the
 *     innermost (D) stride 1; the other strides are given in elements.  States are
 *     contiguous fp32 [*, H, Dk, Dv] with S[i][j], i = key index, j = value index.
 *   - dtype codes: TRIUNE_DT_F32, TRIUNE_DT_BF16, TRIUNE_DT_F16.
 *   - Work is enqueued on `stream` (a hipStream_t, passed as void*) without host
 *     synchronisation or device allocation, so calls can be captured in a hipGraph.
 *   - Return 0 on success or a negative TRIUNE_ERR_* code; nothing is launched on error.
 *
 * Reference interfaces replaced (paths under the reference repository):
 *   triune_hip_gla_decode_step     <- triune_gla_recurrent_step_f32, csrc/engine/api.h:94-103
 *                                     (engine.cpp:419-475); launch_gla_decode_step,
 *                                     csrc/kernels/gla.cu:97-114; the T == 1 branch of
 *                                     fast_chunk_gla, triune/kernels/fast_gla.py:746-753
 *   triune_hip_gla_prefill         <- _triton_chunk_gla_tc_fwd, triune/kernels/fast_gla.py:318-380,
 *                                     and fast_chunk_gla's chunked path, fast_gla.py:692-778
 *   triune_hip_gla_prefill_varlen  <- no reference counterpart (the reference has no
 *                                     cu_seqlens path); one launch = a Python loop of
 *                                     fast_chunk_gla calls over the packed sequences
 *   triune_hip_gla_prefill_bwd     <- the gradients of fast_chunk_gla's training path (autograd through
 *                                     _run_gla_chunks, triune/kernels/fast_gla.py:569-689, and
 *                                     FusedRecurrentScan.backward, fast_gla.py:151-203)
 *   triune_hip_gla_prefill_varlen_pool <- no reference counterpart: the varlen prefill over a
 *                                     device state pool, the device-side form of the reference's
 *                                     per-session (state, offset) caches (triune/api/srsm.py:11-112,
 *                                     triune/model/attention.py:333-358)
 *   triune_hip_recurrent_scan_fwd  <- FusedRecurrentScan.forward, triune/kernels/fast_gla.py:109-149
 *                                     (_recurrent_scan_fwd, fast_gla.py:34-64)
 *   triune_hip_recurrent_scan_bwd  <- FusedRecurrentScan.backward, triune/kernels/fast_gla.py:151-203
 *                                     (_recurrent_scan_bwd, fast_gla.py:67-107)
 *   triune_hip_gdn_prefill         <- fast_chunk_gated_deltanet, triune/kernels/fast_gla.py:839-904,
 *                                     with _triton_gated_deltanet_fwd (fast_gla.py:479-550) and
 *                                     fast_recurrent_gated_deltanet (fast_gla.py:781-836)
 *   triune_hip_gdn_prefill_chunked <- the same operator (fast_gla.py:839-904), chunked form
 *   triune_hip_gdn_prefill_scalar_decay <- the same operator with g broadcast over the head dim
 *                                     (one decay per token and head), chunked form
 *   triune_hip_gdn_bwd             <- the gradients of fast_chunk_gated_deltanet's training path:
 *                                     autograd through fast_recurrent_gated_deltanet
 *                                     (triune/kernels/fast_gla.py:781-836), which the operator runs
 *                                     whenever a gradient is needed (fast_gla.py:885-904)
 *   triune_hip_gla_qkvg_prep       <- _fused_qkv_g_prep_inplace_kernel, triune/model/attention.py:14-79
 *   triune_hip_gla_fused_decode_step <- _fused_qkvg_decode_step_kernel, triune/model/attention.py:81-179
 */
#ifndef TRIUNE_HIP_H
#define TRIUNE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TRIUNE_HIP_ABI_VERSION 3

enum {
    TRIUNE_DT_F32 = 0,
    TRIUNE_DT_BF16 = 1,
    TRIUNE_DT_F16 = 2,
};

enum {
    TRIUNE_OK = 0,
    TRIUNE_ERR_NULL = -1,        /* a required pointer is NULL */
    TRIUNE_ERR_SHAPE = -2,       /* unsupported or inconsistent sizes */
    TRIUNE_ERR_DTYPE = -3,       /* unsupported dtype code */
    TRIUNE_ERR_LAYOUT = -4,      /* stride / alignment requirement not met */
    TRIUNE_ERR_WORKSPACE = -5,   /* workspace missing or smaller than required */
    TRIUNE_ERR_LAUNCH = -6,      /* the HIP runtime rejected a launch */
    TRIUNE_ERR_SCRATCH = -7,     /* larger than the allocation-free entry point's static scratch */
    TRIUNE_ERR_MEMORY = -8,      /* a pointer is not device memory of the current device */
};

/* Prefill flags. */
#define TRIUNE_FLAG_TAIL_UNCLAMPED 0x1 /* last token of each sequence keeps g > 0 (see below) */
#define TRIUNE_FLAG_SEG_SHIFT 8        /* bits 8..15: chunks per segment, 0 = automatic */
#define TRIUNE_FLAG_BWD_ACC_QKG 0x2    /* backward: add dq, dk, dg into their fp32 buffers */
#define TRIUNE_FLAG_BWD_ACC_V 0x4      /* backward: add dv into its fp32 buffer */

/* Gated DeltaNet beta kinds. */
enum {
    TRIUNE_BETA_NONE = 0,  /* beta = 1 */
    TRIUNE_BETA_HEAD = 1,  /* beta [B, T, H]: one scalar per token and head */
    TRIUNE_BETA_KEY = 2,   /* beta [B, T, H, Dk]: scales rows of k u^T (reference PyTorch path) */
    TRIUNE_BETA_VALUE = 3, /* beta [B, T, H, Dv]: scales columns of k u^T (reference Triton path) */
};

int triune_hip_abi_version(void);
const char* triune_hip_error_string(int code);

/* Measurement hook (no reference counterpart; for benchmarks and profilers): arm two hipEvent_t
 * (passed as void*) that the following GLA prefill calls (dense and varlen: the output kernel,
 * the dominant one of the three; the single-launch entry: its one kernel) of this host thread
 * attach to that kernel's dispatch (hipExtLaunchKernel), so its duration can be read with
 * hipEventElapsedTime (including the dispatch latency, about 4 us on MI355X).  Both NULL
 * disarms; exactly one NULL returns TRIUNE_ERR_NULL.  Arming adds no device work. */
int triune_hip_set_output_kernel_events(void* begin, void* end);

/* Batched recurrent decode step, for every row (b, h):
 *     S <- diag(exp(g)) S + k v^T ;   o = S^T q          (g is NOT clamped, as in the reference)
 * q, k, g: [B, 1, H, Dk] (g may be fp32 when q/k/v are 16-bit: g_dtype), v: [B, 1, H, Dv],
 * o: [B, 1, H, Dv] in o_dtype.  strides[10] = (batch, head) element strides of q, k, v, g, o.
 * state_in / state_out: fp32 [n_state_rows, H, Dk, Dv]; they may be the same buffer (in place).
 * slots: NULL (state row b for batch b; n_state_rows >= B) or int32 [B] state-row indices (a
 * state pool); a batch row whose slot lies outside [0, n_state_rows) (e.g. -1 for a padded row)
 * reads and writes no state and gets zero outputs.
 * Supported (Dk, Dv): (32,32), (64,64), (128,128), (64,128), (128,64).
 * Replaces: triune_gla_recurrent_step_f32 (api.h:94-103), launch_gla_decode_step (gla.cu:97-114). */
int triune_hip_gla_decode_step(const void* q, const void* k, const void* v, const void* g, int io_dtype,
                               int g_dtype, const int64_t* strides, const float* state_in, float* state_out,
                               const int32_t* slots, int64_t n_state_rows, void* o, int o_dtype, int64_t B,
                               int64_t H, int Dk, int Dv, void* stream);

/* The reference's own decode-step signatures, for callers that bind them by name (device
 * pointers instead of the reference's host pointers; both run triune_hip_gla_decode_step in
 * place and return nothing, as the reference's do; the status of the last such call on this
 * host thread is triune_hip_last_error()).  Before launching, each asks the HIP runtime where
 * every pointer lives (hipPointerGetAttributes): unless all are device memory of the current
 * device, nothing is launched or written and the status is TRIUNE_ERR_MEMORY.  The reference's
 * caller of triune_gla_recurrent_step_f32 (triune/ops/_c_bridge.py:259-294) passes host memory
 * of CPU tensors; it gets that error here, never a kernel on host pointers. 
 *   launch_gla_decode_step: bf16 Q, K, V, Out [B, 1, H, HD] and fp32 G [B, 1, H, HD], fp32
 *     State [B, H, HD, HD] updated in place, all contiguous, on `stream` (a hipStream_t);
 *     HD in {32, 64, 128}.  Replaces: launch_gla_decode_step, csrc/kernels/gla.cu:97-114.
 *   triune_gla_recurrent_step_f32: fp32 q, k, v, g, out [batch_heads, head_dim] and state
 *     [batch_heads, head_dim, head_dim] updated in place, on the null stream; head_dim in {32, 64,
 *     128}.  Replaces: triune_gla_recurrent_step_f32, csrc/engine/api.h:94-103 (engine.cpp:419-475),
 *     bound by triune/ops/_c_bridge.py:132-142. */
int triune_hip_last_error(void);
void launch_gla_decode_step(const void* Q, const void* K, const void* V, const float* G, float* State, void* Out,
                            int B, int H, int HD, void* stream);
void triune_gla_recurrent_step_f32(const float* q, const float* k, const float* v, const float* g, float* state,
                                   float* out, int batch_heads, int head_dim);

/* Chunked GLA prefill over dense [B, T, H, D] tensors:
 *     S_t = diag(exp(min(g_t, 0))) S_{t-1} + k_t v_t^T ;   o_t = S_t^T q_t ,   S_{-1} = s0 (or 0)
 * q, k, g: Dk wide; v, o: Dv wide.  strides[15] = (batch, token, head) element strides of
 * q, k, v, g, o.  o may alias g when both have the same dtype and strides (the reference's
 * VectorisedGLA passes out=g, attention.py:443-451).  s0 / s_final: fp32 [B, H, Dk, Dv] or NULL.
 * flags: TRIUNE_FLAG_TAIL_UNCLAMPED reproduces fast_chunk_gla's unclamped single-token
 * remainder (fast_gla.py:768-775) for the last token.  (Dk, Dv) in {(32,32), (64,64), (128,128),
 * (64,128), (128,64)}; g_dtype is io_dtype or TRIUNE_DT_F32.
 * workspace: device buffer of at least triune_hip_gla_prefill_workspace_size(...) bytes.
 * Replaces: _triton_chunk_gla_tc_fwd (fast_gla.py:318-380), fast_chunk_gla (fast_gla.py:692-778). */
size_t triune_hip_gla_prefill_workspace_size(int64_t B, int64_t T, int64_t H, int Dk, int Dv, int flags);
int triune_hip_gla_prefill(const void* q, const void* k, const void* v, const void* g, int io_dtype, int g_dtype,
                           const int64_t* strides, const float* s0, void* o, int o_dtype, float* s_final,
                           int64_t B, int64_t T, int64_t H, int Dk, int Dv, int flags, void* workspace,
                           size_t workspace_bytes, void* stream);

/* triune_hip_gla_prefill on raw projections with the VectorisedGLA input pre-processing done by
 * the prefill's segment-state kernel: q, k, v, g are the raw projections (e.g. the qkv[:, :, i]
 * views of [B, T, 3, H, D] and g [B, T, H, D], all in io_dtype, bf16 or fp16).  While it forms the
 * segment states, that kernel writes back, in place and rounded to io_dtype,
 *     q <- RoPE(normalize(elu(q) + 1)),  k <- RoPE(normalize(elu(k) + 1)),  g <- logsigmoid(g)
 * with normalize(a) = a / sqrt(max(sum a^2, 1e-12)) per (token, head) row and RoPE pairing d with
 * d + D/2 from the fp32 tables cos/sin [T, D] (row t for token t, cs_stride elements apart; used
 * when use_rope != 0), and uses those rounded values itself; the output kernel then reads them.
 * Results and the in-place side effect are those of triune_hip_gla_qkvg_prep followed by
 * triune_hip_gla_prefill.  strides[15] as for triune_hip_gla_prefill; o may alias g.  D in {32, 64,
 * 128}; workspace as for triune_hip_gla_prefill(B, T, H, D, D, 0).
 * Replaces: _fused_qkv_g_prep_inplace_kernel (triune/model/attention.py:14-79) followed by
 * _triton_chunk_gla_tc_fwd (fast_gla.py:318-380), as VectorisedGLA launches them
 * (attention.py:425-451), without the prep kernel's separate pass over q, k, g. */
int triune_hip_gla_prefill_prep(const void* q, const void* k, const void* v, const void* g, int io_dtype,
                                const int64_t* strides, const float* cos, const float* sin, int64_t cs_stride,
                                int use_rope, const float* s0, void* o, int o_dtype, float* s_final, int64_t B,
                                int64_t T, int64_t H, int D, void* workspace, size_t workspace_bytes, void* stream);

/* Single-launch GLA prefill for calls of few chunks (Dk = Dv = D = 64, bf16 or fp16 I/O): one
 * workgroup per two consecutive 64-token chunks of each (sequence, head); each publishes the state
 * map of its chunks and folds the earlier ones' into the state it enters with, so pre-processing
 * (prep != 0), states and outputs take one launch instead of the three of
 * triune_hip_gla_prefill(_prep).
 * Arguments as triune_hip_gla_prefill (prep == 0: g_dtype is io_dtype or fp32, flags 0 or
 * TRIUNE_FLAG_TAIL_UNCLAMPED) or triune_hip_gla_prefill_prep (prep != 0: q, k, g raw projections,
 * rewritten in place with RoPE(normalize(elu(x) + 1)) / logsigmoid; g_dtype = io_dtype; flags 0;
 * cos/sin fp32 [T, D] rows cs_stride apart when use_rope).
 * triune_hip_gla_prefill_onepass_supported says whether a call fits: at most 64 chunks per sequence
 * and every workgroup resident at once (one per CU: ceil(B * H / 8) x ceil(chunks / 2) at most
 * CUs / 8); otherwise the entry returns TRIUNE_ERR_SHAPE and launches nothing.
 * workspace: at least triune_hip_gla_prefill_onepass_workspace_size bytes (16 KB per chunk pair).
 * ctrl: caller-owned device buffer of at least triune_hip_gla_prefill_onepass_ctrl_size bytes,
 * 16-byte aligned, ZERO before its first use; each call leaves it ready for the next.  Calls that
 * share a ctrl buffer must be ordered on one stream (concurrent calls need their own).  Word 2 of
 * ctrl is an error mask the kernel sets if a wait for earlier chunks ever ran out (bit 0) or their
 * workgroup ran on another XCD than the reader's (bit 1); neither happens when the hardware hands
 * workgroups to XCDs round robin, as it does; outputs of a call that sets either are not valid.
 * Replaces: VectorisedGLA's prefill tile, _fused_qkv_g_prep_inplace_kernel followed by
 * _triton_chunk_gla_tc_fwd (triune/model/attention.py:14-79, 425-451, 458-499), and
 * _triton_chunk_gla_tc_fwd / fast_chunk_gla on such calls (triune/kernels/fast_gla.py:318-380, 692-778). */
int triune_hip_gla_prefill_onepass_supported(int64_t B, int64_t T, int64_t H, int D, int io_dtype, int g_dtype,
                                             int prep, int flags);
size_t triune_hip_gla_prefill_onepass_workspace_size(int64_t B, int64_t T, int64_t H, int D);
size_t triune_hip_gla_prefill_onepass_ctrl_size(int64_t B, int64_t T, int64_t H, int D);
int triune_hip_gla_prefill_onepass(const void* q, const void* k, const void* v, const void* g, int io_dtype,
                                   int g_dtype, const int64_t* strides, const float* cos, const float* sin,
                                   int64_t cs_stride, int prep, int use_rope, const float* s0, void* o, int o_dtype,
                                   float* s_final, int64_t B, int64_t T, int64_t H, int D, int flags, void* workspace,
                                   size_t workspace_bytes, void* ctrl, size_t ctrl_bytes, void* stream);

/* triune_hip_gla_prefill without a workspace argument, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference.  The workspace is a static device array of
 * TRIUNE_GLA_PREFILL_SCRATCH_BYTES (32 MiB) per GPU, held until the process ends; a call whose
 * workspace (triune_hip_gla_prefill_workspace_size) exceeds it returns TRIUNE_ERR_SCRATCH and
 * launches nothing.  Config 1 (B = 4, T = 16384, H = 6, D = 64) needs about 8 MB; at D = 128 the
 * bound is reached near B * H = 500 (head, sequence) pairs.  Every call on a GPU shares that
 * GPU's array (each call writes what it reads, so nothing needs clearing): calls that overlap on
 * one GPU (other streams or host threads) race and must be serialised by the caller.  stream must
 * belong to the current device.  Same arguments, semantics and results as
 * triune_hip_gla_prefill otherwise.  No device memory is allocated or freed. */
#define TRIUNE_GLA_PREFILL_SCRATCH_BYTES (32u << 20)
size_t triune_hip_gla_prefill_noalloc_max_bytes(void);
int triune_hip_gla_prefill_noalloc(const void* q, const void* k, const void* v, const void* g, int io_dtype,
                                   int g_dtype, const int64_t* strides, const float* s0, void* o, int o_dtype,
                                   float* s_final, int64_t B, int64_t T, int64_t H, int Dk, int Dv, int flags,
                                   void* stream);

/* Packed ragged GLA prefill: sequence i covers rows [cu_seqlens[i], cu_seqlens[i+1]) of the
 * [total_tokens, H, D] tensors, starts from s0[i] (or 0) and ends in s_final[i]; every token's
 * g is clamped at 0.  cu_seqlens: device int32 [n_seqs + 1], non-decreasing, cu[0] = 0,
 * cu[n_seqs] = total_tokens.  strides[10] = (token, head) element strides of q, k, v, g, o.
 * Head dims and dtypes as for triune_hip_gla_prefill.
 * No reference counterpart: the reference has no cu_seqlens path; this is one launch for what
 * would be a loop of fast_chunk_gla calls (fast_gla.py:692-778), one per sequence. */
size_t triune_hip_gla_prefill_varlen_workspace_size(int64_t n_seqs, int64_t total_tokens, int64_t H, int Dk,
                                                    int Dv, int flags);
int triune_hip_gla_prefill_varlen(const void* q, const void* k, const void* v, const void* g, int io_dtype,
                                  int g_dtype, const int64_t* strides, const int32_t* cu_seqlens, int64_t n_seqs,
                                  int64_t total_tokens, const float* s0, void* o, int o_dtype, float* s_final,
                                  int64_t H, int Dk, int Dv, int flags, void* workspace, size_t workspace_bytes,
                                  void* stream);

/* Gradients of triune_hip_gla_prefill (dense, same flags) for the upstream gradients dout (of o,
 * [B, T, H, Dv] in io_dtype) and ds_final (of the final state, fp32 [B, H, Dk, Dv], or NULL = 0):
 *     dq_t = S_t do_t ,  dk_t = D_t v_t ,  dv_t = D_t^T k_t ,  ds0 = diag(a_0) D_0 ,
 *     dg_t[i] = sum_{r >= t} (q_r[i] dq_r[i] - k_r[i] dk_r[i]) + sum_j ds_final[i][j] S_T[i][j]
 * with D_t the total gradient reaching S_t and a_t = exp(g_eff_t); dg is 0 where a clamped token
 * had g > 0 (the derivative of torch.clamp(g, max=0), fast_gla.py:586).  strides[27] = (batch,
 * token, head) element strides of q, k, v, g, dout, dq, dk, dv, dg.  dq, dk, dv in d_dtype, dg in
 * dg_dtype; ds0 fp32 [B, H, Dk, Dv] or NULL.  Dk == Dv in {32, 64} (32 only for fp32 I/O); q, k, v,
 * g, dout rows 16-byte aligned, gradient rows 8-byte aligned.  workspace: at least
 * triune_hip_gla_prefill_bwd_workspace_size() bytes, 16-byte aligned.
 * flags: the prefill's, plus TRIUNE_FLAG_BWD_ACC_QKG / TRIUNE_FLAG_BWD_ACC_V: the call adds its
 * dq, dk, dg / dv to what those buffers hold instead of writing them (fp32 buffers only, else
 * TRIUNE_ERR_DTYPE), so a head wider than the kernels run as key/value blocks sums the blocks'
 * gradients in place.
 * Replaces: the backward of fast_chunk_gla (fast_gla.py:692-778) for T > 1. */
size_t triune_hip_gla_prefill_bwd_workspace_size(int64_t B, int64_t T, int64_t H, int Dk, int Dv, int flags);
int triune_hip_gla_prefill_bwd(const void* q, const void* k, const void* v, const void* g, int io_dtype, int g_dtype,
                               const void* dout, const int64_t* strides, const float* s0, const float* ds_final,
                               void* dq, void* dk, void* dv, int d_dtype, void* dg, int dg_dtype, float* ds0,
                               int64_t B, int64_t T, int64_t H, int Dk, int Dv, int flags, void* workspace,
                               size_t workspace_bytes, void* stream);

/* triune_hip_gla_prefill_varlen over a device-resident state pool: sequence i starts from
 * pool[slots[i]] and its final state is written back to pool[slots[i]] (in place).  pool: fp32
 * [n_slots, H, Dk, Dv], contiguous, 16-byte aligned; slots: int32 [n_seqs] on the device, distinct;
 * a slot outside [0, n_slots) starts from zero and is not written.  Same workspace as
 * triune_hip_gla_prefill_varlen. */
int triune_hip_gla_prefill_varlen_pool(const void* q, const void* k, const void* v, const void* g, int io_dtype,
                                       int g_dtype, const int64_t* strides, const int32_t* cu_seqlens,
                                       int64_t n_seqs, int64_t total_tokens, const int32_t* slots, float* pool,
                                       int64_t n_slots, void* o, int o_dtype, int64_t H, int Dk, int Dv, int flags,
                                       void* workspace, size_t workspace_bytes, void* stream);

/* Exclusive affine scan (FusedRecurrentScan forward), all tensors contiguous:
 *     s_all[b,h,n] = s ;  s = decay[b,h,n,:,None] * s + kv[b,h,n]      (s starts at init or 0)
 *     fin[b,h] = s after the last step
 * kv: [B, H, N, Dk, Dv] in kv_dtype; decay: [B, H, N, Dk] in decay_dtype; init: [B, H, Dk, Dv]
 * in init_dtype (or NULL for zero); s_all [B, H, N, Dk, Dv] and fin [B, H, Dk, Dv] in out_dtype
 * (the reference returns kv.dtype tensors, fast_gla.py:147-149).  Arithmetic in fp32.
 * s_all may alias kv when out_dtype == kv_dtype.  Dv must be a multiple of 4.
 * Replaces: FusedRecurrentScan.forward (fast_gla.py:109-149). */
int triune_hip_recurrent_scan_fwd(const void* kv, int kv_dtype, const void* decay, int decay_dtype, const void* init,
                                  int init_dtype, void* s_all, void* fin, int out_dtype, int64_t B, int64_t H,
                                  int64_t N, int Dk, int Dv, void* stream);

/* Backward of the exclusive scan (FusedRecurrentScan.backward), all tensors contiguous:
 *     d = d_fin ;  for n = N-1 .. 0:  d_kv[b,h,n] = d ;
 *         d_decay[b,h,n,i] = sum_j d[i,j] * s_all[b,h,n,i,j] ;  d = d_s_all[b,h,n] + decay[b,h,n,:,None] * d
 *     d_init[b,h] = d
 * d_s_all: [B, H, N, Dk, Dv] in d_s_all_dtype, d_fin: [B, H, Dk, Dv] in d_fin_dtype (either NULL =
 * zero); decay: [B, H, N, Dk] in decay_dtype; s_all: the forward's exclusive states in fp32
 * [B, H, N, Dk, Dv]; d_kv [B, H, N, Dk, Dv], d_decay [B, H, N, Dk] (summed over Dv) and d_init
 * [B, H, Dk, Dv] in out_dtype (the reference returns kv.dtype gradients, fast_gla.py:199-203).
 * Arithmetic in fp32.  Dv a multiple of 4, at most 256.
 * Replaces: FusedRecurrentScan.backward (fast_gla.py:151-203, kernel :67-107). */
int triune_hip_recurrent_scan_bwd(const void* d_s_all, int d_s_all_dtype, const void* d_fin, int d_fin_dtype,
                                  const void* decay, int decay_dtype, const float* s_all, void* d_kv, void* d_decay,
                                  void* d_init, int out_dtype, int64_t B, int64_t H, int64_t N, int Dk, int Dv,
                                  void* stream);

/* Gated DeltaNet forward, the reference's variant (fast_gla.py:781-836):
 *     u_t = v_t - S_{t-1}^T k_t ;  S_t = diag(exp(min(g_t,0))) S_{t-1} + beta_t . (k_t u_t^T) ;
 *     o_t = S_t^T q_t
 * beta: NULL with TRIUNE_BETA_NONE, else see the TRIUNE_BETA_* kinds (beta_dtype any dtype code).
 * strides[18] = (batch, token, head) element strides of q, k, v, g, beta, o.
 * s0 / s_final: fp32 [B, H, Dk, Dv] or NULL.  (Dk, Dv) in {(32,32), (64,64), (128,128)}.
 * Replaces: fast_chunk_gated_deltanet (fast_gla.py:839-904) for T > 1. */
int triune_hip_gdn_prefill(const void* q, const void* k, const void* v, const void* g, int io_dtype, int g_dtype,
                           const void* beta, int beta_dtype, int beta_kind, const int64_t* strides, const float* s0,
                           void* o, int o_dtype, float* s_final, int64_t B, int64_t T, int64_t H, int Dk, int Dv,
                           void* stream);

/* The same Gated DeltaNet forward in chunked WY/UT form (64-token chunks, MFMA, segment-parallel):
 * same arguments and results as triune_hip_gdn_prefill, plus a workspace of at least
 * triune_hip_gdn_prefill_chunked_workspace_size(B, T, H, Dk, Dv) bytes (16-byte aligned; 0 =
 * unsupported sizes).  Supported: (Dk, Dv) == (64, 64) with any io_dtype, and (128, 128) with
 * bf16 or fp16 I/O (fp32 I/O at 128 returns TRIUNE_ERR_DTYPE: use triune_hip_gdn_prefill);
 * beta_kind NONE, HEAD (any dtype), KEY or VALUE (fp32, [B, T, H, Dk] resp. [B, T, H, Dv] with the
 * strides given for beta).
 * Replaces: fast_chunk_gated_deltanet (fast_gla.py:839-904) for T > 1. */
size_t triune_hip_gdn_prefill_chunked_workspace_size(int64_t B, int64_t T, int64_t H, int Dk, int Dv);
int triune_hip_gdn_prefill_chunked(const void* q, const void* k, const void* v, const void* g, int io_dtype,
                                   int g_dtype, const void* beta, int beta_dtype, int beta_kind,
                                   const int64_t* strides, const float* s0, void* o, int o_dtype, float* s_final,
                                   int64_t B, int64_t T, int64_t H, int Dk, int Dv, void* workspace,
                                   size_t workspace_bytes, void* stream);

/* The chunked Gated DeltaNet forward for a gate that is one value per (token, head): the
 * scalar-decay form, which reaches the reference operator as g broadcast over the head dim
 * (g.expand(B, T, H, HD), read with its head-dim stride by the Triton kernel, fast_gla.py:464).
 * Same arguments and results as triune_hip_gdn_prefill_chunked except that g is [B, T, H]:
 * element (b, t, h) at strides[9..11] (non-negative, any token stride, element-aligned pointer),
 * and beta_kind is NONE or HEAD.  Workspace: at least
 * triune_hip_gdn_prefill_scalar_decay_workspace_size(B, T, H, Dk, Dv) bytes (16-byte aligned).
 * (Dk, Dv) == (64, 64).
 * Replaces: fast_chunk_gated_deltanet (fast_gla.py:839-904) for T > 1 with a broadcast gate. */
size_t triune_hip_gdn_prefill_scalar_decay_workspace_size(int64_t B, int64_t T, int64_t H, int Dk, int Dv);
int triune_hip_gdn_prefill_scalar_decay(const void* q, const void* k, const void* v, const void* g, int io_dtype,
                                        int g_dtype, const void* beta, int beta_dtype, int beta_kind,
                                        const int64_t* strides, const float* s0, void* o, int o_dtype,
                                        float* s_final, int64_t B, int64_t T, int64_t H, int Dk, int Dv,
                                        void* workspace, size_t workspace_bytes, void* stream);

/* Gradients of the Gated DeltaNet recurrence above (triune_hip_gdn_prefill's arithmetic, from s0)
 * for the upstream gradients dout (o's, [B, T, H, Dv] in dout_dtype, NULL = zero) and ds_final
 * (fp32 [B, H, Dk, Dv], NULL = zero).  strides[18] = (batch, token, head) element strides of q, k,
 * v, g, beta, dout.  Outputs, contiguous: dq, dk, dv [B, T, H, D] in io_dtype, dg [B, T, H, D] in
 * g_dtype (zero where g > 0: the clamp passes no gradient there), dbeta in beta_dtype ([B, T, H]
 * for TRIUNE_BETA_HEAD, [B, T, H, D] for KEY and VALUE), ds0 fp32 [B, H, D, D] or NULL.  Dk == Dv
 * in {64, 128}; q, k, v, g, dout (and a per-dim beta) rows 16-byte aligned.  Arithmetic in fp32:
 * the states are recomputed token by token from checkpoints.  workspace: at least
 * triune_hip_gdn_bwd_workspace_size(B, T, H, Dk, Dv, beta_kind) bytes, 16-byte aligned.
 * Replaces: autograd through fast_recurrent_gated_deltanet (fast_gla.py:781-836), the path
 * fast_chunk_gated_deltanet takes when a gradient is needed (fast_gla.py:885-904). */
size_t triune_hip_gdn_bwd_workspace_size(int64_t B, int64_t T, int64_t H, int Dk, int Dv, int beta_kind);
int triune_hip_gdn_bwd(const void* q, const void* k, const void* v, const void* g, int io_dtype, int g_dtype,
                       const void* beta, int beta_dtype, int beta_kind, const int64_t* strides, const float* s0,
                       const void* dout, int dout_dtype, const float* ds_final, void* dq, void* dk, void* dv,
                       void* dg, void* dbeta, float* ds0, int64_t B, int64_t T, int64_t H, int Dk, int Dv,
                       void* workspace, size_t workspace_bytes, void* stream);

/* GLA input pre-processing in place (VectorisedGLA's fused path): for every (b, t, h) row of HD
 * elements, q and k <- RoPE(normalize(elu(x) + 1)) with normalize(a) = a / sqrt(max(sum a^2,
 * 1e-12)) and RoPE pairing elements d and d + HD/2 (out[d] = a[d] cos[t][d] - a[d+HD/2] sin[t][d],
 * out[d+HD/2] = a[d+HD/2] cos[t][d+HD/2] + a[d] sin[t][d+HD/2]); g <- logsigmoid(g); v untouched.
 * qkv: [B, T, 3, H, HD] with element strides strides[0..3] = (batch, token, part, head); g:
 * [B, T, H, HD] with strides[4..6] = (batch, token, head); innermost stride 1, rows 16-byte
 * aligned.  cos/sin: [T, HD] rows cs_stride elements apart (used when use_rope != 0), dtype
 * cs_dtype.  HD in {32, 64, 128}; q/k/v/g share io_dtype.
 * Replaces: _fused_qkv_g_prep_inplace_kernel (triune/model/attention.py:14-79). */
int triune_hip_gla_qkvg_prep(void* qkv, void* g, int io_dtype, const int64_t* strides, const void* cos,
                             const void* sin, int cs_dtype, int64_t cs_stride, int use_rope, int64_t B, int64_t T,
                             int64_t H, int HD, void* stream);

/* One GLA decode step fused with the pre-processing above: qkvg [B, 4, H, HD] raw projections
 * (strides[0..2] = batch, part, head; parts q, k, v, g), cos/sin [HD] of the step's position; q,
 * k pre-processed as above, decay sigmoid(g) (= exp(logsigmoid(g))), then S <- diag(decay) S +
 * k v^T and o = S^T q.  state_in / state_out: contiguous [B, H, HD, HD] in state_dtype (fp32 or
 * io_dtype; state_in NULL = zero state, state_out NULL = state not stored, state_out may equal
 * state_in).  o: [B, H, HD] (o_strides = batch, head).  cs_dtype: fp32 or io_dtype.
 * Replaces: _fused_qkvg_decode_step_kernel (triune/model/attention.py:81-179). */
int triune_hip_gla_fused_decode_step(const void* qkvg, int io_dtype, const int64_t* strides, const void* cos,
                                     const void* sin, int cs_dtype, int use_rope, const void* state_in,
                                     void* state_out, int state_dtype, void* o, int o_dtype,
                                     const int64_t* o_strides, int64_t B, int64_t H, int HD, void* stream);

/* The same fused decode step over a state pool, in place: state_pool [n_slots, H, HD, HD] in
 * state_dtype (16-byte aligned for fp32, 8 for 16-bit), and batch row b reads and writes pool row
 * slots[b] (int32, device); a slot outside [0, n_slots) (a padded batch row) reads no state,
 * stores none and outputs zeros.  Other arguments as triune_hip_gla_fused_decode_step.
 * Replaces: _fused_qkvg_decode_step_kernel (triune/model/attention.py:81-179) on a serving
 * pool's rows, the per-session cache of triune/api/srsm.py:11-112 kept on the device. */
int triune_hip_gla_fused_decode_step_slots(const void* qkvg, int io_dtype, const int64_t* strides, const void* cos,
                                           const void* sin, int cs_dtype, int use_rope, void* state_pool,
                                           int state_dtype, const int32_t* slots, int64_t n_slots, void* o,
                                           int o_dtype, const int64_t* o_strides, int64_t B, int64_t H, int HD,
                                           void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TRIUNE_HIP_H */
