// kernels.h -- parameter blocks and launchers of the gfx950 kernels (internal to libtriune_hip).
#pragma once

#include "common.h"

namespace triune {

struct TokTensor {
    const void* p;
    int64_t sb, st, sh;  // element strides: batch, token, head (innermost stride is 1)
    int64_t extent;      // bytes readable from p (one past the last element)
};

struct PrefillParams {
    TokTensor q, k, v, g;
    void* o;
    int64_t o_sb, o_st, o_sh;
    int g_dt, o_dt;
    const float* s0;       // [n_seqs, H, Dk, Dv] or null
    float* ws_state;       // [n_work, H, Dk, Dv]
    float* ws_gamma;       // [n_work, H, Dk]
    int64_t n_seqs, H, T;  // T: dense sequence length
    int Dk, Dv;
    int P;                 // varlen: chunks per segment
    int nseg_dense;        // dense: segments per sequence (near-equal chunk counts)
    int varlen;
    const int32_t* cu;     // varlen: [n_seqs + 1] token offsets (device)
    const int32_t* seg_off;// varlen: [n_seqs + 1] segment offsets (device, from plan kernel)
    int flags;             // bit 0: the last token of each sequence keeps g unclamped
    // Gated DeltaNet (chunked): write strength beta per token (BETA_HEAD, strides b_sb/b_st/b_sh,
    // dtype beta_dt), per (token, key dim) (BETA_KEY) or per (token, value dim) (BETA_VALUE), both
    // fp32 in `kb`, or none.
    const void* beta;
    int beta_dt, beta_kind;
    int64_t b_sb, b_st, b_sh;
    TokTensor kb;
    float* ws_m;           // GDN: [n_work, H] slots of the segment transition matrices as bf16 parts
    float* ws_spare;       // [n_seqs, H, Dk, Dv] sink for the segment scan's padding steps
    // GDN with beta per value column: one segment per sequence, the output kernel walks it from
    // s0 (or zero) and writes the final state here ([n_seqs, H, Dk, Dv] fp32, or null).
    float* seq_final;
    int gdn_whole;
    // Prefill with the VectorisedGLA pre-processing applied in stage 1 (q, k, g raw projections):
    // fp32 RoPE tables [T, Dk] (row = token of the sequence, token stride cs.st; sb = sh = 0)
    TokTensor cs, sn;
    int use_rope;
};

struct ScanParams {
    const void* kv;
    int kv_dt;
    int64_t kv_so, kv_sh, kv_sn;
    const void* dec;  // decay factor or log-decay, per (n, dim)
    int dec_dt;
    int dec_is_log;
    int64_t d_so, d_sh, d_sn;
    const float* init;  // fp32 or null; [o][h] stride i_so, i_sh, contiguous Dk*Dv
    int64_t i_so, i_sh;
    const void* init_any;  // alternative init in init_dt (FusedRecurrentScan), or null
    int init_dt;
    void* s_all;
    int sa_dt;
    int64_t sa_so, sa_sh, sa_sn;
    void* fin;
    int fin_dt;
    int64_t f_so, f_sh;
    int64_t n_outer, H;
    int Dk, Dv;
    int64_t N;              // steps when seg_off is null
    const int32_t* seg_off; // per outer o: steps N_o = seg_off[o+1]-seg_off[o], first step seg_off[o]
    // Optional row indirection of init and fin (prefill carry only): outer o reads its initial
    // state from row slots[o] of init and writes its final state to row slots[o] of fin; a slot
    // outside [0, n_slots) starts from zero and is not written.
    const int32_t* slots;
    int64_t n_slots;
};

// Gradients of the dense chunked GLA prefill (Dk == Dv == D).  f carries the forward inputs, the
// segment plan and the forward workspaces (ws_state: carried-in state per segment after the
// forward scan; ws_gamma: summed log-decay per segment).
struct BwdParams {
    PrefillParams f;
    TokTensor dout;        // upstream gradient of o, in the I/O dtype, [B, T, H, D]
    void* dq; void* dk; void* dv; void* dg;
    int64_t dq_sb, dq_st, dq_sh, dk_sb, dk_st, dk_sh, dv_sb, dv_st, dv_sh, dg_sb, dg_st, dg_sh;
    int d_dt;              // dtype of dq, dk, dv
    int dg_dt;             // dtype of dg
    int acc;               // bit 0: dq, dk, dg added into their (fp32) buffers; bit 1: dv likewise
    float* ws_chunk;       // [B, H, nchunks, D, D] state at the start of every chunk
    float* ws_r;           // [n_work, H, D, D] segment maps R, then the gradient reaching each segment's end
    float* ws_send;        // [n_work, H, D, D] state at each segment's end
    int64_t nchunks;       // chunks per sequence
};

// Backward of the exclusive scan (FusedRecurrentScan), all tensors contiguous:
// d_s_all / s_all / d_kv [o][h][n][Dk][Dv], decay / d_decay [o][h][n][Dk], d_fin / d_init [o][h][Dk][Dv].
struct ScanBwdParams {
    const void* d_s_all;  // or null (zero)
    int dsa_dt;
    const void* d_fin;    // or null (zero)
    int df_dt;
    const void* dec;      // decay factors
    int dec_dt;
    const float* s_all;   // the forward's exclusive states, fp32
    void* d_kv;
    void* d_dec;
    void* d_init;
    int out_dt;
    int64_t n_outer, H, N;
    int Dk, Dv;
};

struct DecodeParams {
    const void* q; const void* k; const void* v; const void* g;
    int io_dt, g_dt, o_dt;
    int64_t q_sb, q_sh, k_sb, k_sh, v_sb, v_sh, g_sb, g_sh, o_sb, o_sh;  // element strides
    const float* state_in;  // [B, H, Dk, Dv]
    float* state_out;       // may equal state_in
    const int32_t* slots;   // optional: state row of batch b is slots[b] (state pool), or null
    int64_t n_state_rows;   // rows of state_in / state_out; a slot outside [0, n_state_rows) is skipped
    void* o;
    int64_t B, H;
};

enum BetaKind : int { BETA_NONE = 0, BETA_HEAD = 1, BETA_KEY = 2, BETA_VALUE = 3 };

struct GdnParams {
    const void* q; const void* k; const void* v; const void* g; const void* beta;
    int io_dt, g_dt, beta_dt, o_dt, beta_kind;
    int64_t q_sb, q_st, q_sh, k_sb, k_st, k_sh, v_sb, v_st, v_sh, g_sb, g_st, g_sh;
    int64_t b_sb, b_st, b_sh;  // beta strides (batch, token, head); innermost 1 for per-dim kinds
    int64_t o_sb, o_st, o_sh;
    void* o;
    const float* s0;   // [B, H, Dk, Dv] or null
    float* s_final;    // [B, H, Dk, Dv] or null
    int64_t B, T, H;
};

// Gradients of the Gated DeltaNet reference variant (gdn_bwd.hip); D = Dk = Dv in {64, 128}.
struct GdnBwdParams {
    GdnParams f;             // forward inputs and shapes; f.s0 the initial state or null
    const void* dout;        // [B, T, H, Dv] upstream gradient of o (element strides below) or null
    int do_dt;
    int64_t do_sb, do_st, do_sh;
    const float* dsf;        // [B, H, D, D] upstream gradient of the final state or null
    float* ckpt;             // [B, H, NC, D, D] state before tokens 0, L, 2L, ...
    float* part;             // [NQ][NSL][B, T, H, D] per-slice sums over columns: dq, dk, dg, key-beta
    float* part_bh;          // [NSL][B, T, H] head-beta partials
    void* dv;                // [B, T, H, D] contiguous, io dtype
    void* dbeta_v;           // value beta: [B, T, H, D] contiguous in dbeta_dt
    int dbeta_dt;
    float* ds0;              // [B, H, D, D] or null
    int64_t nc;              // sub-chunks per sequence
    int L;                   // tokens per sub-chunk (gdn_bwd_chunk_tokens)
    // Segments of segc sub-chunks walked in parallel (nseg > 1; beta per value column keeps one):
    // [B, H, NSEG, D, D] fp32 each
    int64_t nseg, segc;
    // gdn_bwd_kernel walks coarser segments of bsegr of those (bsegc = bsegr * segc sub-chunks)
    int64_t bsegc, bsegr;
    float* seg_m;            // forward map of segment s: S_end = M_s S_start + N_s
    float* seg_n;            // N_s, the segment's end state from zero
    float* seg_dl;           // gradient reaching the state before segment s, walked from zero
    float* seg_de;           // gradient reaching the last state of segment s
};

// GLA input pre-processing (in place): q, k in qkv [B, T, 3, H, HD] (element strides sb, st, sp
// between the q/k/v parts, sh), g [B, T, H, HD]; cos/sin [T, HD] rows cs_st apart.
struct PrepParams {
    void* qkv;
    int64_t qkv_sb, qkv_st, qkv_sp, qkv_sh;
    void* g;
    int64_t g_sb, g_st, g_sh;
    const void* cos;
    const void* sin;
    int64_t cs_st;
    int use_rope;
    int64_t B, T, H;
};

// Decode step fused with the pre-processing: qkvg [B, 4, H, HD] (element strides x_sb, x_sp, x_sh),
// cos/sin [HD], state [B, H, HD, HD] contiguous (in: null = zero state; out: null = not stored).
struct FusedDecodeParams {
    const void* qkvg;
    int64_t x_sb, x_sp, x_sh;
    const void* cos;
    const void* sin;
    int use_rope, has_init, save_final;
    const void* state_in;
    void* state_out;
    void* o;
    int o_dt;
    int64_t o_sb, o_sh;
    int64_t B, H;
    int max_blocks;  // grid cap (blocks then walk several rows)
    // Optional state pool: row (b, h) reads and writes state row slots[b] * H + h of state_in /
    // state_out; a slot outside [0, n_state_rows) reads no state, stores none and outputs zeros.
    const int32_t* slots;
    int64_t n_state_rows;
};

// Control block of the single-launch prefill (gla_onepass.hip): hdr[0] epoch, hdr[1] workgroups of
// the running call that have read the epoch (back to zero when all have), hdr[2] error bits (1: a
// wait for an earlier chunk pair ran out; 2: a pair's map was written on another XCD than its
// reader's); flags[bh * npair + p] = the epoch + 1 of the call that published chunk pair p of
// (sequence, head) bh (low 32 bits) and the XCD its workgroup ran on (high 32 bits).
struct OnePassCtl {
    uint32_t* hdr;
    uint64_t* flags;
    int64_t nch;    // chunks per sequence
    int64_t npair;  // chunk pairs per sequence: ceil(nch / 2), one workgroup each
    int64_t nh8;    // (sequence, head) pairs per XCD: ceil(B * H / 8)
};

hipError_t launch_recurrent_scan(const ScanParams& a, hipStream_t stream);
hipError_t launch_recurrent_scan_bwd(const ScanBwdParams& a, hipStream_t stream);
bool gla_bwd_supported(int D, int io_dt);
hipError_t launch_gla_bwd_state(const BwdParams& a, int64_t n_work, int io_dt, hipStream_t stream);
hipError_t launch_gla_bwd_chunk(const BwdParams& a, int64_t n_work, int io_dt, hipStream_t stream);
hipError_t launch_gla_prep(const PrepParams& a, int HD, int io_dt, int cs_dt, hipStream_t stream);
hipError_t launch_gla_fused_decode(const FusedDecodeParams& a, int HD, int io_dt, int cs_dt, int s_dt,
                                   hipStream_t stream);
hipError_t launch_gla_decode(const DecodeParams& a, int Dk, int Dv, int max_blocks, hipStream_t stream);
hipError_t launch_gdn_tokenwise(const GdnParams& a, int Dk, int Dv, hipStream_t stream);
// T == 1 of many rows (Dk = Dv = D in {64, 128}; q, k, g, v rows and beta vector-aligned, beta fp32)
hipError_t launch_gdn_decode(const GdnParams& a, int D, int max_blocks, hipStream_t stream);
// GDN backward: checkpoint forward + reverse walk (part, part_bh, ckpt sized by the caller), then
// the per-slice sums are added by launch_gdn_slice_sum.
int gdn_bwd_chunk_tokens(int D, int64_t waves, int64_t cus);
int gdn_bwd_col_slices(int D);
hipError_t launch_gdn_bwd(const GdnBwdParams& p, int D, hipStream_t stream);
hipError_t launch_gdn_slice_sum(const float* src, int nsl, int64_t stride, int64_t n, void* out, int dt,
                                hipStream_t stream);
// Prefill: K1 segment states, K2 scan, K3 outputs (and, for varlen, K0 plan).
hipError_t launch_gla_seg_state(const PrefillParams& a, int64_t n_work, int io_dt, hipStream_t stream);
// ev0 / ev1: if not null, events stamped with the output kernel's own start and end.
hipError_t launch_gla_seg_output(const PrefillParams& a, int64_t n_work, int io_dt, hipStream_t stream,
                                 hipEvent_t ev0 = nullptr, hipEvent_t ev1 = nullptr);
hipError_t launch_gla_varlen_plan(const int32_t* cu, int64_t n_seqs, int P, int32_t* seg_off, hipStream_t stream);
hipError_t launch_gdn_seg_mn(const PrefillParams& a, int64_t n_work, int io_dt, hipStream_t stream);
hipError_t launch_gdn_seg_scan(const PrefillParams& a, float* s_final, int io_dt, hipStream_t stream);
hipError_t launch_gdn_seg_out(const PrefillParams& a, int64_t n_work, int io_dt, hipStream_t stream);
int gdn_seg_out_blocks_per_cu(int io_dt, bool ck, int D);
// Scalar-gate chunked GDN (gdn_scalar.hip): g holds one log-decay per (token, head); same
// workspace layout and segment scan as the per-key-dim kernels.
hipError_t launch_gdn_sg_seg_mn(const PrefillParams& a, int64_t n_work, int io_dt, hipStream_t stream);
hipError_t launch_gdn_sg_seg_out(const PrefillParams& a, int64_t n_work, int io_dt, hipStream_t stream);
int gdn_sg_seg_out_blocks_per_cu(int io_dt, bool ck);
bool prefill_shape_supported(int Dk, int Dv);
bool prefill_dtype_supported(int Dk, int Dv, int io_dt);
// the segment-state kernel that also pre-processes q, k, g in place (gla_prefill_prep.hip)
bool prefill_prep_supported(int D, int io_dt);
hipError_t launch_gla_prep_seg_state(const PrefillParams& a, int64_t n_work, int io_dt, hipStream_t stream);
int gla_seg_output_blocks_per_cu(int Dk, int Dv, bool ck);
// Single-launch prefill (one workgroup per two 64-token chunks, Dk = Dv = 64, 16-bit I/O; prep: q,
// k, g raw projections pre-processed in place).  Every workgroup of the grid must be resident at once.
unsigned gla_onepass_grid(int64_t BH, int64_t npair);
int gla_onepass_max_pairs();
int gla_onepass_blocks_per_cu();
bool gla_onepass_dtypes_ok(int io_dt, int g_dt, bool prep);
hipError_t launch_gla_onepass(const PrefillParams& a, const OnePassCtl& c, int io_dt, bool prep, hipStream_t stream,
                              hipEvent_t ev0 = nullptr, hipEvent_t ev1 = nullptr);

}  // namespace triune
