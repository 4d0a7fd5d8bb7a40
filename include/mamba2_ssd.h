/*
 * mamba2_ssd.h -- C ABI of the MI355X (gfx950) Mamba-2 SSD hot path.
 *
 * Every entry point takes raw device pointers to contiguous fp32 tensors in the
 * public layouts of the reference API, never allocates, and enqueues its work
 * on the given HIP stream (passed as void*, i.e. a hipStream_t; NULL = the null
 * stream).  Calls are reentrant; the only process-wide state is a thread-local
 * error message.  Status codes are 0 on success and negative on failure;
 * mamba2_ssd_last_error() returns the calling thread's last message.
 *
 * Layouts ([B,L,H,P,N,G] = batch, seqlen, nheads, headdim, dstate, ngroups):
 *   x, z, out, dout, dx, dz   [B, L, H, P]
 *   dt, ddt                   [B, L, H]
 *   A, dt_bias, dA, ddt_bias  [H]
 *   B, C, dB, dC              [B, L, G, N]
 *   D, dD                     [H] or [H, P] (MAMBA2_SSD_D_PER_CHANNEL)
 *   initial_states, final_state, dfinal_state, dinitial_states  [B, H, P, N]
 *
 * Reference interfaces replaced (So-cean/mamba-ascendc):
 *   mamba2_ssd_fwd      -- torch.ops.mamba_ascend.mamba2_ssd_fwd schema
 *                          (mamba_ascendc/csrc/register.cpp:175-179) and the
 *                          Python forward paths behind ascend_kernel.mamba2_ssd_fwd
 *                          (mamba_ascendc/python/ascend_kernel/ascend_kernel/mamba2.py:606-702)
 *   mamba2_ssd_bwd_m1   -- the M1 backward composition _chunk_mix_ssd_bwd_m1
 *                          (mamba2.py:1091-1658) reached from
 *                          _Mamba2SsdAutogradM1.backward (mamba2.py:1782-1838)
 *   mamba2_ssd_state_passing -- torch.ops.mamba_ascend.mamba2_ssd_state_passing
 *                          (register.cpp:89-90; op_host mamba2_ssd_state_passing.cpp:12-78),
 *                          fp32 chunk states; mamba2_ssd_state_passing_f16 its fp16 form
 *   mamba2_selective_state_update -- the single-token decode step
 *                          selective_state_update of the reference's Triton port
 *                          (mamba_triton_ascend/mamba2/ops/triton/selective_state_update.py:134-213)
 *   *_workspace_size    -- the ACLNN GetWorkspaceSize phase
 *                          (mamba_ascendc/csrc/utils/torch_aclnn_helper.h:536-546)
 */
#ifndef MAMBA2_SSD_H_
#define MAMBA2_SSD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MAMBA2_SSD_ABI_VERSION 5

/* status codes */
#define MAMBA2_SSD_OK 0
#define MAMBA2_SSD_ERR_INVALID_ARGUMENT (-1) /* bad pointer, shape or flag */
#define MAMBA2_SSD_ERR_UNSUPPORTED (-2)      /* valid but not implemented here */
#define MAMBA2_SSD_ERR_WORKSPACE (-3)        /* workspace missing or too small */
#define MAMBA2_SSD_ERR_LAUNCH (-4)           /* a HIP launch failed */

/* feature flags */
#define MAMBA2_SSD_DT_SOFTPLUS (1u << 0)
#define MAMBA2_SSD_HAS_D (1u << 1)
#define MAMBA2_SSD_D_PER_CHANNEL (1u << 2) /* D is [H, P] instead of [H] */
#define MAMBA2_SSD_HAS_Z (1u << 3)
#define MAMBA2_SSD_HAS_DT_BIAS (1u << 4)
#define MAMBA2_SSD_HAS_INITIAL (1u << 5)
/* forward: write chunk_states; backward: read them instead of recomputing
 * (headdim == dstate == 64 only) */
#define MAMBA2_SSD_SAVED_STATES (1u << 6)
/* packed sequences: seq_idx [B, L] gives every token's sequence id (the
 * seq_idx argument of the reference's Triton port,
 * mamba_triton_ascend/mamba2/ops/triton/ssd_combined.py:359-409);
 * forward: headdim 64 with dstate 64 or 128; backward: headdim = dstate = 64 */
#define MAMBA2_SSD_HAS_SEQ_IDX (1u << 7)
/* forward: also write the state at the end of every sequence of a batch-1
 * input split by cu_seqlens (ssd_combined.py:406-409, chunk_state_varlen);
 * chunk_size must be a multiple of 64 */
#define MAMBA2_SSD_VARLEN_STATES (1u << 8)

typedef struct Mamba2SsdShape {
    int64_t batch;
    int64_t seqlen;
    int64_t nheads;
    int64_t headdim;
    int64_t ngroups;
    int64_t dstate;
    int64_t chunk_size; /* logical chunk (results do not depend on it) */
} Mamba2SsdShape;

typedef struct Mamba2SsdFwdArgs {
    Mamba2SsdShape shape;
    uint32_t flags;
    float dt_limit_min; /* clamp of dt after bias/softplus; use 0 and INFINITY */
    float dt_limit_max; /* for the reference default (0, inf) */
    const float *x, *dt, *A, *B, *C;
    const float *D, *z, *dt_bias, *initial_states; /* NULL unless flagged */
    float *out;         /* [B, L, H, P] */
    float *final_state; /* [B, H, P, N] or NULL */
    float *pre_gate;    /* [B, L, H, P] y + D x before the z gate (written only
                           with HAS_Z; what the backward needs for dz), or NULL */
    float *chunk_states; /* [B, H, ceil(L / 64), P, N]: the state entering each
                            64-token chunk, for the backward; written iff
                            SAVED_STATES, else NULL (the reference's training
                            forward returns states_start the same way:
                            mamba2.py:228,322,408-418 return_states_start,
                            mamba_ascendc_ops/mamba2_ssd_chunk_mix/op_kernel/
                            mamba2_ssd_state_epilogue_train_states.cpp:15) */
    /* members below added in ABI 4 */
    const int32_t *seq_idx;    /* [B, L] iff HAS_SEQ_IDX, else NULL.  With e_k the id of
                                  64-token chunk k's last token (e_{-1} = 0): C_t.B_s
                                  counts only for equal ids, a token enters the state
                                  only if its id is e_k >= 0, the state carries over
                                  chunk k only if e_k == e_{k-1}, and a token reads the
                                  state entering its chunk only if its id is e_{k-1}.
                                  For non-negative, non-decreasing ids this is every
                                  sequence run on its own (the one with id 0 from
                                  initial_states) at any logical chunk size. */
    const int32_t *cu_seqlens; /* [nseqs + 1] token offsets iff VARLEN_STATES, else NULL */
    int64_t nseqs;
    float *varlen_states;      /* [nseqs, H, P, N] iff VARLEN_STATES, else NULL */
} Mamba2SsdFwdArgs;

typedef struct Mamba2SsdBwdArgs {
    Mamba2SsdShape shape;
    uint32_t flags;
    float dt_limit_min;
    float dt_limit_max;
    const float *x, *dt, *A, *B, *C;
    const float *D, *z, *dt_bias, *initial_states;
    const float *dout;         /* [B, L, H, P]; NULL means zero */
    const float *dfinal_state; /* [B, H, P, N]; NULL means zero */
    const float *pre_gate;     /* [B, L, H, P] from the forward; required iff HAS_Z */
    const float *chunk_states; /* [B, H, ceil(L / 64), P, N] from the forward;
                                  required iff SAVED_STATES, else NULL */
    float *dx, *ddt, *dA, *dB, *dC;
    float *dD, *dz, *ddt_bias, *dinitial_states; /* required iff the feature is flagged */
    /* member below added in ABI 4 */
    const int32_t *seq_idx;    /* [B, L] iff HAS_SEQ_IDX (the forward's ids), else NULL */
} Mamba2SsdBwdArgs;

/* Bytes of device workspace mamba2_ssd_fwd needs for this shape/flags
 * (VARLEN_STATES without SAVED_STATES adds the chunk states it reads). */
int mamba2_ssd_fwd_workspace_size(const Mamba2SsdShape *shape, uint32_t flags, size_t *bytes);

/* Forward: out (and final_state when non-NULL). */
int mamba2_ssd_fwd(const Mamba2SsdFwdArgs *args, void *workspace, size_t workspace_bytes,
                   void *stream);

/* Forward with a per-kernel event trace, for benchmarks and profilers.
 * events[] are caller-created hipEvent_t handles (passed as void*): events[0]
 * is recorded on the stream before the first kernel and events[i + 1] right
 * after kernel i.  On return *nkernels holds the number of kernels launched
 * and, when names is non-NULL, names[i] the (static) name of kernel i.
 * Replaces the stage decomposition the reference obtains from the NPU
 * profiler (benchmarks/mamba2_forward_npu_profile.py:36-112, 156-171). */
int mamba2_ssd_fwd_traced(const Mamba2SsdFwdArgs *args, void *workspace, size_t workspace_bytes,
                          void *stream, void *const *events, int nevents, const char **names,
                          int *nkernels);

/* Scratch size of mamba2_ssd_fwd_noalloc (40 MiB): enough for the segment
 * states of every forward plan whose scratch is only those (headdim 64 m with
 * dstate 64 or 128, any length). */
#define MAMBA2_SSD_NOALLOC_SCRATCH_BYTES (40u << 20)

/* Forward that allocates nothing and takes no workspace.  This entry point has
 * no counterpart in the reference; it is for callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc.  Same arguments, results and kernels as mamba2_ssd_fwd;
 * the scratch that call would take from its workspace (size given by
 * mamba2_ssd_fwd_workspace_size) comes from a static device array of
 * MAMBA2_SSD_NOALLOC_SCRATCH_BYTES that the library holds on each GPU it runs
 * on until the process ends (on the calling thread's current device, which
 * must be the device of `stream`).  A forward that needs more scratch returns
 * MAMBA2_SSD_ERR_WORKSPACE before any GPU work.  Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (two streams, or two host
 * threads, without ordering between them) race and must not be issued. */
int mamba2_ssd_fwd_noalloc(const Mamba2SsdFwdArgs *args, void *stream);

/* Bytes of device workspace mamba2_ssd_bwd_m1 needs for this shape/flags
 * (less with SAVED_STATES: the chunk states are not recomputed). */
int mamba2_ssd_bwd_m1_workspace_size(const Mamba2SsdShape *shape, uint32_t flags, size_t *bytes);

/* M1 backward: gradients of the forward for the given upstream gradients.
 * Supported: headdim == dstate == 64, fp32 contiguous, any seqlen and
 * chunk_size (the result does not depend on the logical chunk).  dx, ddt, dA,
 * dB, dC are always written; dD, dz, ddt_bias, dinitial_states when their
 * feature flag is set.  Deterministic: every reduction runs in a fixed order. */
int mamba2_ssd_bwd_m1(const Mamba2SsdBwdArgs *args, void *workspace, size_t workspace_bytes,
                      void *stream);

/* Backward with a per-kernel event trace (same contract as mamba2_ssd_fwd_traced). */
int mamba2_ssd_bwd_m1_traced(const Mamba2SsdBwdArgs *args, void *workspace,
                             size_t workspace_bytes, void *stream, void *const *events,
                             int nevents, const char **names, int *nkernels);

/* Inter-chunk state passing, in the reference's stage-op form:
 *   chunk_states [B, H, K, P, N] (read), chunk_log_decay [B, H, K] (sum of dt*A over
 *   each chunk), initial_states [B, H, P, N] or NULL;
 *   writes states_start [B, H, K, P, N] (may alias chunk_states) and final_state
 *   [B, H, P, N] (may be NULL):
 *     states_start[k] = S ; S = exp(chunk_log_decay[k]) * S + chunk_states[k]. */
int mamba2_ssd_state_passing(const float *chunk_states, const float *chunk_log_decay,
                             const float *initial_states, float *states_start,
                             float *final_state, int64_t batch, int64_t nheads,
                             int64_t nchunks, int64_t headdim, int64_t dstate, void *stream);

/* The same with fp16 chunk_states (IEEE binary16, [B, H, K, P, N]); the log
 * decays, initial_states, states_start and final_state stay fp32, and
 * states_start must not overlap chunk_states.  Replaces the FP16 branch of the
 * reference op (op_host mamba2_ssd_state_passing.cpp:19-23, chunkStatesHalf at
 * :58), which takes FP16 or FP32 chunk states and returns FP32 states. */
int mamba2_ssd_state_passing_f16(const void *chunk_states, const float *chunk_log_decay,
                                 const float *initial_states, float *states_start,
                                 float *final_state, int64_t batch, int64_t nheads,
                                 int64_t nchunks, int64_t headdim, int64_t dstate,
                                 void *stream);

/* ---- decode step ---------------------------------------------------------- */

/* dt [B, H], A [H], dt_bias [H] (the tied head-dim case, Mamba-2 decoding);
 * without it dt [B, H, P], A [H, P, N], dt_bias [H, P] */
#define MAMBA2_SSU_TIED (1u << 16)
/* the element strides in Mamba2SsuArgs.strides are set (else every input has the
 * contiguous layout of its shape) */
#define MAMBA2_SSU_STRIDES (1u << 17)

/* Element strides of the decode inputs (MAMBA2_SSU_STRIDES); any may be 0 (a
 * broadcast).  The innermost dimension of x, z (over P) and of B, C (over N) is
 * contiguous; B and C rows stay 16-byte aligned. */
typedef struct Mamba2SsuStrides {
    int64_t x_b, x_h;            /* x [B, H, P] */
    int64_t z_b, z_h;            /* z [B, H, P] */
    int64_t bc_b, bc_g;          /* B and C [B, G, N] (the same strides for both) */
    int64_t dt_b, dt_h, dt_p;    /* dt [B, H] (TIED: dt_p unused) or [B, H, P] */
    int64_t A_h, A_p, A_n;       /* A [H] (TIED: A_p, A_n unused) or [H, P, N] */
    int64_t bias_h, bias_p;      /* dt_bias [H] (TIED) or [H, P] */
    int64_t D_h, D_p;            /* D [H] or [H, P] (D_PER_CHANNEL) */
} Mamba2SsuStrides;

typedef struct Mamba2SsuArgs {
    int64_t batch, nheads, headdim, dstate, ngroups;
    uint32_t flags;     /* MAMBA2_SSU_TIED, MAMBA2_SSU_STRIDES, MAMBA2_SSD_DT_SOFTPLUS,
                           _HAS_D, _D_PER_CHANNEL (D [H, P], else [H]), _HAS_Z,
                           _HAS_DT_BIAS */
    float *state;       /* slots of [H, P, N] (contiguous within a slot), updated in place */
    int64_t state_slots;       /* number of slots (state batch) */
    int64_t state_slot_stride; /* floats between consecutive slots (>= H * P * N) */
    const int32_t *state_batch_indices; /* [B]: slot of each sequence; < 0 (or >= the
                                           slot count) = padding: no update, output 0;
                                           NULL = slot b */
    const float *x;     /* [B, H, P] */
    const float *dt;    /* [B, H] (TIED) or [B, H, P] */
    const float *A;     /* [H] (TIED) or [H, P, N] */
    const float *B, *C; /* [B, G, N] */
    const float *D;     /* [H] or [H, P], or NULL */
    const float *z;     /* [B, H, P] or NULL */
    const float *dt_bias; /* [H] (TIED) or [H, P], or NULL */
    float *out;         /* [B, H, P] */
    Mamba2SsuStrides strides; /* read iff MAMBA2_SSU_STRIDES (member added in ABI 4) */
} Mamba2SsuArgs;

/* One decode step: for each sequence b and head h, S = exp(A q) S + q x B^T
 * on its state slot and out = S C (+ D x) (* silu z), q = softplus?(dt + dt_bias).
 * dstate must be a multiple of 4 and at most 256; state, B, C (and an untied A)
 * 16-byte aligned.  No workspace; enqueued on `stream`. */
int mamba2_selective_state_update(const Mamba2SsuArgs *args, void *stream);

/* Thread-local message of the last failing call on this thread ("" if none). */
const char *mamba2_ssd_last_error(void);

/* MAMBA2_SSD_ABI_VERSION of the loaded library. */
int mamba2_ssd_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MAMBA2_SSD_H_ */
