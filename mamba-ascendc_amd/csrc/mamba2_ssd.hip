// C ABI of the Mamba-2 SSD hot path (declarations in include/mamba2_ssd.h).
//
// Host side of the library: argument validation (the checks of the reference
// host wrappers, mamba_ascendc/csrc/ops/mamba2_ssd_fwd/op_host/mamba2_ssd_fwd.cpp:15-136),
// workspace sizing, and kernel launches on the caller's stream.  Nothing here
// allocates device memory.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "../../include/mamba2_ssd.h"
#include "ssd_bwd_fused.h"
#include "ssd_bwd_kernels.h"
#include "ssd_decode.h"
#include "ssd_fwd_fused.h"
#include "ssd_fwd_kernels.h"
#include "ssd_fwd_wide.h"
#include "ssd_launch.h"
#include "ssd_varlen.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int ok() {
    g_err[0] = '\0';
    return MAMBA2_SSD_OK;
}

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

constexpr uint32_t kKnownFlags = MAMBA2_SSD_DT_SOFTPLUS | MAMBA2_SSD_HAS_D |
                                 MAMBA2_SSD_D_PER_CHANNEL | MAMBA2_SSD_HAS_Z |
                                 MAMBA2_SSD_HAS_DT_BIAS | MAMBA2_SSD_HAS_INITIAL |
                                 MAMBA2_SSD_SAVED_STATES | MAMBA2_SSD_HAS_SEQ_IDX |
                                 MAMBA2_SSD_VARLEN_STATES;

int check_shape(const Mamba2SsdShape *s, uint32_t flags) {
    if (!s) return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "shape is NULL");
    if (flags & ~kKnownFlags) return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "unknown flag bits 0x%x", flags);
    if ((flags & MAMBA2_SSD_D_PER_CHANNEL) && !(flags & MAMBA2_SSD_HAS_D))
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "D_PER_CHANNEL set without HAS_D");
    if (s->batch <= 0 || s->seqlen < 0 || s->nheads <= 0 || s->headdim <= 0 || s->ngroups <= 0 ||
        s->dstate <= 0)
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT,
                    "non-positive dimension (B=%lld L=%lld H=%lld P=%lld G=%lld N=%lld)",
                    (long long)s->batch, (long long)s->seqlen, (long long)s->nheads,
                    (long long)s->headdim, (long long)s->ngroups, (long long)s->dstate);
    if (s->chunk_size <= 0)
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "chunk_size must be positive, got %lld",
                    (long long)s->chunk_size);
    if (s->nheads % s->ngroups)
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "nheads=%lld not divisible by ngroups=%lld",
                    (long long)s->nheads, (long long)s->ngroups);
    if (s->batch > 65535 || s->nheads > 65535)
        return fail(MAMBA2_SSD_ERR_UNSUPPORTED, "batch and nheads must be <= 65535");
    // the chunk kernels address a chunk's 64 token rows with 32-bit byte
    // offsets from the chunk start
    if (s->nheads * s->headdim > (int64_t)0x7fffffff / (4 * ssd::kChunk) ||
        s->ngroups * s->dstate > (int64_t)0x7fffffff / (4 * ssd::kChunk))
        return fail(MAMBA2_SSD_ERR_UNSUPPORTED,
                    "token rows too wide: nheads*headdim=%lld and ngroups*dstate=%lld must be <= %lld",
                    (long long)(s->nheads * s->headdim), (long long)(s->ngroups * s->dstate),
                    (long long)((int64_t)0x7fffffff / (4 * ssd::kChunk)));
    return MAMBA2_SSD_OK;
}

int64_t nchunks(const Mamba2SsdShape *s) { return (s->seqlen + ssd::kChunk - 1) / ssd::kChunk; }

// Forward plan.  headdim = 64 with dstate = 64 runs the fused segment-serial
// kernel k_fwd_seg, dstate = 128 its wide form k_fwd_wide (two workgroups per
// head, 32 channels each).  With fewer than kMinStreams (b, h, half) streams
// the sequence is cut into segments so the full pass still has about that many
// workgroups: one per CU (it holds a CU's LDS), in one round, so each pays its
// pipeline fill once (C4 [4,2048,16,64,64]: 64 streams; 4 segments of 8 chunks
// ran the full pass in 30 us, 16 segments of 2 chunks in 45 us).  The
// state-only pass that gives each segment's entering state runs on kPreMult
// times finer segments (it fits two workgroups per CU), and full segment s
// starts at the boundary of pre-segment s * kPreMult.  A cut costs two
// launches (the state-only pass and the segment recurrence, about 15 us
// together), so it is made only where it saves at least kMinSavedChunks
// chunk steps of about 3 us each.
#ifndef SSD_MIN_STREAMS
#define SSD_MIN_STREAMS 256
#endif
#ifndef SSD_PRE_MULT
#define SSD_PRE_MULT 2
#endif
constexpr int64_t kMinStreams = SSD_MIN_STREAMS;
constexpr int64_t kPreMult = SSD_PRE_MULT;
// Full segments of at most this many chunks take pre-segments of the same
// length (factor 1): the state-only pass over a few chunks costs mostly its
// pipeline fill, so halving its steps gains less than the full pass loses
// folding twice the entries.  C4 [4,2048,16,64,64] (segments of 8): forward
// 0.0492 -> 0.0470 ms; C2 (16) at factor 1 0.0700 -> 0.0770 ms and C5 (64)
// 0.249 -> 0.257-0.266 ms, so longer segments keep kPreMult.
constexpr int64_t kShortSegment = 8;
constexpr int64_t kMinSavedChunks = 6;
// With at most this many pre-segments before the last full segment, each full
// segment folds the pre-segment contributions onto the initial states in its
// own prologue (independent loads, a few us) instead of a separate segment
// recurrence launch (k_state_pass, about 6 us plus a launch gap at C4).
constexpr int64_t kFoldMax = 12;
// Heads per group from which the dstate-128 forward reads C . B^T from a
// per-chunk precompute (k_chunk_cb) instead of forming it per workgroup: the
// precompute (a launch, B and C read, the products written) pays off when 16
// or more workgroups share each product (C5, 32 heads per group: 0.250 ->
// 0.242 ms; C2, 4 heads per group: 0.072 -> 0.080 ms, so not there).
constexpr int64_t kMinCbHeads = 8;

struct FwdPlan {
    bool fused = false;
    int nseg = 1, M = 1, nsplit = 1;     // nsplit: workgroups per head (2 for dstate 128)
    int nseg_pre = 1, M_pre = 1, mult = 1; // segments of the state-only pass (nseg > 1)
    bool fold = false;                     // full segments fold the pre-segments themselves
    bool cb = false;                     // dstate 128: C . B^T per (b, g, chunk) formed once
    size_t cb_off = 0;                   // workspace offset of those products [B, G, K, 64, 64]
    size_t seg_state = 0, seg_decay = 0; // workspace offsets (fused, nseg > 1)
    size_t states = 0;                   // chunk states for VARLEN_STATES without SAVED_STATES
    size_t ws = 0;
};

bool fused_shape(const Mamba2SsdShape *s) {
    return s->headdim == 64 && (s->dstate == 64 || s->dstate == 128);
}

// A head of dim 64 m (m > 1) with dstate 64 or 128 runs the fused kernels as m
// heads of dim 64: the public layouts of x, z, out, D [H, P] and the initial
// and final states are the same memory read as [.., H m, 64, ..]; dt, A,
// dt_bias and a per-head D are read for head h / m.  (Saved chunk states and
// varlen states keep headdim 64: their layout would differ.)
int head_split(const Mamba2SsdShape *s) {
    return s->headdim > 64 && s->headdim % 64 == 0 && (s->dstate == 64 || s->dstate == 128)
               ? (int)(s->headdim / 64)
               : 1;
}

Mamba2SsdShape fused_view(const Mamba2SsdShape *s) {
    Mamba2SsdShape v = *s;
    const int m = head_split(s);
    v.nheads *= m;
    v.headdim /= m;
    return v;
}

FwdPlan fwd_plan(const Mamba2SsdShape *s, uint32_t flags, bool allow_cb = true) {
    FwdPlan pl;
    if (s->seqlen == 0) return pl;
    const int64_t K = nchunks(s), streams = s->batch * s->nheads;
    const size_t pn = (size_t)s->headdim * s->dstate;
    if (fused_shape(s)) {
        pl.fused = true;
        pl.nsplit = (int)(s->dstate / 64);
        const int64_t wstreams = streams * pl.nsplit;
        int64_t nseg = wstreams >= kMinStreams ? 1 : (kMinStreams + wstreams - 1) / wstreams;
        nseg = nseg < K ? nseg : K;
        if (K - (K + nseg - 1) / nseg < kMinSavedChunks) nseg = 1;
        if (nseg > 1) {
            // full segments of M = mult * M_pre chunks, pre-segments of M_pre
            const int64_t Mt = (K + nseg - 1) / nseg;
            const int64_t mult = Mt <= kShortSegment ? 1 : (kPreMult < Mt ? kPreMult : Mt);
            const int64_t Mp = (Mt + mult - 1) / mult;
            pl.mult = (int)mult;
            pl.M_pre = (int)Mp;
            pl.M = (int)(mult * Mp);
            pl.nseg = (int)((K + pl.M - 1) / pl.M);
            pl.nseg_pre = (int)((K + Mp - 1) / Mp);
            pl.fold = (int64_t)(pl.nseg - 1) * pl.mult <= kFoldMax;
            // folded, only the pre-segments before the last full segment are read
            if (pl.fold) pl.nseg_pre = (pl.nseg - 1) * pl.mult;
        } else {
            pl.M = (int)K;
        }
        size_t off = 0;
        if (pl.nseg > 1) {
            const size_t units = (size_t)streams * pl.nseg_pre;
            pl.seg_state = off;
            off += align256(units * pn * sizeof(float));
            pl.seg_decay = off;
            off += align256(units * sizeof(float));
        }
        if ((flags & MAMBA2_SSD_VARLEN_STATES) && !(flags & MAMBA2_SSD_SAVED_STATES)) {
            pl.states = off;
            off += align256((size_t)streams * K * pn * sizeof(float));
        }
        // dstate 128 with kMinCbHeads or more heads per group: the 2 R
        // workgroups of a group's chunk read one C . B^T (16 KB) instead of
        // each forming it (about 45% of k_fwd_wide's matrix work)
        if (allow_cb && pl.nsplit == 2 && s->nheads / s->ngroups >= kMinCbHeads) {
            pl.cb = true;
            pl.cb_off = off;
            off += align256((size_t)s->batch * s->ngroups * K * 64 * 64 * sizeof(float));
        }
        pl.ws = off;
    }
    return pl;
}

// allow_cb = false: the least workspace the forward runs with (without the
// C . B^T precompute, which is only a speed-up)
// Shapes the fused kernels take after zero padding: a headdim that is not a
// multiple of 64 (padded up to one, the heads then split as usual) and/or a
// dstate below 64 or between 64 and 128 (padded to 64 or 128), for the plain
// forward (no saved chunk states, varlen states or packed sequences, whose
// layouts would change).  The padded channels of x and z and the padded state
// columns of B, C and the initial states are zero, so every padded product
// term is an exact zero: the padded problem's output restricted to the real
// channels, and its final state to the real rows and columns, are the
// forward's (the extra channels come out zero and are dropped).  The
// reference runs such shapes (multiples of 16 with P N <= 8192) on its BMM
// route (mamba2.py:30-44, 429-557); here they reach the MFMA kernels instead
// of the per-row token recurrence.
struct PadPlan {
    bool on = false;
    Mamba2SsdShape ps{};               // the padded shape
    bool pad_p = false, pad_n = false; // which dimensions change
    // workspace offsets: x, z (P padded), B, C (N padded), per-channel D,
    // initial states, out and pre_gate (P padded), final state, inner workspace
    size_t x = 0, z = 0, b = 0, c = 0, d = 0, init = 0, out = 0, pre = 0, fin = 0, inner = 0, total = 0;
};

size_t fwd_ws_bytes(const Mamba2SsdShape *s, uint32_t flags, bool allow_cb = true);

PadPlan pad_plan(const Mamba2SsdShape *s, uint32_t f, bool allow_cb) {
    PadPlan pp;
    const uint32_t layout_flags = MAMBA2_SSD_SAVED_STATES | MAMBA2_SSD_VARLEN_STATES | MAMBA2_SSD_HAS_SEQ_IDX;
    if (s->seqlen == 0 || fused_shape(s) || head_split(s) > 1 || s->dstate > 128 || (f & layout_flags))
        return pp;
    pp.on = true;
    pp.ps = *s;
    pp.ps.headdim = (s->headdim + 63) / 64 * 64;
    pp.ps.dstate = s->dstate <= 64 ? 64 : 128;
    pp.pad_p = pp.ps.headdim != s->headdim;
    pp.pad_n = pp.ps.dstate != s->dstate;
    const size_t blh = (size_t)s->batch * s->seqlen * s->nheads, blg = (size_t)s->batch * s->seqlen * s->ngroups;
    const size_t bh = (size_t)s->batch * s->nheads, P = pp.ps.headdim, N = pp.ps.dstate;
    size_t off = 0;
    auto take = [&](size_t &at, size_t floats) {
        at = off;
        off += align256(floats * sizeof(float));
    };
    if (pp.pad_p) take(pp.x, blh * P);
    if (pp.pad_p && (f & MAMBA2_SSD_HAS_Z)) take(pp.z, blh * P);
    if (pp.pad_n) {
        take(pp.b, blg * N);
        take(pp.c, blg * N);
    }
    if (pp.pad_p && (f & MAMBA2_SSD_D_PER_CHANNEL)) take(pp.d, (size_t)s->nheads * P);
    if (f & MAMBA2_SSD_HAS_INITIAL) take(pp.init, bh * P * N);
    if (pp.pad_p) take(pp.out, blh * P);
    if (pp.pad_p && (f & MAMBA2_SSD_HAS_Z)) take(pp.pre, blh * P);
    take(pp.fin, bh * P * N);
    pp.inner = off;
    pp.total = off + fwd_ws_bytes(&pp.ps, f, allow_cb);
    return pp;
}

size_t fwd_ws_bytes(const Mamba2SsdShape *s, uint32_t flags, bool allow_cb) {
    const PadPlan pp = pad_plan(s, flags, allow_cb);
    if (pp.on) return pp.total;
    const Mamba2SsdShape v = fused_view(s);
    return fwd_plan(&v, flags, allow_cb).ws;
}

// Optional per-kernel event trace: events[0] is recorded before the first
// kernel and events[i + 1] right after kernel i, all on the launch stream.
struct Trace {
    void *const *events = nullptr;
    int capacity = 0;
    int used = 0;
    const char **names = nullptr; // kernel name of stage i (static strings)
};

int record(Trace *tr, hipStream_t st, const char *name) {
    if (!tr || !tr->events) return MAMBA2_SSD_OK;
    if (tr->used >= tr->capacity)
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "trace needs more than %d events",
                    tr->capacity);
    hipError_t e = hipEventRecord((hipEvent_t)tr->events[tr->used], st);
    if (e != hipSuccess)
        return fail(MAMBA2_SSD_ERR_LAUNCH, "hipEventRecord failed: %s", hipGetErrorString(e));
    if (name && tr->names && tr->used > 0) tr->names[tr->used - 1] = name;
    ++tr->used;
    return MAMBA2_SSD_OK;
}

int launch_status(const char *what, Trace *tr = nullptr, hipStream_t st = nullptr) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return fail(MAMBA2_SSD_ERR_LAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
    return record(tr, st, what);
}

}  // namespace

extern "C" {

int mamba2_ssd_abi_version(void) { return MAMBA2_SSD_ABI_VERSION; }

const char *mamba2_ssd_last_error(void) { return g_err; }

int mamba2_ssd_fwd_workspace_size(const Mamba2SsdShape *shape, uint32_t flags, size_t *bytes) {
    if (int rc = check_shape(shape, flags)) return rc;
    if (!bytes) return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "bytes is NULL");
    *bytes = fwd_ws_bytes(shape, flags);
    return ok();
}

}  // extern "C"

namespace {

int fwd_impl(const Mamba2SsdFwdArgs *a, void *workspace, size_t workspace_bytes, void *stream, Trace *tr);

// [outer, rs, cs] -> [outer, rd, cd] with zero fill (or the padding cut off)
int pad_copy(const float *src, int64_t outer, int64_t rs, int64_t cs, float *dst, int64_t rd, int64_t cd,
             hipStream_t st, Trace *tr) {
    const int64_t total = outer * rd * cd;
    const int64_t blocks = std::min<int64_t>((total + ssd::kPadThreads - 1) / ssd::kPadThreads, 8192);
    hipLaunchKernelGGL(ssd::k_pad_copy, dim3((unsigned)std::max<int64_t>(blocks, 1)), dim3(ssd::kPadThreads), 0, st,
                       src, outer, (int)rs, (int)cs, dst, (int)rd, (int)cd);
    return launch_status("k_pad_copy", tr, st);
}

// The forward on a zero-padded copy of the problem (PadPlan), then the real
// channels of out / pre_gate and the real rows and columns of the final state
// copied back.
int fwd_padded(const Mamba2SsdFwdArgs *a, const PadPlan &pp, char *ws, size_t have, hipStream_t st, Trace *tr) {
    const Mamba2SsdShape *s = &a->shape;
    const uint32_t f = a->flags;
    const int64_t P = s->headdim, N = s->dstate, Pp = pp.ps.headdim, Np = pp.ps.dstate;
    const int64_t blh = s->batch * s->seqlen * s->nheads, blg = s->batch * s->seqlen * s->ngroups;
    const int64_t bh = s->batch * s->nheads;
    Mamba2SsdFwdArgs pa = *a;
    pa.shape = pp.ps;
    auto at = [&](size_t off) { return (float *)(ws + off); };
    // inputs: padded copies of what changes shape (traced with the inner kernels' events)
    if (pp.pad_p) {
        if (int rc = pad_copy(a->x, blh, 1, P, at(pp.x), 1, Pp, st, nullptr)) return rc;
        pa.x = at(pp.x);
        if (f & MAMBA2_SSD_HAS_Z) {
            if (int rc = pad_copy(a->z, blh, 1, P, at(pp.z), 1, Pp, st, nullptr)) return rc;
            pa.z = at(pp.z);
        }
        if (f & MAMBA2_SSD_D_PER_CHANNEL) {
            if (int rc = pad_copy(a->D, s->nheads, 1, P, at(pp.d), 1, Pp, st, nullptr)) return rc;
            pa.D = at(pp.d);
        }
        pa.out = at(pp.out);
        pa.pre_gate = (f & MAMBA2_SSD_HAS_Z) && a->pre_gate ? at(pp.pre) : nullptr;
    }
    if (pp.pad_n) {
        if (int rc = pad_copy(a->B, blg, 1, N, at(pp.b), 1, Np, st, nullptr)) return rc;
        if (int rc = pad_copy(a->C, blg, 1, N, at(pp.c), 1, Np, st, nullptr)) return rc;
        pa.B = at(pp.b);
        pa.C = at(pp.c);
    }
    if (f & MAMBA2_SSD_HAS_INITIAL) {
        if (int rc = pad_copy(a->initial_states, bh, P, N, at(pp.init), Pp, Np, st, nullptr)) return rc;
        pa.initial_states = at(pp.init);
    }
    pa.final_state = a->final_state ? at(pp.fin) : nullptr;
    if (int rc = fwd_impl(&pa, ws + pp.inner, have - pp.inner, st, tr)) return rc;
    if (pp.pad_p) {
        if (int rc = pad_copy(pa.out, blh, 1, Pp, a->out, 1, P, st, tr)) return rc;
        if (pa.pre_gate)
            if (int rc = pad_copy(pa.pre_gate, blh, 1, Pp, a->pre_gate, 1, P, st, tr)) return rc;
    }
    if (a->final_state)
        if (int rc = pad_copy(pa.final_state, bh, Pp, Np, a->final_state, P, N, st, tr)) return rc;
    return ok();
}

int fwd_impl(const Mamba2SsdFwdArgs *a, void *workspace, size_t workspace_bytes, void *stream,
             Trace *tr) {
    if (!a) return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "args is NULL");
    const Mamba2SsdShape *s = &a->shape;
    if (int rc = check_shape(s, a->flags)) return rc;
    if (!a->x || !a->dt || !a->A || !a->B || !a->C || !a->out)
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "x, dt, A, B, C and out must be non-NULL");
    const uint32_t f = a->flags;
    if (bool(f & MAMBA2_SSD_HAS_D) != (a->D != nullptr))
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "D pointer and HAS_D flag disagree");
    if (bool(f & MAMBA2_SSD_HAS_Z) != (a->z != nullptr))
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "z pointer and HAS_Z flag disagree");
    if (bool(f & MAMBA2_SSD_HAS_DT_BIAS) != (a->dt_bias != nullptr))
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "dt_bias pointer and HAS_DT_BIAS flag disagree");
    if (bool(f & MAMBA2_SSD_HAS_INITIAL) != (a->initial_states != nullptr))
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT,
                    "initial_states pointer and HAS_INITIAL flag disagree");
    if (!(a->dt_limit_min <= a->dt_limit_max))
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "dt_limit_min > dt_limit_max");
    if (bool(f & MAMBA2_SSD_SAVED_STATES) != (a->chunk_states != nullptr))
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT,
                    "chunk_states pointer and SAVED_STATES flag disagree");
    if ((f & (MAMBA2_SSD_SAVED_STATES | MAMBA2_SSD_VARLEN_STATES)) && !fused_shape(s))
        return fail(MAMBA2_SSD_ERR_UNSUPPORTED,
                    "SAVED_STATES and VARLEN_STATES need headdim 64 with dstate 64 or 128 "
                    "(got %lld, %lld)",
                    (long long)s->headdim, (long long)s->dstate);
    if ((f & MAMBA2_SSD_HAS_SEQ_IDX) && !fused_shape(s) && head_split(s) == 1)
        return fail(MAMBA2_SSD_ERR_UNSUPPORTED,
                    "HAS_SEQ_IDX needs a headdim that is a multiple of 64 with dstate 64 or 128 "
                    "(got %lld, %lld)",
                    (long long)s->headdim, (long long)s->dstate);
    if (bool(f & MAMBA2_SSD_HAS_SEQ_IDX) != (a->seq_idx != nullptr))
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "seq_idx pointer and HAS_SEQ_IDX flag disagree");
    const bool varlen = (f & MAMBA2_SSD_VARLEN_STATES) != 0;
    if (varlen != (a->cu_seqlens != nullptr) || varlen != (a->varlen_states != nullptr))
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT,
                    "cu_seqlens / varlen_states pointers and VARLEN_STATES flag disagree");
    if (varlen) {
        if (s->batch != 1)
            return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT,
                        "VARLEN_STATES needs batch 1 (got %lld)", (long long)s->batch);
        if (a->nseqs <= 0 || a->nseqs > 65535)
            return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "nseqs must be in [1, 65535], got %lld",
                        (long long)a->nseqs);
        if (s->chunk_size % ssd::kChunk)
            return fail(MAMBA2_SSD_ERR_UNSUPPORTED,
                        "VARLEN_STATES needs chunk_size a multiple of 64 (got %lld)",
                        (long long)s->chunk_size);
        if (s->seqlen > 0x7fffffff || s->chunk_size > 0x40000000)
            return fail(MAMBA2_SSD_ERR_UNSUPPORTED,
                        "VARLEN_STATES needs seqlen < 2^31 and chunk_size <= 2^30");
    }
    // a workspace of the queried size runs the full plan; one that only holds
    // the plan without the C . B^T precompute runs that plan
    const size_t need = fwd_ws_bytes(s, f), need_min = fwd_ws_bytes(s, f, false);
    const size_t have = workspace ? workspace_bytes : 0;
    if (need_min && have < need_min)
        return fail(MAMBA2_SSD_ERR_WORKSPACE, "workspace of %zu bytes needed, got %zu", need, have);
    const bool allow_cb = have >= need;
    hipStream_t st = (hipStream_t)stream;
    const PadPlan pp = pad_plan(s, f, allow_cb);
    if (pp.on) return fwd_padded(a, pp, (char *)workspace, have, st, tr);

    ssd::FwdParams prm{};
    prm.x = a->x;
    prm.dt = a->dt;
    prm.A = a->A;
    prm.B = a->B;
    prm.C = a->C;
    prm.D = a->D;
    prm.z = a->z;
    prm.dt_bias = a->dt_bias;
    prm.init = a->initial_states;
    prm.out = a->out;
    prm.final_state = a->final_state;
    prm.pre_gate = (f & MAMBA2_SSD_HAS_Z) ? a->pre_gate : nullptr;
    prm.chunk_states = a->chunk_states;
    prm.seq_idx = a->seq_idx;
    prm.L = s->seqlen;
    prm.H = (int)s->nheads;
    prm.G = (int)s->ngroups;
    prm.R = (int)(s->nheads / s->ngroups);
    prm.K = (int)nchunks(s);
    prm.hdiv = 1;
    prm.softplus = (f & MAMBA2_SSD_DT_SOFTPLUS) != 0;
    prm.has_D = (f & MAMBA2_SSD_HAS_D) != 0;
    prm.d_per_channel = (f & MAMBA2_SSD_D_PER_CHANNEL) != 0;
    prm.has_z = (f & MAMBA2_SSD_HAS_Z) != 0;
    prm.lo = a->dt_limit_min;
    prm.hi = a->dt_limit_max;

    const int B = (int)s->batch;
    if (s->seqlen == 0) {
        // no tokens: the final state is the initial state (or zero), and
        // every varlen state is zero; written by a kernel (no memset or
        // memcpy, so a captured forward holds kernel nodes only)
        auto fill = [&](const float *src, float *dst, int64_t n) {
            const int64_t blocks = std::min<int64_t>((n + ssd::kPadThreads - 1) / ssd::kPadThreads, 4096);
            hipLaunchKernelGGL(ssd::k_copy_or_zero, dim3((unsigned)std::max<int64_t>(blocks, 1)),
                               dim3(ssd::kPadThreads), 0, st, src, dst, n);
            return launch_status("k_copy_or_zero", tr, st);
        };
        if (int rc = record(tr, st, nullptr)) return rc;
        if (a->final_state)
            if (int rc = fill(a->initial_states, a->final_state, s->batch * s->nheads * s->headdim * s->dstate))
                return rc;
        if (varlen)
            if (int rc = fill(nullptr, a->varlen_states, a->nseqs * s->nheads * s->headdim * s->dstate)) return rc;
        return ok();
    }
    // the fused kernels' view of the shape (heads of dim 64)
    const Mamba2SsdShape vs = fused_view(s);
    const int m = head_split(s);
    const FwdPlan pl = fwd_plan(&vs, f, allow_cb);
    if (pl.fused && m > 1) {
        prm.H = (int)vs.nheads;
        prm.R = (int)(vs.nheads / vs.ngroups);
        prm.hdiv = m;
    }
    if (varlen && !prm.chunk_states) prm.chunk_states = (float *)((char *)workspace + pl.states);
    const bool seq = prm.seq_idx != nullptr;
    if (pl.fused) {
        ssd::SegParams sp{};
        sp.nseg = pl.nseg;
        sp.M = pl.M;
        sp.nsplit = pl.nsplit;
        const unsigned units = (unsigned)(vs.batch * vs.nheads * pl.nseg * pl.nsplit);
        ssd::FwdParams kp = prm;
        if (int rc = record(tr, st, nullptr)) return rc;
        if (pl.nseg > 1) {
            // each pre-segment's contribution, then the states at their boundaries
            ssd::SegParams pre = sp;
            pre.nseg = pl.nseg_pre;
            pre.M = pl.M_pre;
            pre.seg_state = (float *)((char *)workspace + pl.seg_state);
            pre.seg_log_decay = (float *)((char *)workspace + pl.seg_decay);
            const unsigned pre_units = (unsigned)(vs.batch * vs.nheads * pl.nseg_pre * pl.nsplit);
            ssd::launch_fwd_seg(true, false, false, seq, dim3(pre_units), st, kp, pre);
            if (int rc = launch_status("k_fwd_seg_state", tr, st)) return rc;
            sp.seg_in = pre.seg_state;
            sp.seg_in_n = pl.nseg_pre;
            sp.in_mult = pl.mult;
            if (pl.fold) {
                // each full segment folds the contributions itself; the last writes the final state
                sp.seg_in_log_decay = pre.seg_log_decay;
                sp.write_final = 1;
            } else {
                const int PN = (int)(vs.headdim * vs.dstate);
                const dim3 sgrid((PN / 4 + ssd::kThreads - 1) / ssd::kThreads, B * prm.H);
                hipLaunchKernelGGL(ssd::k_state_pass, sgrid, dim3(ssd::kThreads), 0, st, pre.seg_state,
                                   pre.seg_log_decay, prm.init, pre.seg_state, prm.final_state, pl.nseg_pre, PN);
                if (int rc = launch_status("k_state_pass", tr, st)) return rc;
                sp.write_final = 0;
            }
        } else {
            sp.write_final = 1;
        }
        kp.chunk_states = prm.chunk_states;
        if (pl.cb) {
            kp.cb = (const float *)((char *)workspace + pl.cb_off);
            ssd::launch_chunk_cb((int)vs.dstate, dim3((unsigned)(vs.batch * vs.ngroups * prm.K)), st, prm.C,
                                 prm.B, (float *)kp.cb, prm.L, prm.G, prm.K);
            if (int rc = launch_status("k_chunk_cb", tr, st)) return rc;
        }
        if (pl.nsplit > 1) {
            // dstate 128: two workgroups per head, 32 channels and all 128
            // state columns each, writing out directly
            ssd::launch_fwd_wide(kp.chunk_states != nullptr, kp.has_z != 0, seq, dim3(units), st, kp, sp);
            if (int rc = launch_status(kp.chunk_states ? "k_fwd_wide_save" : "k_fwd_wide", tr, st)) return rc;
        } else {
            // one round of workgroups (at most one per CU): the latency form
            ssd::launch_fwd_seg(false, kp.chunk_states != nullptr, kp.has_z != 0, seq, dim3(units), st, kp, sp,
                                (int64_t)units <= kMinStreams);
            if (int rc = launch_status(kp.chunk_states ? "k_fwd_seg_save" : "k_fwd_seg", tr, st)) return rc;
        }
        if (varlen) {
            hipLaunchKernelGGL(ssd::k_varlen_states, dim3((unsigned)a->nseqs, prm.H),
                               dim3(ssd::kVarlenThreads), 0, st, prm, a->cu_seqlens,
                               (const float *)prm.chunk_states, a->varlen_states,
                               (int)s->chunk_size, (int)s->headdim, (int)s->dstate);
            if (int rc = launch_status("k_varlen_states", tr, st)) return rc;
        }
        return ok();
    }
    if (s->dstate > 256)
        return fail(MAMBA2_SSD_ERR_UNSUPPORTED, "dstate=%lld > 256 is not supported",
                    (long long)s->dstate);
    const dim3 grid((unsigned)s->headdim, prm.H, B);
    if (int rc = record(tr, st, nullptr)) return rc;
    hipLaunchKernelGGL(ssd::k_generic_fwd, grid, dim3(64), 0, st, prm, (int)s->headdim,
                       (int)s->dstate);
    if (int rc = launch_status("k_generic_fwd", tr, st)) return rc;
    return ok();
}

// Work units of the chunk backward kernel: one workgroup per CU (it holds a
// CU's LDS), in one round, so each pays its pipeline fill once (C4: 16 (b, g)
// streams of 32 chunks as 16 runs of 2 chunks).
constexpr int64_t kBwdUnits = 256;

// The reverse fused chunk backward (k_bwd_ws<., R>, R = 1, 2 or 4 heads per
// group) walks runs of chunks from last to first, carrying the state
// gradients of the group's R heads in registers.  With at least kBwdUnits
// (b, g) streams each stream is one run; with fewer, each is cut into about
// kBwdUnits / (B G) runs of M chunks, and the gradient entering every run
// from the right comes from a pre-pass over the same runs (k_bwd_run_grad:
// each run's own contribution and log decay) and the reverse
// recurrence over runs (k_state_pass_bwd).  nseg = 0: other R, the split path
// (per-chunk dU through HBM).
struct RevPlan {
    int64_t nseg, M;
};

RevPlan bwd_rev_plan(const Mamba2SsdShape *s) {
    const int64_t R = s->nheads / s->ngroups, K = nchunks(s), bg = s->batch * s->ngroups;
    if (!(R == 1 || R == 2 || R == 4)) return {0, 0};
    int64_t nseg = (kBwdUnits + bg - 1) / bg;
    nseg = nseg < K ? nseg : K;
    const int64_t M = (K + nseg - 1) / nseg;
    return {(K + M - 1) / M, M};
}

// Backward workspace: states [B,H,K,P,N] and, for the recompute of long
// sequences with few streams, the forward plan's segment states and log decays
// (both unless SAVED_STATES) | log decay [B,H,K] | dstates [B,H,K,P,N] (split
// path) or, for the reverse fused path with several runs per stream, the run
// carries [B,H,nseg,P,N] and run log decays [B,H,nseg] | dA partials [B,H,K] |
// ddt_bias partials [B,H,K,slots] | dD partials [B,H,K,slots,P] (slots = one
// per consumer wave of the chunk kernel).
struct BwdLayout {
    size_t states, seg_state, seg_decay, log_decay, dstates, rev_carry, rev_decay, part_dA, part_db,
        part_dD, total;
    FwdPlan recompute; // plan of the state recompute (when the states are not passed in)
    RevPlan rev;
};

BwdLayout bwd_layout(const Mamba2SsdShape *s, uint32_t flags) {
    const size_t bhk = (size_t)s->batch * s->nheads * nchunks(s);
    const size_t pn = (size_t)s->headdim * s->dstate;
    BwdLayout l{};
    size_t off = 0;
    l.states = off; // absent when the forward's chunk states are passed in
    if (!(flags & MAMBA2_SSD_SAVED_STATES)) {
        off += align256(bhk * pn * sizeof(float));
        l.recompute = fwd_plan(s, 0);
        if (l.recompute.nseg > 1) {
            const size_t units = (size_t)s->batch * s->nheads * l.recompute.nseg_pre;
            l.seg_state = off;
            off += align256(units * pn * sizeof(float));
            l.seg_decay = off;
            off += align256(units * sizeof(float));
        }
    }
    l.log_decay = off;
    off += align256(bhk * sizeof(float));
    l.rev = bwd_rev_plan(s);
    l.dstates = off;
    if (l.rev.nseg == 0) off += align256(bhk * pn * sizeof(float));
    l.rev_carry = off;
    if (l.rev.nseg > 1) {
        const size_t runs = (size_t)s->batch * s->nheads * l.rev.nseg;
        off += align256(runs * pn * sizeof(float));
        l.rev_decay = off;
        off += align256(runs * sizeof(float));
    }
    l.part_dA = off;
    off += align256(bhk * sizeof(float));
    l.part_db = off;
    off += align256(bhk * ssd::kBwsSlots * sizeof(float));
    l.part_dD = off;
    off += align256(bhk * ssd::kBwsSlots * (size_t)s->headdim * sizeof(float));
    l.total = off;
    return l;
}

bool bwd_supported(const Mamba2SsdShape *s) { return s->headdim == 64 && s->dstate == 64; }

size_t bwd_ws_bytes(const Mamba2SsdShape *s, uint32_t flags) {
    if (!bwd_supported(s) || s->seqlen == 0) return 0;
    return bwd_layout(s, flags).total;
}

// The reverse state-gradient pass walks each (b, h) stream serially; with
// fewer streams than this it runs as a chunk-parallel dS_off kernel plus an
// elementwise reverse recurrence instead.
constexpr int64_t kMinRevStreams = 512;

int bwd_impl(const Mamba2SsdBwdArgs *a, void *workspace, size_t workspace_bytes, void *stream,
             Trace *tr) {
    if (!a) return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "args is NULL");
    const Mamba2SsdShape *s = &a->shape;
    if (int rc = check_shape(s, a->flags)) return rc;
    const uint32_t f = a->flags;
    if (!a->x || !a->dt || !a->A || !a->B || !a->C)
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "x, dt, A, B and C must be non-NULL");
    if (!a->dx || !a->ddt || !a->dA || !a->dB || !a->dC)
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "dx, ddt, dA, dB and dC must be non-NULL");
    if (bool(f & MAMBA2_SSD_HAS_D) != (a->D != nullptr) ||
        bool(f & MAMBA2_SSD_HAS_D) != (a->dD != nullptr))
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "D / dD pointers and HAS_D flag disagree");
    if (bool(f & MAMBA2_SSD_HAS_Z) != (a->z != nullptr) ||
        bool(f & MAMBA2_SSD_HAS_Z) != (a->dz != nullptr))
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "z / dz pointers and HAS_Z flag disagree");
    if ((f & MAMBA2_SSD_HAS_Z) && !a->pre_gate)
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "HAS_Z needs the forward's pre_gate");
    if (bool(f & MAMBA2_SSD_HAS_DT_BIAS) != (a->dt_bias != nullptr) ||
        bool(f & MAMBA2_SSD_HAS_DT_BIAS) != (a->ddt_bias != nullptr))
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT,
                    "dt_bias / ddt_bias pointers and HAS_DT_BIAS flag disagree");
    if (bool(f & MAMBA2_SSD_HAS_INITIAL) != (a->initial_states != nullptr) ||
        bool(f & MAMBA2_SSD_HAS_INITIAL) != (a->dinitial_states != nullptr))
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT,
                    "initial_states / dinitial_states pointers and HAS_INITIAL flag disagree");
    if (!(a->dt_limit_min <= a->dt_limit_max))
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "dt_limit_min > dt_limit_max");
    if (bool(f & MAMBA2_SSD_SAVED_STATES) != (a->chunk_states != nullptr))
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT,
                    "chunk_states pointer and SAVED_STATES flag disagree");
    if (bool(f & MAMBA2_SSD_HAS_SEQ_IDX) != (a->seq_idx != nullptr))
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "seq_idx pointer and HAS_SEQ_IDX flag disagree");
    if (f & MAMBA2_SSD_VARLEN_STATES)
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "VARLEN_STATES is a forward-only flag");
    if (!bwd_supported(s))
        return fail(MAMBA2_SSD_ERR_UNSUPPORTED,
                    "mamba2_ssd_bwd_m1 needs headdim == dstate == 64 (got %lld, %lld)",
                    (long long)s->headdim, (long long)s->dstate);
    if (s->seqlen == 0)
        return fail(MAMBA2_SSD_ERR_UNSUPPORTED, "mamba2_ssd_bwd_m1 needs seqlen > 0");
    // the reverse state pass addresses a stream's chunk states with 32-bit
    // byte offsets
    if (nchunks(s) * 64 * 64 * 4 > (int64_t)0x7fffffff)
        return fail(MAMBA2_SSD_ERR_UNSUPPORTED, "mamba2_ssd_bwd_m1 needs seqlen < %lld",
                    (long long)((int64_t)0x7fffffff / (64 * 64 * 4) * 64));
    const BwdLayout lay = bwd_layout(s, f);
    if (!workspace || workspace_bytes < lay.total)
        return fail(MAMBA2_SSD_ERR_WORKSPACE, "workspace of %zu bytes needed, got %zu", lay.total,
                    workspace ? workspace_bytes : (size_t)0);
    hipStream_t st = (hipStream_t)stream;
    char *ws = (char *)workspace;
    const int B = (int)s->batch, H = (int)s->nheads, K = (int)nchunks(s);
    const int PN = 64 * 64;

    // parameters of the chunk-state recompute (skipped when the forward's
    // chunk states are passed in)
    ssd::FwdParams fp{};
    fp.x = a->x;
    fp.dt = a->dt;
    fp.A = a->A;
    fp.B = a->B;
    fp.C = a->C;
    fp.dt_bias = a->dt_bias;
    fp.init = a->initial_states;
    const bool saved = (f & MAMBA2_SSD_SAVED_STATES) != 0;
    fp.states = saved ? const_cast<float *>(a->chunk_states) : (float *)(ws + lay.states);
    fp.chunk_log_decay = (float *)(ws + lay.log_decay);
    fp.L = s->seqlen;
    fp.H = H;
    fp.G = (int)s->ngroups;
    fp.R = (int)(s->nheads / s->ngroups);
    fp.K = K;
    fp.hdiv = 1; // heads are not split here (headdim 64)
    fp.softplus = (f & MAMBA2_SSD_DT_SOFTPLUS) != 0;
    fp.lo = a->dt_limit_min;
    fp.hi = a->dt_limit_max;

    ssd::BwdParams bp{};
    bp.x = a->x;
    bp.dt = a->dt;
    bp.A = a->A;
    bp.B = a->B;
    bp.C = a->C;
    bp.D = a->D;
    bp.z = a->z;
    bp.dt_bias = a->dt_bias;
    bp.dout = a->dout;
    bp.pre_gate = a->pre_gate;
    bp.dx = a->dx;
    bp.ddt = a->ddt;
    bp.dB = a->dB;
    bp.dC = a->dC;
    bp.dz = a->dz;
    bp.states = fp.states;
    bp.log_decay = fp.chunk_log_decay;
    bp.dstates = (float *)(ws + lay.dstates);
    bp.dfinal = a->dfinal_state;
    bp.dinit = a->dinitial_states;
    bp.seq_idx = a->seq_idx;
    const bool seq = a->seq_idx != nullptr;
    bp.part_dA = (float *)(ws + lay.part_dA);
    bp.part_dbias = (float *)(ws + lay.part_db);
    bp.part_dD = (float *)(ws + lay.part_dD);
    bp.L = s->seqlen;
    bp.H = H;
    bp.G = fp.G;
    bp.R = fp.R;
    bp.K = K;
    bp.softplus = fp.softplus;
    bp.has_D = (f & MAMBA2_SSD_HAS_D) != 0;
    bp.d_per_channel = (f & MAMBA2_SSD_D_PER_CHANNEL) != 0;
    bp.has_z = (f & MAMBA2_SSD_HAS_Z) != 0;
    bp.lo = fp.lo;
    bp.hi = fp.hi;

    const dim3 chunk_grid(K, H, B);
    const dim3 state_grid((PN / 4 + ssd::kThreads - 1) / ssd::kThreads, B * H);
    if (int rc = record(tr, st, nullptr)) return rc;
    if (!saved) {
        // recompute of the chunk-start states by the fused forward's state
        // pass (x, dt and B streamed once, the states written once); with
        // segments, their contributions and the segment recurrence first
        ssd::FwdParams kp = fp;
        kp.seq_idx = a->seq_idx;
        ssd::FwdParams sp_prm = fp;
        sp_prm.chunk_states = fp.states;
        sp_prm.seq_idx = a->seq_idx;
        ssd::SegParams sp{};
        sp.nseg = lay.recompute.nseg;
        sp.M = lay.recompute.M;
        sp.nsplit = 1;
        const unsigned units = (unsigned)(B * H * sp.nseg);
        const bool seq = a->seq_idx != nullptr;
        if (sp.nseg > 1) {
            ssd::SegParams pre = sp;
            pre.nseg = lay.recompute.nseg_pre;
            pre.M = lay.recompute.M_pre;
            pre.seg_state = (float *)(ws + lay.seg_state);
            pre.seg_log_decay = (float *)(ws + lay.seg_decay);
            ssd::launch_fwd_seg(true, false, false, seq, dim3((unsigned)(B * H * pre.nseg)), st, kp, pre);
            if (int rc = launch_status("k_fwd_seg_state", tr, st)) return rc;
            if (lay.recompute.fold) {
                sp.seg_in_log_decay = pre.seg_log_decay;
            } else {
                hipLaunchKernelGGL(ssd::k_state_pass, dim3((PN / 4 + ssd::kThreads - 1) / ssd::kThreads, B * H),
                                   dim3(ssd::kThreads), 0, st, pre.seg_state, pre.seg_log_decay, fp.init,
                                   pre.seg_state, (float *)nullptr, pre.nseg, PN);
                if (int rc = launch_status("k_state_pass", tr, st)) return rc;
            }
            sp.seg_in = pre.seg_state;
            sp.seg_in_n = pre.nseg;
            sp.in_mult = lay.recompute.mult;
        }
        if (sp.nseg == 1 && !seq && sp_prm.R == 4 && B * s->ngroups >= kMinStreams) {
            // one workgroup per (b, g) walking its four heads per chunk: B read
            // once; with fewer (b, g) streams than CUs the per-head pass keeps
            // more of the GPU busy
            ssd::launch_fwd_state_group(dim3((unsigned)(B * s->ngroups)), st, sp_prm);
            if (int rc = launch_status("k_fwd_state_group", tr, st)) return rc;
        } else {
            ssd::launch_fwd_seg(true, true, false, seq, dim3(units), st, sp_prm, sp);
            if (int rc = launch_status("k_fwd_seg_state_save", tr, st)) return rc;
        }
    }
    const int64_t bg = (int64_t)B * s->ngroups;
    if (lay.rev.nseg > 0) {
        // reverse chunk order, state gradients carried in registers; with
        // several runs per stream, the gradient entering each run first
        const int nseg = (int)lay.rev.nseg;
        if (nseg > 1) {
            ssd::RevSeg rs{};
            rs.nseg = nseg;
            rs.M = (int)lay.rev.M;
            rs.seg_carry = (float *)(ws + lay.rev_carry);
            rs.seg_log_decay = (float *)(ws + lay.rev_decay);
            // each run's own contribution and log decay, one workgroup per (b, h, run)
            ssd::launch_bwd_run_grad(bp.has_z != 0, seq, dim3((unsigned)(B * H * nseg)), st, bp, rs);
            if (int rc = launch_status("k_bwd_run_grad", tr, st)) return rc;
            // in place: run s's slot becomes the gradient entering it from the right
            hipLaunchKernelGGL(ssd::k_state_pass_bwd, state_grid, dim3(ssd::kThreads), 0, st, rs.seg_carry,
                               rs.seg_log_decay, a->dfinal_state, (float *)nullptr, nseg, PN);
            if (int rc = launch_status("k_state_pass_bwd", tr, st)) return rc;
            bp.carry_in = rs.seg_carry;
        }
        ssd::launch_bwd_ws(bp.has_z != 0, bp.R, seq, dim3((unsigned)(bg * nseg)), st, bp, nseg,
                           (int)lay.rev.M);
        if (int rc = launch_status("k_bwd_ws_rev", tr, st)) return rc;
        hipLaunchKernelGGL(ssd::k_bwd_finalize_slots, dim3(H), dim3(ssd::kThreads), 0, st, bp.part_dA,
                           bp.part_dbias, bp.part_dD, a->dA, a->ddt_bias, a->dD, B, H, K, 64,
                           ssd::kBwsSlots, bp.has_D, bp.d_per_channel);
        if (int rc = launch_status("k_bwd_finalize", tr, st)) return rc;
        return ok();
    }
    // state gradients dU_k (and dinitial_states)
    if ((int64_t)B * H >= kMinRevStreams) {
        ssd::launch_bwd_dstate_rev(bp.has_z != 0, seq, dim3((unsigned)(B * H)), st, bp, a->dfinal_state,
                                   a->dinitial_states);
        if (int rc = launch_status("k_bwd_dstate_rev", tr, st)) return rc;
    } else {
        hipLaunchKernelGGL(ssd::bwd::k_bwd_dstate, chunk_grid, dim3(ssd::kThreads), 0, st, bp);
        if (int rc = launch_status("k_bwd_dstate", tr, st)) return rc;
        hipLaunchKernelGGL(ssd::k_state_pass_bwd, state_grid, dim3(ssd::kThreads), 0, st, bp.dstates,
                           fp.chunk_log_decay, a->dfinal_state, a->dinitial_states, K, PN);
        if (int rc = launch_status("k_state_pass_bwd", tr, st)) return rc;
    }
    // chunk backward: (b, g, run of chunks) work units, about kBwdUnits of them
    int64_t nseg = (kBwdUnits + bg - 1) / bg;
    nseg = nseg < K ? nseg : K;
    const int M = (int)((K + nseg - 1) / nseg);
    nseg = (K + M - 1) / M;
    ssd::launch_bwd_ws(bp.has_z != 0, 0, seq, dim3((unsigned)(bg * nseg)), st, bp, (int)nseg, M);
    if (int rc = launch_status("k_bwd_ws", tr, st)) return rc;
    hipLaunchKernelGGL(ssd::k_bwd_finalize_slots, dim3(H), dim3(ssd::kThreads), 0, st, bp.part_dA,
                       bp.part_dbias, bp.part_dD, a->dA, a->ddt_bias, a->dD, B, H, K, 64,
                       ssd::kBwsSlots, bp.has_D, bp.d_per_channel);
    if (int rc = launch_status("k_bwd_finalize", tr, st)) return rc;
    return ok();
}

}  // namespace

extern "C" {

int mamba2_ssd_fwd(const Mamba2SsdFwdArgs *a, void *workspace, size_t workspace_bytes,
                   void *stream) {
    return fwd_impl(a, workspace, workspace_bytes, stream, nullptr);
}

int mamba2_ssd_fwd_traced(const Mamba2SsdFwdArgs *a, void *workspace, size_t workspace_bytes,
                          void *stream, void *const *events, int nevents, const char **names,
                          int *nkernels) {
    if (!events || nevents < 2 || !nkernels)
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "traced call needs events[>=2] and nkernels");
    Trace tr;
    tr.events = events;
    tr.capacity = nevents;
    tr.names = names;
    const int rc = fwd_impl(a, workspace, workspace_bytes, stream, &tr);
    *nkernels = tr.used > 0 ? tr.used - 1 : 0;
    return rc;
}

}  // extern "C"

namespace {

// Checks and launch shared by the fp32 and fp16 forms of the stage op.
template <typename Tin>
int state_passing_impl(const Tin *chunk_states, const float *chunk_log_decay, const float *initial_states,
                       float *states_start, float *final_state, int64_t batch, int64_t nheads, int64_t nchunks_,
                       int64_t headdim, int64_t dstate, void *stream) {
    if (!chunk_states || !chunk_log_decay || !states_start)
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT,
                    "chunk_states, chunk_log_decay and states_start must be non-NULL");
    if (batch <= 0 || nheads <= 0 || nchunks_ <= 0 || headdim <= 0 || dstate <= 0)
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "non-positive dimension");
    const int64_t PN = headdim * dstate;
    if (PN % 4)
        return fail(MAMBA2_SSD_ERR_UNSUPPORTED, "headdim*dstate must be a multiple of 4");
    // k_state_pass addresses its ring of kStateRing chunks and the log decays
    // with 32-bit byte offsets: 16 chunks of PN floats and (K + 2 * 16) floats
    if (batch * nheads > 65535)
        return fail(MAMBA2_SSD_ERR_UNSUPPORTED, "batch * nheads must be <= 65535");
    if (PN * 4 * ssd::kStateRing > (int64_t)0x7fffffff ||
        (nchunks_ + 2 * ssd::kStateRing) * 4 > (int64_t)0x7fffffff)
        return fail(MAMBA2_SSD_ERR_UNSUPPORTED,
                    "headdim*dstate=%lld must be <= %lld and nchunks=%lld <= %lld",
                    (long long)PN, (long long)(0x7fffffff / (4 * ssd::kStateRing)),
                    (long long)nchunks_, (long long)(0x7fffffff / 4 - 2 * ssd::kStateRing));
    const dim3 grid((unsigned)((PN / 4 + ssd::kThreads - 1) / ssd::kThreads), (unsigned)(batch * nheads));
    if constexpr (sizeof(Tin) == 2) {
        // fp16 in, fp32 out: the output cannot share the input's memory
        const char *in = (const char *)chunk_states, *out = (const char *)states_start;
        const size_t in_bytes = (size_t)(batch * nheads * nchunks_ * PN) * 2, out_bytes = in_bytes * 2;
        if (in < out + out_bytes && out < in + in_bytes)
            return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT,
                        "states_start (fp32) must not overlap the fp16 chunk_states");
        hipLaunchKernelGGL(ssd::k_state_pass_f16, grid, dim3(ssd::kThreads), 0, (hipStream_t)stream,
                           (const _Float16 *)chunk_states, chunk_log_decay, initial_states, states_start,
                           final_state, (int)nchunks_, (int)PN);
        if (int rc = launch_status("k_state_pass_f16")) return rc;
    } else {
        hipLaunchKernelGGL(ssd::k_state_pass, grid, dim3(ssd::kThreads), 0, (hipStream_t)stream, chunk_states,
                           chunk_log_decay, initial_states, states_start, final_state, (int)nchunks_, (int)PN);
        if (int rc = launch_status("k_state_pass")) return rc;
    }
    return ok();
}

}  // namespace

extern "C" {

int mamba2_ssd_state_passing(const float *chunk_states, const float *chunk_log_decay,
                             const float *initial_states, float *states_start,
                             float *final_state, int64_t batch, int64_t nheads, int64_t nchunks_,
                             int64_t headdim, int64_t dstate, void *stream) {
    return state_passing_impl(chunk_states, chunk_log_decay, initial_states, states_start, final_state, batch,
                              nheads, nchunks_, headdim, dstate, stream);
}

int mamba2_ssd_state_passing_f16(const void *chunk_states, const float *chunk_log_decay,
                                 const float *initial_states, float *states_start, float *final_state,
                                 int64_t batch, int64_t nheads, int64_t nchunks_, int64_t headdim,
                                 int64_t dstate, void *stream) {
    return state_passing_impl((const _Float16 *)chunk_states, chunk_log_decay, initial_states, states_start,
                              final_state, batch, nheads, nchunks_, headdim, dstate, stream);
}

int mamba2_selective_state_update(const Mamba2SsuArgs *a, void *stream) {
    if (!a) return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "args is NULL");
    constexpr uint32_t kKnown = MAMBA2_SSU_TIED | MAMBA2_SSU_STRIDES | MAMBA2_SSD_DT_SOFTPLUS |
                                MAMBA2_SSD_HAS_D | MAMBA2_SSD_D_PER_CHANNEL | MAMBA2_SSD_HAS_Z |
                                MAMBA2_SSD_HAS_DT_BIAS;
    const uint32_t f = a->flags;
    if (f & ~kKnown) return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "unknown flag bits 0x%x", f & ~kKnown);
    if (a->batch <= 0 || a->nheads <= 0 || a->headdim <= 0 || a->dstate <= 0 || a->ngroups <= 0)
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "non-positive dimension");
    if (a->nheads % a->ngroups)
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "nheads (%lld) must be divisible by ngroups (%lld)",
                    (long long)a->nheads, (long long)a->ngroups);
    if (!a->state || !a->x || !a->dt || !a->A || !a->B || !a->C || !a->out)
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "state, x, dt, A, B, C and out must be non-NULL");
    if (bool(f & MAMBA2_SSD_HAS_D) != (a->D != nullptr))
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "D pointer and HAS_D flag disagree");
    if (bool(f & MAMBA2_SSD_HAS_Z) != (a->z != nullptr))
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "z pointer and HAS_Z flag disagree");
    if (bool(f & MAMBA2_SSD_HAS_DT_BIAS) != (a->dt_bias != nullptr))
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "dt_bias pointer and HAS_DT_BIAS flag disagree");
    if (a->dstate % 4 || a->dstate > 256)
        return fail(MAMBA2_SSD_ERR_UNSUPPORTED, "dstate must be a multiple of 4 and <= 256 (got %lld)",
                    (long long)a->dstate);
    const int64_t slot_elems = a->nheads * a->headdim * a->dstate;
    if (a->state_slots <= 0 || a->state_slot_stride < slot_elems || a->state_slot_stride % 4)
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT,
                    "state needs >= 1 slot and a slot stride >= H*P*N, a multiple of 4");
    if (!a->state_batch_indices && a->state_slots < a->batch)
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "fewer state slots (%lld) than sequences (%lld)",
                    (long long)a->state_slots, (long long)a->batch);
    for (const void *ptr : {(const void *)a->state, (const void *)a->B, (const void *)a->C,
                            (const void *)((f & MAMBA2_SSU_TIED) ? nullptr : a->A)})
        if ((uintptr_t)ptr % 16)
            return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "state, B, C (and A [H, P, N]) must be 16-byte aligned");
    if (a->batch * a->nheads > 65535 || a->headdim > (1 << 24))
        return fail(MAMBA2_SSD_ERR_UNSUPPORTED, "batch * nheads must be <= 65535");
    ssd::SsuParams prm{};
    prm.state = a->state;
    prm.state_bstride = a->state_slot_stride;
    prm.nslots = a->state_slots;
    prm.x = a->x;
    prm.dt = a->dt;
    prm.A = a->A;
    prm.B = a->B;
    prm.C = a->C;
    prm.D = a->D;
    prm.z = a->z;
    prm.dt_bias = a->dt_bias;
    prm.slot = a->state_batch_indices;
    prm.out = a->out;
    prm.H = (int)a->nheads;
    prm.P = (int)a->headdim;
    prm.N = (int)a->dstate;
    prm.G = (int)a->ngroups;
    prm.R = (int)(a->nheads / a->ngroups);
    int lpr = 1;
    while (lpr * 4 < prm.N) lpr *= 2;
    prm.lpr = lpr;
    prm.tied = (f & MAMBA2_SSU_TIED) != 0;
    prm.softplus = (f & MAMBA2_SSD_DT_SOFTPLUS) != 0;
    prm.has_D = (f & MAMBA2_SSD_HAS_D) != 0;
    prm.d_per_channel = (f & MAMBA2_SSD_D_PER_CHANNEL) != 0;
    prm.has_z = (f & MAMBA2_SSD_HAS_Z) != 0;
    const int64_t H = a->nheads, P = a->headdim, N = a->dstate, G = a->ngroups;
    if (f & MAMBA2_SSU_STRIDES) {
        const Mamba2SsuStrides &st = a->strides;
        prm.x_b = st.x_b, prm.x_h = st.x_h, prm.z_b = st.z_b, prm.z_h = st.z_h;
        prm.bc_b = st.bc_b, prm.bc_g = st.bc_g;
        prm.dt_b = st.dt_b, prm.dt_h = st.dt_h, prm.dt_p = st.dt_p;
        prm.A_h = st.A_h, prm.A_p = st.A_p, prm.A_n = st.A_n;
        prm.bias_h = st.bias_h, prm.bias_p = st.bias_p, prm.D_h = st.D_h, prm.D_p = st.D_p;
    } else {
        // the contiguous layouts of the shapes
        prm.x_b = prm.z_b = H * P, prm.x_h = prm.z_h = P;
        prm.bc_b = G * N, prm.bc_g = N;
        if (prm.tied) {
            prm.dt_b = H, prm.dt_h = 1, prm.dt_p = 0;
            prm.A_h = 1, prm.A_p = 0, prm.A_n = 0;
            prm.bias_h = 1, prm.bias_p = 0;
        } else {
            prm.dt_b = H * P, prm.dt_h = P, prm.dt_p = 1;
            prm.A_h = P * N, prm.A_p = N, prm.A_n = 1;
            prm.bias_h = P, prm.bias_p = 1;
        }
        prm.D_h = prm.d_per_channel ? P : 1, prm.D_p = prm.d_per_channel ? 1 : 0;
    }
    // the 16-byte loads of B, C rows and of a contiguous untied A row
    if (prm.bc_b % 4 || prm.bc_g % 4)
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "B and C strides must be multiples of 4 elements");
    if (!prm.tied && prm.A_n == 1 && (prm.A_h % 4 || prm.A_p % 4))
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT,
                    "an untied A with unit dstate stride needs head and dim strides that are multiples of 4");
    // one workgroup per (b, h) walks all rows; with few (b, h) pairs the rows
    // are split over up to 8 workgroups so the grid still has ~2k of them
    const int rows = 256 / lpr;
    const int64_t passes = (prm.P + rows - 1) / rows, bh = a->batch * a->nheads;
    int64_t gx = (2048 + bh - 1) / bh;
    gx = gx < passes ? gx : passes;
    gx = gx < 8 ? gx : 8;
    const dim3 grid((unsigned)gx, (unsigned)bh);
    hipLaunchKernelGGL(ssd::k_ssu, grid, dim3(256), 0, (hipStream_t)stream, prm);
    if (int rc = launch_status("k_ssu")) return rc;
    return ok();
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free forward (mamba2_ssd_fwd_noalloc): the forward's scratch (the
// segment states and log decays of long sequences with few streams, and the
// other buffers fwd_plan lays out) comes from this file-scope device array
// instead of a caller workspace.  Each GPU the library runs on holds its own
// copy until the process ends; host code reaches it only through the address
// hipGetSymbolAddress returns for that device.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[MAMBA2_SSD_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the calling thread's current device, looked
// up once per device with that device current.
int scratch_for_current_device(void **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(MAMBA2_SSD_ERR_LAUNCH, "hipGetDevice failed: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices)
        return fail(MAMBA2_SSD_ERR_UNSUPPORTED, "device %d: the allocation-free forward supports %d devices",
                    dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(MAMBA2_SSD_ERR_LAUNCH, "hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                        hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return MAMBA2_SSD_OK;
}

}  // namespace

extern "C" {

int mamba2_ssd_fwd_noalloc(const Mamba2SsdFwdArgs *a, void *stream) {
    if (!a) return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "args is NULL");
    if (int rc = check_shape(&a->shape, a->flags)) return rc;
    // the least workspace the forward runs with (fwd_impl leaves out the
    // C . B^T precompute when the scratch cannot also hold it)
    const size_t need = fwd_ws_bytes(&a->shape, a->flags, false);
    if (need > (size_t)MAMBA2_SSD_NOALLOC_SCRATCH_BYTES)
        return fail(MAMBA2_SSD_ERR_WORKSPACE,
                    "this forward needs %zu bytes of scratch; mamba2_ssd_fwd_noalloc has %zu "
                    "(use mamba2_ssd_fwd with a workspace)",
                    need, (size_t)MAMBA2_SSD_NOALLOC_SCRATCH_BYTES);
    void *ws = nullptr;
    const bool any = fwd_ws_bytes(&a->shape, a->flags) > 0;
    if (any)
        if (int rc = scratch_for_current_device(&ws)) return rc;
    return fwd_impl(a, ws, any ? (size_t)MAMBA2_SSD_NOALLOC_SCRATCH_BYTES : 0, stream, nullptr);
}

int mamba2_ssd_bwd_m1_workspace_size(const Mamba2SsdShape *shape, uint32_t flags, size_t *bytes) {
    if (int rc = check_shape(shape, flags)) return rc;
    if (!bytes) return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "bytes is NULL");
    *bytes = bwd_ws_bytes(shape, flags);
    return ok();
}

int mamba2_ssd_bwd_m1(const Mamba2SsdBwdArgs *a, void *workspace, size_t workspace_bytes,
                      void *stream) {
    return bwd_impl(a, workspace, workspace_bytes, stream, nullptr);
}

int mamba2_ssd_bwd_m1_traced(const Mamba2SsdBwdArgs *a, void *workspace, size_t workspace_bytes,
                             void *stream, void *const *events, int nevents, const char **names,
                             int *nkernels) {
    if (!events || nevents < 2 || !nkernels)
        return fail(MAMBA2_SSD_ERR_INVALID_ARGUMENT, "traced call needs events[>=2] and nkernels");
    Trace tr;
    tr.events = events;
    tr.capacity = nevents;
    tr.names = names;
    const int rc = bwd_impl(a, workspace, workspace_bytes, stream, &tr);
    *nkernels = tr.used > 0 ? tr.used - 1 : 0;
    return rc;
}

}  // extern "C"
