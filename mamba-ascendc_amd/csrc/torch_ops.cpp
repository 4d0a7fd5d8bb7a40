// torch.ops.mamba_ascend.* in C++ over the library's C ABI.
//
// The operator schemas are the reference's (mamba_ascendc/csrc/register.cpp:
// 175-179 for mamba2_ssd_fwd, 89-90 for mamba2_ssd_state_passing) plus this
// build's M1 backward and one internal forward that also returns the training
// tensors.  Each operator validates its tensors with the messages and check
// order of the Python layer (ascend_kernel/mamba2.py, which restates the
// reference host wrapper mamba_ascendc/csrc/ops/mamba2_ssd_fwd/op_host/
// mamba2_ssd_fwd.cpp:15-113), allocates outputs and workspace from torch's
// caching allocator, and enqueues the library's kernels on the current HIP
// stream: a call costs a few microseconds of host time instead of the tens a
// Python wrapper with ctypes takes.  CPU tensors reach the same functions
// (registered for the CPU key too) and are rejected by the device check.
// torch on ROCm keeps the CUDA device type for HIP devices, so the device
// guard and the current stream are the "masquerading as CUDA" forms.
#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/library.h>

#include <cmath>
#include <string>
#include <tuple>

#include "../../include/mamba2_ssd.h"

namespace {

using at::Tensor;
using c10::optional;

const char *status_name(int rc) {
    switch (rc) {
    case MAMBA2_SSD_ERR_INVALID_ARGUMENT: return "INVALID_ARGUMENT";
    case MAMBA2_SSD_ERR_UNSUPPORTED: return "UNSUPPORTED";
    case MAMBA2_SSD_ERR_WORKSPACE: return "WORKSPACE";
    case MAMBA2_SSD_ERR_LAUNCH: return "LAUNCH";
    default: return "ERROR";
    }
}

void check_status(int rc, const char *what) {
    TORCH_CHECK(rc == MAMBA2_SSD_OK, what, ": ", status_name(rc), ": ", mamba2_ssd_last_error());
}

void check_tensor(const char *op, const char *name, const Tensor &t) {
    TORCH_CHECK(t.device().is_cuda(), op, ": ", name, " must be a ROCm GPU tensor (got device ",
                t.device().str(), ")");
    TORCH_CHECK(t.scalar_type() == at::kFloat, op, ": ", name, " must be float32 (got ",
                c10::toString(t.scalar_type()), ")");
    TORCH_CHECK(t.is_contiguous(), op, ": ", name, " must be contiguous");
}

void check_opt(const char *op, const char *name, const optional<Tensor> &t) {
    if (t.has_value()) check_tensor(op, name, *t);
}

const float *cptr(const optional<Tensor> &t) { return t.has_value() ? t->data_ptr<float>() : nullptr; }

float upper_limit(double v) {
    // the schema default 3.402823466e+38 (FLT_MAX) and +inf both mean "no upper clamp"
    return v >= 3.4e38 ? INFINITY : (float)v;
}

int64_t nchunks(const Tensor &x) { return (x.size(1) + 63) / 64; }

// The checks of the reference host wrapper, in its order.
void validate_fwd(const char *op, const Tensor &x, const Tensor &dt, const Tensor &A, const Tensor &B,
                  const Tensor &C, int64_t chunk_size, const optional<Tensor> &D, const optional<Tensor> &z,
                  const optional<Tensor> &dt_bias, const optional<Tensor> &init, double lo, double hi) {
    check_tensor(op, "x", x);
    check_tensor(op, "dt", dt);
    check_tensor(op, "A", A);
    check_tensor(op, "B", B);
    check_tensor(op, "C", C);
    check_opt(op, "D", D);
    check_opt(op, "z", z);
    check_opt(op, "dt_bias", dt_bias);
    check_opt(op, "initial_states", init);
    TORCH_CHECK(x.dim() == 4, op, ": x must have shape [B,L,H,P]");
    TORCH_CHECK(dt.dim() == 3, op, ": dt must have shape [B,L,H]");
    TORCH_CHECK(A.dim() == 1, op, ": A must have shape [H]");
    TORCH_CHECK(B.dim() == 4 && C.dim() == 4, op, ": B and C must have shape [B,L,G,N]");
    const int64_t batch = x.size(0), seqlen = x.size(1), nheads = x.size(2), headdim = x.size(3);
    const int64_t ngroups = B.size(2), dstate = B.size(3);
    TORCH_CHECK(std::min(std::min(batch, seqlen), std::min(nheads, headdim)) > 0, op,
                ": zero-sized dimensions are not supported");
    TORCH_CHECK(dstate > 0 && ngroups > 0, op, ": dstate and ngroups must be positive");
    TORCH_CHECK(dt.size(0) == batch && dt.size(1) == seqlen && dt.size(2) == nheads, op,
                ": dt shape must equal [B,L,H]");
    TORCH_CHECK(A.size(0) == nheads, op, ": A shape must equal [H]");
    TORCH_CHECK(B.sizes() == C.sizes(), op, ": B and C shapes must match");
    TORCH_CHECK(B.size(0) == batch && B.size(1) == seqlen, op,
                ": B/C batch and sequence dimensions must match x");
    TORCH_CHECK(nheads % ngroups == 0, op, ": nheads must be divisible by ngroups");
    TORCH_CHECK(chunk_size > 0, op, ": chunk_size must be positive");
    TORCH_CHECK(lo <= hi, op, ": dt_limit_min must not exceed dt_limit_max");
    if (D.has_value())
        TORCH_CHECK((D->dim() == 1 && D->size(0) == nheads) ||
                        (D->dim() == 2 && D->size(0) == nheads && D->size(1) == headdim),
                    op, ": D must have shape [H] or [H,P]");
    if (z.has_value()) TORCH_CHECK(z->sizes() == x.sizes(), op, ": z shape must match x");
    if (dt_bias.has_value())
        TORCH_CHECK(dt_bias->dim() == 1 && dt_bias->size(0) == nheads, op, ": dt_bias shape must equal [H]");
    if (init.has_value())
        TORCH_CHECK(init->dim() == 4 && init->size(0) == batch && init->size(1) == nheads &&
                        init->size(2) == headdim && init->size(3) == dstate,
                    op, ": initial_states must have shape [B,H,P,N]");
    const at::Device dev = x.device();
    for (const Tensor *t : {&dt, &A, &B, &C})
        TORCH_CHECK(t->device() == dev, op, ": all tensors must be on the same device");
    for (const optional<Tensor> *t : {&D, &z, &dt_bias, &init})
        if (t->has_value()) TORCH_CHECK((*t)->device() == dev, op, ": all tensors must be on the same device");
}

uint32_t feature_flags(const optional<Tensor> &D, const optional<Tensor> &z, const optional<Tensor> &dt_bias,
                       const optional<Tensor> &init, bool softplus) {
    uint32_t f = softplus ? MAMBA2_SSD_DT_SOFTPLUS : 0u;
    if (D.has_value()) f |= MAMBA2_SSD_HAS_D | (D->dim() == 2 ? MAMBA2_SSD_D_PER_CHANNEL : 0u);
    if (z.has_value()) f |= MAMBA2_SSD_HAS_Z;
    if (dt_bias.has_value()) f |= MAMBA2_SSD_HAS_DT_BIAS;
    if (init.has_value()) f |= MAMBA2_SSD_HAS_INITIAL;
    return f;
}

Mamba2SsdShape shape_of(const Tensor &x, const Tensor &B, int64_t chunk_size) {
    return Mamba2SsdShape{x.size(0), x.size(1), x.size(2), x.size(3), B.size(2), B.size(3), chunk_size};
}

Tensor workspace(const Tensor &like, size_t bytes) {
    return at::empty({(int64_t)std::max<size_t>(bytes, 1)}, like.options().dtype(at::kByte));
}

// Forward with the optional outputs of the training forward: (out, final,
// pre_gate, chunk_states), absent ones as empty tensors.
std::tuple<Tensor, Tensor, Tensor, Tensor> fwd_ex(const Tensor &x, const Tensor &dt, const Tensor &A,
                                                  const Tensor &B, const Tensor &C, const optional<Tensor> &D,
                                                  const optional<Tensor> &z, const optional<Tensor> &dt_bias,
                                                  const optional<Tensor> &init, int64_t chunk_size,
                                                  bool dt_softplus, double lo, double hi, bool want_final,
                                                  bool want_pre_gate, bool want_states) {
    const char *op = "mamba2_ssd_fwd";
    validate_fwd(op, x, dt, A, B, C, chunk_size, D, z, dt_bias, init, lo, hi);
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    const Mamba2SsdShape shape = shape_of(x, B, chunk_size);
    uint32_t flags = feature_flags(D, z, dt_bias, init, dt_softplus);
    if (want_states) flags |= MAMBA2_SSD_SAVED_STATES;
    size_t ws_bytes = 0;
    check_status(mamba2_ssd_fwd_workspace_size(&shape, flags, &ws_bytes), "mamba2_ssd_fwd_workspace_size");
    Tensor out = at::empty_like(x);
    const Tensor none = at::empty({0}, x.options());
    Tensor final_state = want_final ? at::empty({x.size(0), x.size(2), x.size(3), B.size(3)}, x.options()) : none;
    Tensor pre_gate = (want_pre_gate && z.has_value()) ? at::empty_like(x) : none;
    Tensor states = want_states ? at::empty({x.size(0), x.size(2), nchunks(x), x.size(3), B.size(3)}, x.options())
                                : none;
    Tensor ws = workspace(x, ws_bytes);
    Mamba2SsdFwdArgs a{};
    a.shape = shape;
    a.flags = flags;
    a.dt_limit_min = (float)lo;
    a.dt_limit_max = upper_limit(hi);
    a.x = x.data_ptr<float>();
    a.dt = dt.data_ptr<float>();
    a.A = A.data_ptr<float>();
    a.B = B.data_ptr<float>();
    a.C = C.data_ptr<float>();
    a.D = cptr(D);
    a.z = cptr(z);
    a.dt_bias = cptr(dt_bias);
    a.initial_states = cptr(init);
    a.out = out.data_ptr<float>();
    a.final_state = want_final ? final_state.data_ptr<float>() : nullptr;
    a.pre_gate = pre_gate.numel() ? pre_gate.data_ptr<float>() : nullptr;
    a.chunk_states = want_states ? states.data_ptr<float>() : nullptr;
    const hipStream_t st = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(x.device().index()).stream();
    check_status(mamba2_ssd_fwd(&a, ws.data_ptr(), ws_bytes, st), "mamba2_ssd_fwd");
    return {out, final_state, pre_gate, states};
}

std::tuple<Tensor, Tensor> fwd(const Tensor &x, const Tensor &dt, const Tensor &A, const Tensor &B,
                               const Tensor &C, const optional<Tensor> &D, const optional<Tensor> &z,
                               const optional<Tensor> &dt_bias, const optional<Tensor> &init, int64_t chunk_size,
                               bool dt_softplus, double lo, double hi) {
    auto r = fwd_ex(x, dt, A, B, C, D, z, dt_bias, init, chunk_size, dt_softplus, lo, hi, true, false, false);
    return {std::get<0>(r), std::get<1>(r)};
}

using Grads = std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor>;

Grads bwd(const Tensor &x, const Tensor &dt, const Tensor &A, const Tensor &B, const Tensor &C, const Tensor &dout,
          const optional<Tensor> &dfinal, const optional<Tensor> &D, const optional<Tensor> &z,
          const optional<Tensor> &dt_bias, const optional<Tensor> &init, const optional<Tensor> &pre_gate,
          const optional<Tensor> &chunk_states, int64_t chunk_size, bool dt_softplus, double lo, double hi,
          const optional<Tensor> &seq_idx) {
    const char *op = "mamba2_ssd_bwd_m1";
    validate_fwd(op, x, dt, A, B, C, chunk_size, D, z, dt_bias, init, lo, hi);
    check_tensor(op, "dout", dout);
    TORCH_CHECK(dout.sizes() == x.sizes(), op, ": dout shape must match x");
    const int64_t b = x.size(0), l = x.size(1), h = x.size(2), p = x.size(3), n = B.size(3);
    if (dfinal.has_value()) {
        check_tensor(op, "dfinal_state", *dfinal);
        TORCH_CHECK(dfinal->dim() == 4 && dfinal->size(0) == b && dfinal->size(1) == h && dfinal->size(2) == p &&
                        dfinal->size(3) == n,
                    op, ": dfinal_state must have shape [B,H,P,N]");
    }
    if (z.has_value()) {
        TORCH_CHECK(pre_gate.has_value(), op, ": z needs the forward's pre_gate (y + D x before the gate)");
        check_tensor(op, "pre_gate", *pre_gate);
        TORCH_CHECK(pre_gate->sizes() == x.sizes(), op, ": pre_gate shape must match x");
    }
    if (chunk_states.has_value()) {
        check_tensor(op, "chunk_states", *chunk_states);
        const int64_t k = nchunks(x);
        const auto s = chunk_states->sizes();
        TORCH_CHECK(s.size() == 5 && s[0] == b && s[1] == h && s[2] == k && s[3] == p && s[4] == n, op,
                    ": chunk_states must have shape [B,H,ceil(L/64),P,N] = [", b, ", ", h, ", ", k, ", ", p,
                    ", ", n, "]");
    }
    Tensor ids;
    if (seq_idx.has_value()) {
        const Tensor &s = *seq_idx;
        TORCH_CHECK(at::isIntegralType(s.scalar_type(), /*includeBool=*/false), op,
                    ": seq_idx must be an integer tensor");
        TORCH_CHECK(s.dim() == 2 && s.size(0) == b && s.size(1) == l, op, ": seq_idx must have shape (", b,
                    ", ", l, ")");
        TORCH_CHECK(s.device() == x.device(), op, ": seq_idx must be on x's device");
        TORCH_CHECK_NOT_IMPLEMENTED(p % 64 == 0 && (n == 64 || n == 128), op,
                                    ": seq_idx needs a headdim that is a multiple of 64 with dstate 64 or 128");
        ids = s.to(at::kInt).contiguous();
    }
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    const Mamba2SsdShape shape = shape_of(x, B, chunk_size);
    uint32_t flags = feature_flags(D, z, dt_bias, init, dt_softplus);
    if (chunk_states.has_value()) flags |= MAMBA2_SSD_SAVED_STATES;
    if (ids.defined()) flags |= MAMBA2_SSD_HAS_SEQ_IDX;
    size_t ws_bytes = 0;
    check_status(mamba2_ssd_bwd_m1_workspace_size(&shape, flags, &ws_bytes), "mamba2_ssd_bwd_m1_workspace_size");
    const Tensor none = at::empty({0}, x.options());
    Tensor dx = at::empty_like(x), ddt = at::empty_like(dt), dA = at::empty_like(A), dB = at::empty_like(B),
           dC = at::empty_like(C);
    Tensor dD = D.has_value() ? at::empty_like(*D) : none;
    Tensor dz = z.has_value() ? at::empty_like(*z) : none;
    Tensor ddt_bias = dt_bias.has_value() ? at::empty_like(*dt_bias) : none;
    Tensor dinit = init.has_value() ? at::empty_like(*init) : none;
    Tensor ws = workspace(x, ws_bytes);
    Mamba2SsdBwdArgs a{};
    a.shape = shape;
    a.flags = flags;
    a.dt_limit_min = (float)lo;
    a.dt_limit_max = upper_limit(hi);
    a.x = x.data_ptr<float>();
    a.dt = dt.data_ptr<float>();
    a.A = A.data_ptr<float>();
    a.B = B.data_ptr<float>();
    a.C = C.data_ptr<float>();
    a.D = cptr(D);
    a.z = cptr(z);
    a.dt_bias = cptr(dt_bias);
    a.initial_states = cptr(init);
    a.dout = dout.data_ptr<float>();
    a.dfinal_state = cptr(dfinal);
    a.pre_gate = z.has_value() ? cptr(pre_gate) : nullptr;
    a.chunk_states = cptr(chunk_states);
    a.dx = dx.data_ptr<float>();
    a.ddt = ddt.data_ptr<float>();
    a.dA = dA.data_ptr<float>();
    a.dB = dB.data_ptr<float>();
    a.dC = dC.data_ptr<float>();
    a.dD = D.has_value() ? dD.data_ptr<float>() : nullptr;
    a.dz = z.has_value() ? dz.data_ptr<float>() : nullptr;
    a.ddt_bias = dt_bias.has_value() ? ddt_bias.data_ptr<float>() : nullptr;
    a.dinitial_states = init.has_value() ? dinit.data_ptr<float>() : nullptr;
    a.seq_idx = ids.defined() ? ids.data_ptr<int32_t>() : nullptr;
    const hipStream_t st = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(x.device().index()).stream();
    check_status(mamba2_ssd_bwd_m1(&a, ws.data_ptr(), ws_bytes, st), "mamba2_ssd_bwd_m1");
    return {dx, ddt, dA, dB, dC, dD, dz, ddt_bias, dinit};
}

std::tuple<Tensor, Tensor> state_passing(const Tensor &chunk_states, const Tensor &dA_cumsum,
                                         const optional<Tensor> &init) {
    const char *op = "mamba2_ssd_state_passing";
    // chunk_states in fp32 or fp16, the rest fp32, the states out in fp32
    // (the reference op's dtypes: op_host mamba2_ssd_state_passing.cpp:19-23, 50-53)
    const bool half = chunk_states.scalar_type() == at::kHalf;
    TORCH_CHECK(chunk_states.device().is_cuda(), op, ": chunk_states must be a ROCm GPU tensor (got device ",
                chunk_states.device().str(), ")");
    TORCH_CHECK(half || chunk_states.scalar_type() == at::kFloat, op,
                ": chunk_states must be float32 or float16 (got ", c10::toString(chunk_states.scalar_type()), ")");
    TORCH_CHECK(chunk_states.is_contiguous(), op, ": chunk_states must be contiguous");
    check_tensor(op, "dA_cumsum", dA_cumsum);
    TORCH_CHECK(chunk_states.dim() == 5, op, ": chunk_states must have shape [B,H,K,P,N]");
    const int64_t b = chunk_states.size(0), h = chunk_states.size(1), k = chunk_states.size(2),
                  p = chunk_states.size(3), n = chunk_states.size(4);
    TORCH_CHECK(dA_cumsum.dim() == 4 && dA_cumsum.size(0) == b && dA_cumsum.size(1) == h && dA_cumsum.size(2) == k,
                op, ": dA_cumsum must have shape [B,H,K,T]");
    if (init.has_value()) {
        check_tensor(op, "initial_states", *init);
        TORCH_CHECK(init->dim() == 4 && init->size(0) == b && init->size(1) == h && init->size(2) == p &&
                        init->size(3) == n,
                    op, ": initial_states must have shape [B,H,P,N]");
    }
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(chunk_states.device());
    const Tensor log_decay = dA_cumsum.select(3, dA_cumsum.size(3) - 1).contiguous();
    const auto f32 = chunk_states.options().dtype(at::kFloat);
    Tensor states = at::empty({b, h, k, p, n}, f32);
    Tensor final_state = at::empty({b, h, p, n}, f32);
    const hipStream_t st = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(chunk_states.device().index()).stream();
    if (half)
        check_status(mamba2_ssd_state_passing_f16(chunk_states.data_ptr(), log_decay.data_ptr<float>(), cptr(init),
                                                  states.data_ptr<float>(), final_state.data_ptr<float>(), b, h, k,
                                                  p, n, st),
                     op);
    else
        check_status(mamba2_ssd_state_passing(chunk_states.data_ptr<float>(), log_decay.data_ptr<float>(),
                                              cptr(init), states.data_ptr<float>(), final_state.data_ptr<float>(),
                                              b, h, k, p, n, st),
                     op);
    return {states, final_state};
}

// ----------------------------------------------------------------------- Meta
std::tuple<Tensor, Tensor, Tensor, Tensor> fwd_ex_meta(const Tensor &x, const Tensor &, const Tensor &,
                                                       const Tensor &B, const Tensor &, const optional<Tensor> &,
                                                       const optional<Tensor> &z, const optional<Tensor> &,
                                                       const optional<Tensor> &, int64_t, bool, double, double,
                                                       bool want_final, bool want_pre_gate, bool want_states) {
    const Tensor none = at::empty({0}, x.options());
    return {at::empty_like(x),
            want_final ? at::empty({x.size(0), x.size(2), x.size(3), B.size(3)}, x.options()) : none,
            (want_pre_gate && z.has_value()) ? at::empty_like(x) : none,
            want_states ? at::empty({x.size(0), x.size(2), nchunks(x), x.size(3), B.size(3)}, x.options()) : none};
}

std::tuple<Tensor, Tensor> fwd_meta(const Tensor &x, const Tensor &, const Tensor &, const Tensor &B, const Tensor &,
                                    const optional<Tensor> &, const optional<Tensor> &, const optional<Tensor> &,
                                    const optional<Tensor> &, int64_t, bool, double, double) {
    return {at::empty_like(x), at::empty({x.size(0), x.size(2), x.size(3), B.size(3)}, x.options())};
}

Grads bwd_meta(const Tensor &x, const Tensor &dt, const Tensor &A, const Tensor &B, const Tensor &C, const Tensor &,
               const optional<Tensor> &, const optional<Tensor> &D, const optional<Tensor> &z,
               const optional<Tensor> &dt_bias, const optional<Tensor> &init, const optional<Tensor> &,
               const optional<Tensor> &, int64_t, bool, double, double, const optional<Tensor> &) {
    auto like = [&](const optional<Tensor> &t) { return t.has_value() ? at::empty_like(*t) : at::empty({0}, x.options()); };
    return {at::empty_like(x), at::empty_like(dt), at::empty_like(A), at::empty_like(B), at::empty_like(C),
            like(D), like(z), like(dt_bias), like(init)};
}

std::tuple<Tensor, Tensor> state_passing_meta(const Tensor &cs, const Tensor &, const optional<Tensor> &) {
    const auto f32 = cs.options().dtype(at::kFloat);
    return {at::empty(cs.sizes(), f32), at::empty({cs.size(0), cs.size(1), cs.size(3), cs.size(4)}, f32)};
}

}  // namespace

TORCH_LIBRARY(mamba_ascend, m) {
    m.def("mamba2_ssd_fwd(Tensor x, Tensor dt, Tensor A, Tensor B, Tensor C, Tensor? D=None, "
          "Tensor? z=None, Tensor? dt_bias=None, Tensor? initial_states=None, int chunk_size=256, "
          "bool dt_softplus=False, float dt_limit_min=0.0, float dt_limit_max=3.402823466e+38) "
          "-> (Tensor, Tensor)");
    m.def("mamba2_ssd_bwd_m1(Tensor x, Tensor dt, Tensor A, Tensor B, Tensor C, Tensor dout, "
          "Tensor? dfinal_state=None, Tensor? D=None, Tensor? z=None, Tensor? dt_bias=None, "
          "Tensor? initial_states=None, Tensor? pre_gate=None, Tensor? chunk_states=None, "
          "int chunk_size=64, bool dt_softplus=False, float dt_limit_min=0.0, "
          "float dt_limit_max=3.402823466e+38, Tensor? seq_idx=None) "
          "-> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)");
    m.def("mamba2_ssd_state_passing(Tensor chunk_states, Tensor dA_cumsum, "
          "Tensor? initial_states=None) -> (Tensor, Tensor)");
    // this build's forward with the training outputs: (out, final_state,
    // pre_gate, chunk_states), absent ones empty
    m.def("mamba2_ssd_fwd_ex(Tensor x, Tensor dt, Tensor A, Tensor B, Tensor C, Tensor? D, Tensor? z, "
          "Tensor? dt_bias, Tensor? initial_states, int chunk_size, bool dt_softplus, float dt_limit_min, "
          "float dt_limit_max, bool want_final, bool want_pre_gate, bool want_states) "
          "-> (Tensor, Tensor, Tensor, Tensor)");
}

TORCH_LIBRARY_IMPL(mamba_ascend, CUDA, m) {
    m.impl("mamba2_ssd_fwd", &fwd);
    m.impl("mamba2_ssd_bwd_m1", &bwd);
    m.impl("mamba2_ssd_state_passing", &state_passing);
    m.impl("mamba2_ssd_fwd_ex", &fwd_ex);
}

// CPU tensors: the same functions, whose device check rejects them
TORCH_LIBRARY_IMPL(mamba_ascend, CPU, m) {
    m.impl("mamba2_ssd_fwd", &fwd);
    m.impl("mamba2_ssd_bwd_m1", &bwd);
    m.impl("mamba2_ssd_state_passing", &state_passing);
    m.impl("mamba2_ssd_fwd_ex", &fwd_ex);
}

TORCH_LIBRARY_IMPL(mamba_ascend, Meta, m) {
    m.impl("mamba2_ssd_fwd", &fwd_meta);
    m.impl("mamba2_ssd_bwd_m1", &bwd_meta);
    m.impl("mamba2_ssd_state_passing", &state_passing_meta);
    m.impl("mamba2_ssd_fwd_ex", &fwd_ex_meta);
}
