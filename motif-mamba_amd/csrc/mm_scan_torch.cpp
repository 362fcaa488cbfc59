// mm_scan_torch.cpp -- thin PyTorch-ROCm binding over the C ABI of libmm_scan.so.
//
// fwd(...)        mirrors selective_scan_cuda.fwd (reference csrc/selective_scan/selective_scan.cpp:
//                 270-413, pybind :620-627): same argument names, checks and outputs
//                 [out, x, out_z?], where x is the (batch, dim, ceil(L/2048), 2*dstate) float32
//                 chunk-state tensor of interleaved (prod a, h) pairs.
// fwd_infer(...)  the inference form used by SelectiveScanFn: writes only the returned output
//                 (out_z when z is given, else out) and, on request, a contiguous last_state.
// state_update(.) the decode step (replaces upstream selective_state_update, called at
//                 mamba_ssm/modules/mamba_simplemotif.py:397-399).
// Validation failures raise RuntimeError through TORCH_CHECK, like the reference binding.
// ROCm torch reports GPU tensors with device type "cuda"; the generic c10::DeviceGuard accepts it,
// and c10::hip::getCurrentHIPStream() is the stream torch launches its own HIP work on.
#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <cstdlib>
#include <vector>

#include "mm_conv1d.h"
#include "mm_norm.h"
#include "mm_scan.h"

namespace {

#define CHECK_SHAPE(x, ...) \
    TORCH_CHECK(x.sizes() == torch::IntArrayRef({__VA_ARGS__}), #x " must have shape (" #__VA_ARGS__ ")")

mm_dtype to_mm(at::ScalarType t) {
    switch (t) {
        case at::ScalarType::Float: return MM_FLOAT32;
        case at::ScalarType::Half: return MM_FLOAT16;
        case at::ScalarType::BFloat16: return MM_BFLOAT16;
        default: AT_ERROR("selective_scan_fwd not implemented for input type '", c10::toString(t), "'");
    }
}

void check_rc(int rc, const char *what) {
    if (rc == MM_ERR_UNSUPPORTED) {
        // A shape the kernels do not cover: NotImplementedError (a RuntimeError) in Python.
        throw c10::NotImplementedError({__func__, __FILE__, uint32_t(__LINE__)},
                                       c10::str(what, " failed (code ", rc, "): ", mm_last_error()));
    }
    TORCH_CHECK(rc == MM_OK, what, " failed (code ", rc, "): ", mm_last_error());
}

struct FwdSetup {
    mm_scan_fwd_params p;
    int64_t n_chunks;
};

// Shared validation (selective_scan.cpp:280-381, without the P/Q/gamma and complex branches,
// which attach_pq and the complex-A refusal below cover).
FwdSetup setup_fwd(const at::Tensor &u, const at::Tensor &delta, const at::Tensor &A, const at::Tensor &B,
                   const at::Tensor &C, const c10::optional<at::Tensor> &D_, const c10::optional<at::Tensor> &z_,
                   const c10::optional<at::Tensor> &delta_bias_, bool delta_softplus) {
    const auto input_type = u.scalar_type();
    const auto weight_type = A.scalar_type();
    TORCH_CHECK(input_type == at::ScalarType::Float || input_type == at::ScalarType::Half ||
                input_type == at::ScalarType::BFloat16);
    TORCH_CHECK(weight_type == at::ScalarType::Float || weight_type == at::ScalarType::ComplexFloat);
    if (weight_type == at::ScalarType::ComplexFloat) {
        throw c10::NotImplementedError({__func__, __FILE__, uint32_t(__LINE__)},
                                       "complex A is not supported by the MI355X selective scan");
    }
    const bool is_variable_B = B.dim() >= 3;
    const bool is_variable_C = C.dim() >= 3;
    TORCH_CHECK(delta.scalar_type() == input_type);
    TORCH_CHECK(B.scalar_type() == (!is_variable_B ? weight_type : input_type));
    TORCH_CHECK(C.scalar_type() == (!is_variable_C ? weight_type : input_type));
    TORCH_CHECK(u.is_cuda());
    TORCH_CHECK(delta.is_cuda());
    TORCH_CHECK(A.is_cuda());
    TORCH_CHECK(B.is_cuda());
    TORCH_CHECK(C.is_cuda());
    TORCH_CHECK(u.stride(-1) == 1 || u.size(-1) == 1);
    TORCH_CHECK(delta.stride(-1) == 1 || delta.size(-1) == 1);

    TORCH_CHECK(u.dim() == 3, "u must have shape (batch, dim, seqlen)");
    const int64_t batch_size = u.size(0), dim = u.size(1), seqlen = u.size(2);
    TORCH_CHECK(A.dim() == 2, "A must have shape (dim, dstate)");
    const int64_t dstate = A.size(1);
    TORCH_CHECK(!is_variable_B || B.dim() == 4, "variable B must be 4-D (batch, n_groups, dstate, seqlen)");
    const int64_t n_groups = is_variable_B ? B.size(1) : 1;
    TORCH_CHECK(dstate <= MM_SCAN_MAX_DSTATE, "selective_scan only supports state dimension <= 256");

    CHECK_SHAPE(u, batch_size, dim, seqlen);
    CHECK_SHAPE(delta, batch_size, dim, seqlen);
    CHECK_SHAPE(A, dim, dstate);
    if (!is_variable_B) {
        CHECK_SHAPE(B, dim, dstate);
    } else {
        CHECK_SHAPE(B, batch_size, n_groups, dstate, seqlen);
        TORCH_CHECK(B.stride(-1) == 1 || B.size(-1) == 1);
    }
    if (!is_variable_C) {
        CHECK_SHAPE(C, dim, dstate);
    } else {
        TORCH_CHECK(C.dim() == 4, "variable C must be 4-D (batch, n_groups, dstate, seqlen)");
        CHECK_SHAPE(C, batch_size, n_groups, dstate, seqlen);
        TORCH_CHECK(C.stride(-1) == 1 || C.size(-1) == 1);
    }
    TORCH_CHECK(n_groups >= 1 && dim % n_groups == 0, "dim must be a multiple of n_groups");
    if (D_.has_value()) {
        const auto &D = D_.value();
        TORCH_CHECK(D.scalar_type() == at::ScalarType::Float);
        TORCH_CHECK(D.is_cuda());
        TORCH_CHECK(D.stride(-1) == 1 || D.size(-1) == 1);
        CHECK_SHAPE(D, dim);
    }
    if (delta_bias_.has_value()) {
        const auto &db = delta_bias_.value();
        TORCH_CHECK(db.scalar_type() == at::ScalarType::Float);
        TORCH_CHECK(db.is_cuda());
        TORCH_CHECK(db.stride(-1) == 1 || db.size(-1) == 1);
        CHECK_SHAPE(db, dim);
    }
    if (z_.has_value()) {
        const auto &z = z_.value();
        TORCH_CHECK(z.scalar_type() == input_type);
        TORCH_CHECK(z.is_cuda());
        TORCH_CHECK(z.stride(-1) == 1 || z.size(-1) == 1);
        CHECK_SHAPE(z, batch_size, dim, seqlen);
    }

    FwdSetup s;
    std::memset(&s.p, 0, sizeof(s.p));
    mm_scan_fwd_params &p = s.p;
    p.batch = batch_size;
    p.dim = dim;
    p.seqlen = seqlen;
    p.dstate = dstate;
    p.n_groups = n_groups;
    p.itype = to_mm(input_type);
    p.is_variable_B = is_variable_B;
    p.is_variable_C = is_variable_C;
    p.delta_softplus = delta_softplus;
    p.u = u.data_ptr();
    p.delta = delta.data_ptr();
    p.A = A.data_ptr<float>();
    p.B = B.data_ptr();
    p.C = C.data_ptr();
    p.D = D_.has_value() ? D_.value().data_ptr<float>() : nullptr;
    p.z = z_.has_value() ? z_.value().data_ptr() : nullptr;
    p.delta_bias = delta_bias_.has_value() ? delta_bias_.value().data_ptr<float>() : nullptr;
    p.u_batch_stride = u.stride(0);
    p.u_d_stride = u.stride(1);
    p.delta_batch_stride = delta.stride(0);
    p.delta_d_stride = delta.stride(1);
    if (z_.has_value()) {
        p.z_batch_stride = z_.value().stride(0);
        p.z_d_stride = z_.value().stride(1);
    }
    p.A_d_stride = A.stride(0);
    p.A_dstate_stride = A.stride(1);
    if (is_variable_B) {
        p.B_batch_stride = B.stride(0);
        p.B_group_stride = B.stride(1);
        p.B_dstate_stride = B.stride(2);
    } else {
        p.B_d_stride = B.stride(0);
        p.B_dstate_stride = B.stride(1);
    }
    if (is_variable_C) {
        p.C_batch_stride = C.stride(0);
        p.C_group_stride = C.stride(1);
        p.C_dstate_stride = C.stride(2);
    } else {
        p.C_d_stride = C.stride(0);
        p.C_dstate_stride = C.stride(1);
    }
    s.n_chunks = (seqlen + MM_SCAN_CHUNK - 1) / MM_SCAN_CHUNK;
    return s;
}

void set_out(mm_scan_fwd_params &p, const at::Tensor &out) {
    p.out = out.data_ptr();
    p.out_batch_stride = out.stride(0);
    p.out_d_stride = out.stride(1);
}

void set_out_z(mm_scan_fwd_params &p, const at::Tensor &out_z) {
    p.out_z = out_z.data_ptr();
    p.out_z_batch_stride = out_z.stride(0);
    p.out_z_d_stride = out_z.stride(1);
}

// Low-rank coupling P/Q and gamma (checks of selective_scan.cpp:342-369, strides as
// set_ssm_params_fwd, selective_scan.cpp:149-164). P and Q are read as float32: the reference's
// dense kernel reinterprets them as float and its full-matrix path upcasts them with .float().
// gamma is validated and carried, not read (neither reference forward reads it). Returns the
// float32 P/Q the parameter block points at; the caller keeps them alive until the launch.
std::vector<at::Tensor> attach_pq(mm_scan_fwd_params &p, const at::Tensor &u, const c10::optional<at::Tensor> &P_,
                                  const c10::optional<at::Tensor> &Q_, const c10::optional<at::Tensor> &gamma_) {
    TORCH_CHECK(!P_.has_value() || Q_.has_value(), "Q must be provided when P is provided");
    TORCH_CHECK(!Q_.has_value() || P_.has_value(), "P must be provided when Q is provided");
    std::vector<at::Tensor> keep;
    if (P_.has_value()) {
        const at::Tensor &P = P_.value(), &Q = Q_.value();
        TORCH_CHECK(P.is_cuda() && Q.is_cuda(), "P and Q must be CUDA tensors");
        TORCH_CHECK(P.device() == u.device() && Q.device() == u.device(), "P and Q must be on the device of u");
        TORCH_CHECK(P.dim() == Q.dim() && (P.dim() == 2 || P.dim() == 3), "P/Q must be 2D or 3D with same rank");
        if (P.dim() == 2) {
            TORCH_CHECK(P.size(0) == p.dstate && Q.size(1) == p.dstate && P.size(1) == Q.size(0),
                        "Expect P(dstate, r), Q(r, dstate)");
        } else {
            TORCH_CHECK(P.size(0) == p.dim && Q.size(0) == p.dim, "P/Q dim mismatch");
            TORCH_CHECK(P.size(1) == p.dstate && Q.size(2) == p.dstate && P.size(2) == Q.size(1),
                        "Expect P(dim, dstate, r), Q(dim, r, dstate)");
        }
        TORCH_CHECK(P.size(-1) <= 8, "Current dense CUDA forward supports pq_rank <= 8");
        const at::Tensor Pf = P.to(at::ScalarType::Float), Qf = Q.to(at::ScalarType::Float);
        keep = {Pf, Qf};
        p.P = Pf.data_ptr<float>();
        p.Q = Qf.data_ptr<float>();
        p.pq_rank = P.size(-1);
        p.P_d_stride = P.dim() == 3 ? Pf.stride(0) : 0;
        p.P_dstate_stride = Pf.stride(P.dim() - 2);
        p.P_r_stride = Pf.stride(P.dim() - 1);
        p.Q_d_stride = Q.dim() == 3 ? Qf.stride(0) : 0;
        p.Q_r_stride = Qf.stride(Q.dim() - 2);
        p.Q_dstate_stride = Qf.stride(Q.dim() - 1);
    }
    if (gamma_.has_value()) {
        const at::Tensor &gamma = gamma_.value();
        TORCH_CHECK(gamma.is_cuda(), "gamma must be CUDA tensor");
        TORCH_CHECK(gamma.dim() == 1 || gamma.dim() == 2, "gamma must be 1D or 2D");
        if (gamma.dim() == 1) {
            TORCH_CHECK(gamma.size(0) == p.dstate, "gamma(1D) shape must be (dstate,)");
        } else {
            TORCH_CHECK(gamma.size(0) == p.dim && gamma.size(1) == p.dstate, "gamma(2D) shape must be (dim, dstate)");
        }
        p.gamma = static_cast<const float *>(gamma.data_ptr());
        p.gamma_d_stride = gamma.dim() == 2 ? gamma.stride(0) : 0;
        p.gamma_dstate_stride = gamma.stride(-1);
    }
    return keep;
}

// Scratch for the sequence-parallel segments (only for shapes that use them), from the caching
// allocator on the launch stream: released when the caller's reference drops, stream-ordered.
at::Tensor attach_workspace(mm_scan_fwd_params &p, const at::Tensor &like) {
    const int64_t bytes = mm_scan_fwd_workspace_size(&p);
    if (bytes <= 0) return at::Tensor();
    at::Tensor ws = torch::empty({bytes}, like.options().dtype(at::ScalarType::Byte));
    p.workspace = ws.data_ptr();
    p.workspace_bytes = bytes;
    return ws;
}

std::vector<at::Tensor> fwd(const at::Tensor &u, const at::Tensor &delta, const at::Tensor &A,
                            const at::Tensor &B, const at::Tensor &C, const c10::optional<at::Tensor> &D_,
                            const c10::optional<at::Tensor> &z_, const c10::optional<at::Tensor> &delta_bias_,
                            const c10::optional<at::Tensor> &P_, const c10::optional<at::Tensor> &Q_,
                            const c10::optional<at::Tensor> &gamma_, bool delta_softplus, bool tile_states) {
    FwdSetup s = setup_fwd(u, delta, A, B, C, D_, z_, delta_bias_, delta_softplus);
    mm_scan_fwd_params &p = s.p;
    const std::vector<at::Tensor> pq = attach_pq(p, u, P_, Q_, gamma_);
    // Output layouts follow the reference: out like delta, out_z like z (like out when z is a
    // non-dense view such as half of xz), x contiguous.
    at::Tensor out = torch::empty_like(delta);
    at::Tensor x = torch::empty({p.batch, p.dim, s.n_chunks, p.dstate * 2}, u.options().dtype(A.scalar_type()));
    at::Tensor out_z;
    set_out(p, out);
    if (z_.has_value()) {
        out_z = z_.value().is_non_overlapping_and_dense() ? torch::empty_like(z_.value()) : torch::empty_like(out);
        set_out_z(p, out_z);
    }
    p.chunk_states = x.data_ptr<float>();
    // tile_states (this build's addition): the states before every 16-step tile, appended to the
    // outputs for the backward -- None when the kernels cannot write them for this request (the
    // query sees the final parameter block, outputs included).
    at::Tensor ck;
    if (tile_states && mm_scan_fwd_tile_states_size(&p) > 0) {
        ck = torch::empty({(p.seqlen + 15) / 16, p.batch, p.dim, 16}, u.options().dtype(at::ScalarType::Float));
        p.tile_states = ck.data_ptr<float>();
    }
    const c10::DeviceGuard device_guard{u.device()};
    const at::Tensor ws = attach_workspace(p, u);
    check_rc(mm_scan_fwd(&p, c10::hip::getCurrentHIPStream().stream()), "mm_scan_fwd");
    std::vector<at::Tensor> result = {out, x};
    if (z_.has_value()) result.push_back(out_z);
    if (tile_states) result.push_back(ck);
    return result;
}

// Shortest lengths (not multiples of 8) that fwd_infer pads for the fast kernels.
constexpr int64_t kMinPaddedDiag = 14, kMinPaddedPQ = 5;

std::vector<at::Tensor> fwd_infer(const at::Tensor &u, const at::Tensor &delta, const at::Tensor &A,
                                  const at::Tensor &B, const at::Tensor &C, const c10::optional<at::Tensor> &D_,
                                  const c10::optional<at::Tensor> &z_,
                                  const c10::optional<at::Tensor> &delta_bias_, bool delta_softplus,
                                  bool return_last_state, const c10::optional<at::Tensor> &P_,
                                  const c10::optional<at::Tensor> &Q_, const c10::optional<at::Tensor> &gamma_) {
    FwdSetup s = setup_fwd(u, delta, A, B, C, D_, z_, delta_bias_, delta_softplus);
    mm_scan_fwd_params &p = s.p;
    const std::vector<at::Tensor> pq = attach_pq(p, u, P_, Q_, gamma_);
    // A length that is not a multiple of 8 keeps a request off the fast kernels (their lanes move
    // vectors of 2 to 8 steps) and on the general one, ~14x slower at the Mamba-2.8B layer shape.
    // Such requests run on copies padded in front to a multiple of 32 steps with u, delta, z, B and
    // C zero: from the zero initial state a step with u = 0 leaves the state exactly zero, whatever
    // its decay (and, with P/Q, whatever the coupling), so the real steps run the recurrence of the
    // unpadded request; the outputs are the padded call's last L steps, the last state its own.
    // MM_SCAN_PAD=0 turns this off (read per call: the tests run the general kernels with it).
    // Short requests stay on the general kernels: the padded call's five pad copies, allocations
    // and output copy cost ~50 us of host time, more than the general kernels take for a few
    // steps (measured, bf16, batch 1 and 64: the diagonal general kernel is as fast up to L 13 at
    // 5,120 channels, the P/Q one up to L 4 at 2,048; the Motif decode step calls the P/Q scan
    // with L 1: 17 us against 58 us padded).
    const char *pad_env = std::getenv("MM_SCAN_PAD");
    const bool pad_off = pad_env && pad_env[0] == '0';
    const bool fast_shape = p.is_variable_B && p.is_variable_C && p.dim % 16 == 0 &&
                            (p.dim / p.n_groups) % 16 == 0 && p.dstate <= 64;   // diagonal or P/Q
    const int64_t min_padded = p.P ? kMinPaddedPQ : kMinPaddedDiag;
    if (!pad_off && fast_shape && p.seqlen % 8 != 0 && p.seqlen >= min_padded) {
        const int64_t L = p.seqlen, pad = (L + 31) / 32 * 32 - L;
        auto front = [&](const at::Tensor &t) { return at::constant_pad_nd(t, {pad, 0}, 0); };
        const c10::optional<at::Tensor> zp = z_.has_value() ? c10::optional<at::Tensor>(front(z_.value()))
                                                            : c10::optional<at::Tensor>();
        std::vector<at::Tensor> res = fwd_infer(front(u), front(delta), A, front(B), front(C), D_, zp, delta_bias_,
                                                delta_softplus, return_last_state, P_, Q_, gamma_);
        res[0] = res[0].narrow(-1, pad, L).contiguous();
        return res;
    }
    at::Tensor main;
    if (z_.has_value()) {
        main = z_.value().is_non_overlapping_and_dense() ? torch::empty_like(z_.value()) : torch::empty_like(delta);
        set_out_z(p, main);
    } else {
        main = torch::empty_like(delta);
        set_out(p, main);
    }
    at::Tensor last_state;
    if (return_last_state) {
        last_state = torch::empty({p.batch, p.dim, p.dstate}, u.options().dtype(at::ScalarType::Float));
        p.last_state = last_state.data_ptr<float>();
    }
    const c10::DeviceGuard device_guard{u.device()};
    const at::Tensor ws = attach_workspace(p, u);
    check_rc(mm_scan_fwd(&p, c10::hip::getCurrentHIPStream().stream()), "mm_scan_fwd");
    if (return_last_state) return {main, last_state};
    return {main};
}


// selective_scan_cuda.bwd (selective_scan.cpp:415-612): [du, ddelta, dA, dB, dC, dD, ddelta_bias,
// dz?, out_z?]. x (the forward's chunk states) is checked like the reference but not read: the
// backward recomputes the forward states itself. With P/Q the exact gradient of the coupled
// recurrence runs (pq_rank 1..8, dstate <= 16, dim and dim / n_groups multiples of 16; other
// P/Q shapes raise).
std::vector<at::Tensor> bwd(const at::Tensor &u, const at::Tensor &delta, const at::Tensor &A, const at::Tensor &B,
                            const at::Tensor &C, const c10::optional<at::Tensor> &D_,
                            const c10::optional<at::Tensor> &z_, const c10::optional<at::Tensor> &delta_bias_,
                            const c10::optional<at::Tensor> &P_, const c10::optional<at::Tensor> &Q_,
                            const c10::optional<at::Tensor> &gamma_, const at::Tensor &dout,
                            const c10::optional<at::Tensor> &x_, const c10::optional<at::Tensor> &out_,
                            c10::optional<at::Tensor> dz_, const c10::optional<at::Tensor> &dP_out_,
                            const c10::optional<at::Tensor> &dQ_out_, bool delta_softplus, bool recompute_out_z,
                            const c10::optional<at::Tensor> &tile_states_) {
    FwdSetup s = setup_fwd(u, delta, A, B, C, D_, z_, delta_bias_, delta_softplus);
    // P/Q (and gamma, validated and not read, as in the forward): the float32 copies stay alive
    // until the launch is enqueued.
    const std::vector<at::Tensor> pq_keep = attach_pq(s.p, u, P_, Q_, gamma_);
    const mm_scan_fwd_params &f = s.p;
    // Rank-0 P/Q couple nothing: their forward is the diagonal scan and so is the backward (dP and
    // dQ are empty).
    const bool has_pq = P_.has_value() && f.pq_rank > 0;
    TORCH_CHECK(P_.has_value() || (!dP_out_.has_value() && !dQ_out_.has_value()), "dP_out and dQ_out need P and Q");
    (void)pq_keep;
    TORCH_CHECK(dout.scalar_type() == u.scalar_type());
    TORCH_CHECK(dout.is_cuda());
    TORCH_CHECK(dout.stride(-1) == 1 || dout.size(-1) == 1);
    CHECK_SHAPE(dout, f.batch, f.dim, f.seqlen);
    at::Tensor out, dz, out_z;
    const bool has_z = z_.has_value();
    if (has_z) {
        TORCH_CHECK(out_.has_value());
        out = out_.value();
        TORCH_CHECK(out.scalar_type() == u.scalar_type());
        TORCH_CHECK(out.is_cuda());
        TORCH_CHECK(out.stride(-1) == 1 || out.size(-1) == 1);
        CHECK_SHAPE(out, f.batch, f.dim, f.seqlen);
        if (dz_.has_value()) {
            dz = dz_.value();
            TORCH_CHECK(dz.scalar_type() == u.scalar_type());
            TORCH_CHECK(dz.is_cuda());
            TORCH_CHECK(dz.stride(-1) == 1 || dz.size(-1) == 1);
            CHECK_SHAPE(dz, f.batch, f.dim, f.seqlen);
        } else {
            dz = torch::empty_like(z_.value());
        }
        if (recompute_out_z) out_z = torch::empty_like(out);
    }
    if (s.n_chunks > 1) TORCH_CHECK(x_.has_value());
    if (x_.has_value()) {
        const at::Tensor &x = x_.value();
        TORCH_CHECK(x.scalar_type() == A.scalar_type());
        TORCH_CHECK(x.is_cuda());
        TORCH_CHECK(x.is_contiguous());
        CHECK_SHAPE(x, f.batch, f.dim, s.n_chunks, 2 * f.dstate);
    }
    at::Tensor du = torch::empty_like(u);
    at::Tensor ddelta = torch::empty_like(delta);
    at::Tensor dA = torch::empty_like(A);
    at::Tensor dB = torch::empty(B.sizes(), B.options().dtype(at::ScalarType::Float));
    at::Tensor dC = torch::empty(C.sizes(), C.options().dtype(at::ScalarType::Float));
    at::Tensor dD, ddelta_bias;
    if (D_.has_value()) dD = torch::empty_like(D_.value());
    if (delta_bias_.has_value()) ddelta_bias = torch::empty_like(delta_bias_.value());

    mm_scan_bwd_params p;
    std::memset(&p, 0, sizeof(p));
    p.batch = f.batch; p.dim = f.dim; p.seqlen = f.seqlen; p.dstate = f.dstate; p.n_groups = f.n_groups;
    p.itype = f.itype; p.is_variable_B = f.is_variable_B; p.is_variable_C = f.is_variable_C;
    p.delta_softplus = f.delta_softplus;
    p.u = f.u; p.delta = f.delta; p.A = f.A; p.B = f.B; p.C = f.C; p.D = f.D; p.z = f.z; p.delta_bias = f.delta_bias;
    p.u_batch_stride = f.u_batch_stride; p.u_d_stride = f.u_d_stride;
    p.delta_batch_stride = f.delta_batch_stride; p.delta_d_stride = f.delta_d_stride;
    p.z_batch_stride = f.z_batch_stride; p.z_d_stride = f.z_d_stride;
    p.A_d_stride = f.A_d_stride; p.A_dstate_stride = f.A_dstate_stride;
    p.B_batch_stride = f.B_batch_stride; p.B_group_stride = f.B_group_stride;
    p.B_dstate_stride = f.B_dstate_stride; p.B_d_stride = f.B_d_stride;
    p.C_batch_stride = f.C_batch_stride; p.C_group_stride = f.C_group_stride;
    p.C_dstate_stride = f.C_dstate_stride; p.C_d_stride = f.C_d_stride;
    p.dout = dout.data_ptr();
    p.dout_batch_stride = dout.stride(0); p.dout_d_stride = dout.stride(1);
    if (has_z) {
        p.out = out.data_ptr(); p.out_batch_stride = out.stride(0); p.out_d_stride = out.stride(1);
        p.dz = dz.data_ptr(); p.dz_batch_stride = dz.stride(0); p.dz_d_stride = dz.stride(1);
        if (recompute_out_z) {
            p.out_z = out_z.data_ptr(); p.out_z_batch_stride = out_z.stride(0); p.out_z_d_stride = out_z.stride(1);
        }
    }
    p.du = du.data_ptr(); p.du_batch_stride = du.stride(0); p.du_d_stride = du.stride(1);
    p.ddelta = ddelta.data_ptr(); p.ddelta_batch_stride = ddelta.stride(0); p.ddelta_d_stride = ddelta.stride(1);
    p.dA = dA.data_ptr<float>(); p.dA_d_stride = dA.stride(0); p.dA_dstate_stride = dA.stride(1);
    p.dB = dB.data_ptr<float>();
    p.dC = dC.data_ptr<float>();
    if (f.is_variable_B) {
        p.dB_batch_stride = dB.stride(0); p.dB_group_stride = dB.stride(1); p.dB_dstate_stride = dB.stride(2);
    } else {
        p.dB_d_stride = dB.stride(0); p.dB_dstate_stride = dB.stride(1);
    }
    if (f.is_variable_C) {
        p.dC_batch_stride = dC.stride(0); p.dC_group_stride = dC.stride(1); p.dC_dstate_stride = dC.stride(2);
    } else {
        p.dC_d_stride = dC.stride(0); p.dC_dstate_stride = dC.stride(1);
    }
    if (D_.has_value()) p.dD = dD.data_ptr<float>();
    if (delta_bias_.has_value()) p.ddelta_bias = ddelta_bias.data_ptr<float>();
    // dP / dQ (selective_scan.cpp:580-590): the exact gradients of the coupled recurrence are
    // added into dP_out / dQ_out (float32, the shapes of P and Q) when given, as the reference
    // accumulates into them; without them they are computed and dropped, as there, and the
    // result list is the reference's either way.
    at::Tensor dP, dQ;
    if (has_pq) {
        const at::Tensor &P = P_.value(), &Q = Q_.value();
        if (dP_out_.has_value() || dQ_out_.has_value()) {
            TORCH_CHECK(dP_out_.has_value() && dQ_out_.has_value(), "dP_out and dQ_out go together");
            const at::Tensor &dPo = dP_out_.value(), &dQo = dQ_out_.value();
            TORCH_CHECK(dPo.is_cuda() && dQo.is_cuda(), "dP_out and dQ_out must be CUDA tensors");
            TORCH_CHECK(dPo.scalar_type() == at::ScalarType::Float && dQo.scalar_type() == at::ScalarType::Float,
                        "dP_out and dQ_out must be float32");
            TORCH_CHECK(dPo.sizes() == P.sizes(), "dP_out shape mismatch");
            TORCH_CHECK(dQo.sizes() == Q.sizes(), "dQ_out shape mismatch");
        }
        dP = torch::empty(P.sizes(), P.options().dtype(at::ScalarType::Float));
        dQ = torch::empty(Q.sizes(), Q.options().dtype(at::ScalarType::Float));
        p.P = f.P; p.Q = f.Q; p.pq_rank = f.pq_rank;
        p.P_d_stride = f.P_d_stride; p.P_dstate_stride = f.P_dstate_stride; p.P_r_stride = f.P_r_stride;
        p.Q_d_stride = f.Q_d_stride; p.Q_r_stride = f.Q_r_stride; p.Q_dstate_stride = f.Q_dstate_stride;
        p.dP = dP.data_ptr<float>();
        p.dQ = dQ.data_ptr<float>();
        p.dP_d_stride = P.dim() == 3 ? dP.stride(0) : 0;
        p.dP_dstate_stride = dP.stride(P.dim() - 2);
        p.dP_r_stride = dP.stride(P.dim() - 1);
        p.dQ_d_stride = Q.dim() == 3 ? dQ.stride(0) : 0;
        p.dQ_r_stride = dQ.stride(Q.dim() - 2);
        p.dQ_dstate_stride = dQ.stride(Q.dim() - 1);
    }
    if (tile_states_.has_value()) {
        const at::Tensor &ck = tile_states_.value();
        TORCH_CHECK(ck.is_cuda() && ck.scalar_type() == at::ScalarType::Float && ck.is_contiguous() &&
                        ck.sizes() == at::IntArrayRef({(f.seqlen + 15) / 16, f.batch, f.dim, 16}),
                    "tile_states must be the contiguous float32 (ceil(L / 16), batch, dim, 16) tensor of the forward");
        p.tile_states = ck.data_ptr<float>();
    }
    const c10::DeviceGuard device_guard{u.device()};
    at::Tensor ws;
    const int64_t ws_bytes = mm_scan_bwd_workspace_size(&p);
    if (ws_bytes > 0) {
        ws = torch::empty({ws_bytes}, u.options().dtype(at::ScalarType::Byte));
        p.workspace = ws.data_ptr();
        p.workspace_bytes = ws_bytes;
    }
    check_rc(mm_scan_bwd(&p, c10::hip::getCurrentHIPStream().stream()), "mm_scan_bwd");
    std::vector<at::Tensor> result = {du, ddelta, dA, dB.to(B.scalar_type()), dC.to(C.scalar_type()), dD, ddelta_bias};
    if (has_z) result.push_back(dz);
    if (recompute_out_z) result.push_back(out_z);
    if (has_pq && dP_out_.has_value()) {
        dP_out_.value().add_(dP);
        dQ_out_.value().add_(dQ);
    }
    return result;
}


mm_dtype conv_dtype(const at::Tensor &t, const char *what) {
    const auto st = t.scalar_type();
    TORCH_CHECK(st == at::ScalarType::Float || st == at::ScalarType::Half || st == at::ScalarType::BFloat16,
                what, " must be float32, float16 or bfloat16");
    return to_mm(st);
}

// causal_conv1d_fwd (package causal-conv1d; fallback mamba_simplemotif.py:298-299): out (written into
// `out` when given, in any layout contiguous along seqlen), and the last width - 1 inputs into
// final_states_out when given.
at::Tensor conv1d_fwd(const at::Tensor &x, const at::Tensor &weight, const c10::optional<at::Tensor> &bias_,
                      const c10::optional<at::Tensor> &initial_states_, const c10::optional<at::Tensor> &final_states_out_,
                      bool silu, const c10::optional<at::Tensor> &out_) {
    TORCH_CHECK(x.is_cuda() && weight.is_cuda(), "x and weight must be on the GPU");
    TORCH_CHECK(x.dim() == 3, "x must have shape (batch, dim, seqlen)");
    TORCH_CHECK(x.stride(-1) == 1 || x.size(-1) == 1, "x must be contiguous along seqlen");
    const int64_t batch = x.size(0), dim = x.size(1), seqlen = x.size(2);
    TORCH_CHECK(weight.dim() == 2 && weight.size(0) == dim, "weight must have shape (dim, width)");
    const int64_t width = weight.size(1);
    TORCH_CHECK(width >= 1 && width <= MM_CONV1D_MAX_WIDTH, "width must be between 1 and 8");
    at::Tensor out;
    if (out_.has_value()) {
        out = out_.value();
        CHECK_SHAPE(out, batch, dim, seqlen);
        TORCH_CHECK(out.is_cuda() && out.scalar_type() == x.scalar_type(), "out must have the dtype of x");
        TORCH_CHECK(out.stride(-1) == 1 || seqlen == 1, "out must be contiguous along seqlen");
    } else {
        out = torch::empty_like(x);
    }
    mm_conv1d_fwd_params p;
    std::memset(&p, 0, sizeof(p));
    p.batch = batch; p.dim = dim; p.seqlen = seqlen; p.width = width;
    p.itype = conv_dtype(x, "x");
    p.wtype = conv_dtype(weight, "weight");
    p.silu = silu;
    p.x = x.data_ptr(); p.x_batch_stride = x.stride(0); p.x_d_stride = x.stride(1);
    p.out = out.data_ptr(); p.out_batch_stride = out.stride(0); p.out_d_stride = out.stride(1);
    p.weight = weight.data_ptr(); p.weight_d_stride = weight.stride(0); p.weight_w_stride = weight.stride(1);
    if (bias_.has_value()) {
        const at::Tensor &bias = bias_.value();
        TORCH_CHECK(bias.is_cuda() && bias.dim() == 1 && bias.size(0) == dim, "bias must have shape (dim,)");
        TORCH_CHECK(bias.scalar_type() == weight.scalar_type(), "bias must have the dtype of weight");
        p.bias = bias.data_ptr(); p.bias_stride = bias.stride(0);
    }
    if (initial_states_.has_value()) {
        const at::Tensor &ini = initial_states_.value();
        TORCH_CHECK(ini.is_cuda() && ini.dim() == 3 && ini.size(0) == batch && ini.size(1) == dim && ini.size(2) == width - 1,
                    "initial_states must have shape (batch, dim, width - 1)");
        TORCH_CHECK(ini.scalar_type() == x.scalar_type(), "initial_states must have the dtype of x");
        p.initial_states = ini.data_ptr();
        p.init_batch_stride = ini.stride(0); p.init_d_stride = ini.stride(1); p.init_w_stride = ini.stride(2);
    }
    if (final_states_out_.has_value()) {
        const at::Tensor &fin = final_states_out_.value();
        TORCH_CHECK(fin.is_cuda() && fin.dim() == 3 && fin.size(0) == batch && fin.size(1) == dim && fin.size(2) == width - 1,
                    "final_states_out must have shape (batch, dim, width - 1)");
        TORCH_CHECK(fin.scalar_type() == x.scalar_type(), "final_states_out must have the dtype of x");
        p.final_states = fin.data_ptr();
        p.final_batch_stride = fin.stride(0); p.final_d_stride = fin.stride(1); p.final_w_stride = fin.stride(2);
    }
    const c10::DeviceGuard device_guard{x.device()};
    check_rc(mm_causal_conv1d_fwd(&p, c10::hip::getCurrentHIPStream().stream()), "mm_causal_conv1d_fwd");
    return out;
}

// causal_conv1d_bwd (package causal-conv1d, as MambaInnerFn.backward calls it,
// selective_scan_interface.py:635-637): [dx, dweight, dbias?] for the gradient dout of the forward's
// output; dx is written into dx_out when given (MambaInnerFn passes a slice of dxz). dweight and dbias
// are summed in float32 and returned in the dtypes of weight and bias.
std::vector<at::Tensor> conv1d_bwd(const at::Tensor &x, const at::Tensor &weight, const c10::optional<at::Tensor> &bias_,
                                   const at::Tensor &dout, const c10::optional<at::Tensor> &dx_out_, bool silu) {
    TORCH_CHECK(x.is_cuda() && weight.is_cuda() && dout.is_cuda(), "x, weight and dout must be on the GPU");
    TORCH_CHECK(x.dim() == 3, "x must have shape (batch, dim, seqlen)");
    TORCH_CHECK(x.stride(-1) == 1 || x.size(-1) == 1, "x must be contiguous along seqlen");
    const int64_t batch = x.size(0), dim = x.size(1), seqlen = x.size(2);
    TORCH_CHECK(weight.dim() == 2 && weight.size(0) == dim, "weight must have shape (dim, width)");
    const int64_t width = weight.size(1);
    TORCH_CHECK(width >= 1 && width <= MM_CONV1D_MAX_WIDTH, "width must be between 1 and 8");
    CHECK_SHAPE(dout, batch, dim, seqlen);
    TORCH_CHECK(dout.scalar_type() == x.scalar_type(), "dout must have the dtype of x");
    TORCH_CHECK(dout.stride(-1) == 1 || seqlen == 1, "dout must be contiguous along seqlen");
    at::Tensor dx;
    if (dx_out_.has_value()) {
        dx = dx_out_.value();
        CHECK_SHAPE(dx, batch, dim, seqlen);
        TORCH_CHECK(dx.is_cuda() && dx.scalar_type() == x.scalar_type(), "dx must have the dtype of x");
        TORCH_CHECK(dx.stride(-1) == 1 || seqlen == 1, "dx must be contiguous along seqlen");
    } else {
        dx = torch::empty_like(x);
    }
    at::Tensor dweight = torch::empty({dim, width}, x.options().dtype(at::kFloat));
    at::Tensor dbias;
    mm_conv1d_bwd_params p;
    std::memset(&p, 0, sizeof(p));
    p.batch = batch; p.dim = dim; p.seqlen = seqlen; p.width = width;
    p.itype = conv_dtype(x, "x");
    p.wtype = conv_dtype(weight, "weight");
    p.silu = silu;
    p.x = x.data_ptr(); p.x_batch_stride = x.stride(0); p.x_d_stride = x.stride(1);
    p.dout = dout.data_ptr(); p.dout_batch_stride = dout.stride(0); p.dout_d_stride = dout.stride(1);
    p.dx = dx.data_ptr(); p.dx_batch_stride = dx.stride(0); p.dx_d_stride = dx.stride(1);
    p.weight = weight.data_ptr(); p.weight_d_stride = weight.stride(0); p.weight_w_stride = weight.stride(1);
    p.dweight = dweight.data_ptr<float>();
    if (bias_.has_value()) {
        const at::Tensor &bias = bias_.value();
        TORCH_CHECK(bias.is_cuda() && bias.dim() == 1 && bias.size(0) == dim, "bias must have shape (dim,)");
        TORCH_CHECK(bias.scalar_type() == weight.scalar_type(), "bias must have the dtype of weight");
        p.bias = bias.data_ptr(); p.bias_stride = bias.stride(0);
        dbias = torch::empty({dim}, x.options().dtype(at::kFloat));
        p.dbias = dbias.data_ptr<float>();
    }
    const c10::DeviceGuard device_guard{x.device()};
    check_rc(mm_causal_conv1d_bwd(&p, c10::hip::getCurrentHIPStream().stream()), "mm_causal_conv1d_bwd");
    std::vector<at::Tensor> res{dx, dweight.to(weight.scalar_type())};
    if (dbias.defined()) res.push_back(dbias.to(bias_.value().scalar_type()));
    return res;
}

// causal_conv1d_update (package causal-conv1d; fallback mamba_simplemotif.py:353-358): x (batch, dim)
// or (batch, dim, seqlen), conv_state (batch, dim, state_len) updated in place.
at::Tensor conv1d_update(const at::Tensor &x, const at::Tensor &conv_state, const at::Tensor &weight,
                         const c10::optional<at::Tensor> &bias_, bool silu) {
    TORCH_CHECK(x.is_cuda() && conv_state.is_cuda() && weight.is_cuda(), "x, conv_state and weight must be on the GPU");
    TORCH_CHECK(x.dim() == 2 || x.dim() == 3, "x must have shape (batch, dim) or (batch, dim, seqlen)");
    const at::Tensor x3 = x.dim() == 2 ? x.unsqueeze(-1) : x;
    const int64_t batch = x3.size(0), dim = x3.size(1), seqlen = x3.size(2);
    TORCH_CHECK(weight.dim() == 2 && weight.size(0) == dim, "weight must have shape (dim, width)");
    const int64_t width = weight.size(1);
    TORCH_CHECK(width >= 1 && width <= MM_CONV1D_MAX_WIDTH, "width must be between 1 and 8");
    TORCH_CHECK(conv_state.dim() == 3 && conv_state.size(0) == batch && conv_state.size(1) == dim,
                "conv_state must have shape (batch, dim, state_len)");
    TORCH_CHECK(conv_state.size(2) >= width - 1, "conv_state must hold at least width - 1 steps");
    at::Tensor out = torch::empty_like(x3);
    mm_conv1d_update_params p;
    std::memset(&p, 0, sizeof(p));
    p.batch = batch; p.dim = dim; p.seqlen = seqlen; p.width = width; p.state_len = conv_state.size(2);
    p.itype = conv_dtype(x, "x");
    p.wtype = conv_dtype(weight, "weight");
    p.stype = conv_dtype(conv_state, "conv_state");
    p.silu = silu;
    p.x = x3.data_ptr(); p.x_batch_stride = x3.stride(0); p.x_d_stride = x3.stride(1); p.x_l_stride = x3.stride(2);
    p.conv_state = conv_state.data_ptr();
    p.state_batch_stride = conv_state.stride(0); p.state_d_stride = conv_state.stride(1);
    p.state_l_stride = conv_state.stride(2);
    p.out = out.data_ptr(); p.out_batch_stride = out.stride(0); p.out_d_stride = out.stride(1);
    p.out_l_stride = out.stride(2);
    p.weight = weight.data_ptr(); p.weight_d_stride = weight.stride(0); p.weight_w_stride = weight.stride(1);
    if (bias_.has_value()) {
        const at::Tensor &bias = bias_.value();
        TORCH_CHECK(bias.is_cuda() && bias.dim() == 1 && bias.size(0) == dim, "bias must have shape (dim,)");
        TORCH_CHECK(bias.scalar_type() == weight.scalar_type(), "bias must have the dtype of weight");
        p.bias = bias.data_ptr(); p.bias_stride = bias.stride(0);
    }
    const c10::DeviceGuard device_guard{x.device()};
    check_rc(mm_causal_conv1d_update(&p, c10::hip::getCurrentHIPStream().stream()), "mm_causal_conv1d_update");
    return x.dim() == 2 ? out.squeeze(-1) : out;
}

// rms_norm_forward (selective_scan_interface.py:217-234) over dim 1 of a 3-D x (n0, cols, n2), in
// the layout the scan reads: out[i0, :, i2] = x[i0, :, i2] * weight / rms. out is a new tensor with
// x's shape and dtype (x's layout when x is dense), or the given `out` (which may be x itself).
at::Tensor rms_norm_fwd(const at::Tensor &x, const at::Tensor &weight, double eps,
                        const c10::optional<at::Tensor> &out_) {
    TORCH_CHECK(x.is_cuda() && weight.is_cuda(), "x and weight must be on the GPU");
    TORCH_CHECK(x.dim() == 3, "x must have shape (n0, cols, n2)");
    const int64_t n0 = x.size(0), cols = x.size(1), n2 = x.size(2);
    CHECK_SHAPE(weight, cols);
    at::Tensor out = out_.has_value() ? out_.value() : torch::empty_like(x);
    CHECK_SHAPE(out, n0, cols, n2);
    TORCH_CHECK(out.is_cuda() && out.scalar_type() == x.scalar_type(), "out must have the dtype of x");
    mm_rms_norm_params p;
    std::memset(&p, 0, sizeof(p));
    p.n0 = n0; p.cols = cols; p.n2 = n2;
    p.itype = conv_dtype(x, "x");
    p.wtype = conv_dtype(weight, "weight");
    p.eps = static_cast<float>(eps);
    p.x = x.data_ptr(); p.weight = weight.data_ptr(); p.out = out.data_ptr();
    p.x_stride0 = x.stride(0); p.x_stride_c = x.stride(1); p.x_stride2 = x.stride(2);
    p.out_stride0 = out.stride(0); p.out_stride_c = out.stride(1); p.out_stride2 = out.stride(2);
    p.weight_stride = weight.stride(0);
    const c10::DeviceGuard device_guard{x.device()};
    check_rc(mm_rms_norm_fwd(&p, c10::hip::getCurrentHIPStream().stream()), "mm_rms_norm_fwd");
    return out;
}

at::Tensor state_update(const at::Tensor &state, const at::Tensor &x, const at::Tensor &dt, const at::Tensor &A,
                        const at::Tensor &B, const at::Tensor &C, const c10::optional<at::Tensor> &D_,
                        const c10::optional<at::Tensor> &z_, const c10::optional<at::Tensor> &dt_bias_,
                        bool dt_softplus) {
    TORCH_CHECK(state.dim() == 3, "state must have shape (batch, dim, dstate)");
    auto float_type = [](at::ScalarType t) {
        return t == at::ScalarType::Float || t == at::ScalarType::Half || t == at::ScalarType::BFloat16;
    };
    TORCH_CHECK(float_type(state.scalar_type()), "state must be float32, float16 or bfloat16");
    const int64_t batch = state.size(0), dim = state.size(1), dstate = state.size(2);
    const auto itype = x.scalar_type();
    TORCH_CHECK(state.is_cuda() && x.is_cuda() && dt.is_cuda() && A.is_cuda() && B.is_cuda() && C.is_cuda());
    CHECK_SHAPE(x, batch, dim);
    CHECK_SHAPE(dt, batch, dim);
    CHECK_SHAPE(A, dim, dstate);
    TORCH_CHECK(dt.scalar_type() == itype, "dt must have the dtype of x");
    TORCH_CHECK(A.scalar_type() == at::ScalarType::Float, "A must be float32");
    TORCH_CHECK(B.dim() == 2 || B.dim() == 3, "B must be (batch, dstate) or (batch, n_groups, dstate)");
    TORCH_CHECK(C.dim() == B.dim(), "B and C must have the same rank");
    const int64_t n_groups = B.dim() == 3 ? B.size(1) : 1;
    if (B.dim() == 2) {
        CHECK_SHAPE(B, batch, dstate);
        CHECK_SHAPE(C, batch, dstate);
    } else {
        CHECK_SHAPE(B, batch, n_groups, dstate);
        CHECK_SHAPE(C, batch, n_groups, dstate);
    }
    TORCH_CHECK(B.scalar_type() == itype && C.scalar_type() == itype, "B and C must have the dtype of x");
    TORCH_CHECK(n_groups >= 1 && dim % n_groups == 0, "dim must be a multiple of n_groups");
    if (D_.has_value()) {
        CHECK_SHAPE(D_.value(), dim);
        TORCH_CHECK(float_type(D_.value().scalar_type()) && D_.value().is_cuda(),
                    "D must be float32, float16 or bfloat16 on the GPU");
    }
    if (dt_bias_.has_value()) {
        CHECK_SHAPE(dt_bias_.value(), dim);
        TORCH_CHECK(float_type(dt_bias_.value().scalar_type()) && dt_bias_.value().is_cuda(),
                    "dt_bias must be float32, float16 or bfloat16 on the GPU");
    }
    if (z_.has_value()) {
        CHECK_SHAPE(z_.value(), batch, dim);
        TORCH_CHECK(z_.value().scalar_type() == itype && z_.value().is_cuda(), "z must have the dtype of x");
    }
    at::Tensor out = torch::empty({batch, dim}, x.options());
    at::Tensor Dc = D_.has_value() ? D_.value().contiguous() : at::Tensor();
    at::Tensor bc = dt_bias_.has_value() ? dt_bias_.value().contiguous() : at::Tensor();

    mm_state_update_params p;
    std::memset(&p, 0, sizeof(p));
    p.batch = batch;
    p.dim = dim;
    p.dstate = dstate;
    p.n_groups = n_groups;
    p.itype = to_mm(itype);
    p.dt_softplus = dt_softplus;
    p.state = state.data_ptr();
    p.state_type = to_mm(state.scalar_type());
    p.x = x.data_ptr();
    p.dt = dt.data_ptr();
    p.A = A.data_ptr<float>();
    p.B = B.data_ptr();
    p.C = C.data_ptr();
    p.D = Dc.defined() ? Dc.data_ptr() : nullptr;
    p.D_type = Dc.defined() ? to_mm(Dc.scalar_type()) : MM_FLOAT32;
    p.z = z_.has_value() ? z_.value().data_ptr() : nullptr;
    p.dt_bias = bc.defined() ? bc.data_ptr() : nullptr;
    p.dt_bias_type = bc.defined() ? to_mm(bc.scalar_type()) : MM_FLOAT32;
    p.out = out.data_ptr();
    p.state_batch_stride = state.stride(0);
    p.state_d_stride = state.stride(1);
    p.state_dstate_stride = state.stride(2);
    p.x_batch_stride = x.stride(0);
    p.x_d_stride = x.stride(1);
    p.dt_batch_stride = dt.stride(0);
    p.dt_d_stride = dt.stride(1);
    if (z_.has_value()) {
        p.z_batch_stride = z_.value().stride(0);
        p.z_d_stride = z_.value().stride(1);
    }
    p.out_batch_stride = out.stride(0);
    p.out_d_stride = out.stride(1);
    p.A_d_stride = A.stride(0);
    p.A_dstate_stride = A.stride(1);
    if (B.dim() == 3) {
        p.B_batch_stride = B.stride(0);
        p.B_group_stride = B.stride(1);
        p.B_dstate_stride = B.stride(2);
        p.C_batch_stride = C.stride(0);
        p.C_group_stride = C.stride(1);
        p.C_dstate_stride = C.stride(2);
    } else {
        p.B_batch_stride = B.stride(0);
        p.B_dstate_stride = B.stride(1);
        p.C_batch_stride = C.stride(0);
        p.C_dstate_stride = C.stride(1);
    }
    const c10::DeviceGuard device_guard{state.device()};
    check_rc(mm_state_update(&p, c10::hip::getCurrentHIPStream().stream()), "mm_state_update");
    return out;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.def("fwd", &fwd, "Selective scan forward (reference-compatible outputs [out, x, out_z?])",
          pybind11::arg("u"), pybind11::arg("delta"), pybind11::arg("A"), pybind11::arg("B"), pybind11::arg("C"),
          pybind11::arg("D") = pybind11::none(), pybind11::arg("z") = pybind11::none(),
          pybind11::arg("delta_bias") = pybind11::none(), pybind11::arg("P") = pybind11::none(),
          pybind11::arg("Q") = pybind11::none(), pybind11::arg("gamma") = pybind11::none(),
          pybind11::arg("delta_softplus") = false, pybind11::arg("tile_states") = false);
    m.def("bwd", &bwd, "Selective scan backward (reference-compatible outputs)",
          pybind11::arg("u"), pybind11::arg("delta"), pybind11::arg("A"), pybind11::arg("B"), pybind11::arg("C"),
          pybind11::arg("D") = pybind11::none(), pybind11::arg("z") = pybind11::none(),
          pybind11::arg("delta_bias") = pybind11::none(), pybind11::arg("P") = pybind11::none(),
          pybind11::arg("Q") = pybind11::none(), pybind11::arg("gamma") = pybind11::none(), pybind11::arg("dout"),
          pybind11::arg("x"), pybind11::arg("out"), pybind11::arg("dz"), pybind11::arg("dP_out") = pybind11::none(),
          pybind11::arg("dQ_out") = pybind11::none(), pybind11::arg("delta_softplus"),
          pybind11::arg("recompute_out_z"), pybind11::arg("tile_states") = pybind11::none());
    m.def("fwd_infer", &fwd_infer, "Selective scan forward, inference outputs [out_z|out, last_state?]",
          pybind11::arg("u"), pybind11::arg("delta"), pybind11::arg("A"), pybind11::arg("B"), pybind11::arg("C"),
          pybind11::arg("D") = pybind11::none(), pybind11::arg("z") = pybind11::none(),
          pybind11::arg("delta_bias") = pybind11::none(), pybind11::arg("delta_softplus") = false,
          pybind11::arg("return_last_state") = false, pybind11::arg("P") = pybind11::none(),
          pybind11::arg("Q") = pybind11::none(), pybind11::arg("gamma") = pybind11::none());
    m.def("state_update", &state_update, "Single-token selective state update (in place on state)",
          pybind11::arg("state"), pybind11::arg("x"), pybind11::arg("dt"), pybind11::arg("A"), pybind11::arg("B"),
          pybind11::arg("C"), pybind11::arg("D") = pybind11::none(), pybind11::arg("z") = pybind11::none(),
          pybind11::arg("dt_bias") = pybind11::none(), pybind11::arg("dt_softplus") = false);
    m.def("conv1d_fwd", &conv1d_fwd, "Causal depthwise conv1d forward",
          pybind11::arg("x"), pybind11::arg("weight"), pybind11::arg("bias") = pybind11::none(),
          pybind11::arg("initial_states") = pybind11::none(), pybind11::arg("final_states_out") = pybind11::none(),
          pybind11::arg("silu") = false, pybind11::arg("out") = pybind11::none());
    m.def("conv1d_bwd", &conv1d_bwd, "Causal depthwise conv1d backward [dx, dweight, dbias?]",
          pybind11::arg("x"), pybind11::arg("weight"), pybind11::arg("bias"), pybind11::arg("dout"),
          pybind11::arg("dx") = pybind11::none(), pybind11::arg("silu") = false);
    m.def("conv1d_update", &conv1d_update, "Causal depthwise conv1d decode update (in place on conv_state)",
          pybind11::arg("x"), pybind11::arg("conv_state"), pybind11::arg("weight"),
          pybind11::arg("bias") = pybind11::none(), pybind11::arg("silu") = false);
    m.def("rms_norm_fwd", &rms_norm_fwd, "Row RMSNorm over dim 1 of a 3-D tensor",
          pybind11::arg("x"), pybind11::arg("weight"), pybind11::arg("eps") = 1e-6,
          pybind11::arg("out") = pybind11::none());
    m.def("abi_version", []() { return mm_abi_version(); });
}
