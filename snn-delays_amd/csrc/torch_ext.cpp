// Host-side autograd Function for the axonal layer's common regime, in C++.
//
// The module path of the axonal layer (reference delay_layers_triton.py:21-79 ->
// AxonalRecdelTriton, recdel_base.py:349-439) spends most of its host time in Python:
// argument structs, a dozen tensor allocations and the Python backward on the autograd
// thread. This Function does the same calls to the C ABI (include/delrec.h) from C++ for
// the regime the straight-line kernels serve: soft triangle taps of a uniform half-width,
// decay charge, hard reset to 0, no learned spread, no STE / rounded taps, N <= 256.
//
// The forward does not read the window length: delrec_axonal_fwd runs with L = 0 and writes
// max d into a slot of pinned host memory from inside the scan (no copy, no event); the
// backward takes that slot by its ticket. A slot reused by later forwards before
// this backward runs, or a value that does not arrive, makes the backward read max d again
// (synchronously).
#include <torch/extension.h>

#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime.h>

#include <cmath>
#include <mutex>
#include <unordered_map>
#include <stdexcept>
#include <string>

#include "delrec.h"

namespace {

using torch::autograd::AutogradContext;
using torch::autograd::variable_list;
using at::Tensor;

void check(int status, const char* fn) {
    if (status != DELREC_OK)
        throw std::runtime_error(std::string(fn) + " failed: status " + std::to_string(status) + " (" +
                                 delrec_strerror(status) + ")");
}

// the largest delay each backward took, by the delay tensor's storage: the Python layer reads
// it (seen_dmax) to decide whether the next forward may run before reading the window length
std::mutex g_seen_mu;
std::unordered_map<const void*, float> g_seen;

void note_seen(const void* d, float v) {
    std::lock_guard<std::mutex> lk(g_seen_mu);
    g_seen[d] = v;
}

void forget_dmax(const Tensor& d) {
    std::lock_guard<std::mutex> lk(g_seen_mu);
    g_seen.erase(d.data_ptr());
}

double seen_dmax(const Tensor& d) {
    std::lock_guard<std::mutex> lk(g_seen_mu);
    const auto it = g_seen.find(d.data_ptr());
    return it == g_seen.end() ? std::nan("") : (double)it->second;
}

// max d posted by the forward (its ticket for delrec_max_take), or a fresh synchronous read of
// `fallback` when the slot was reused or the value did not arrive
float take_max(int64_t ticket, const Tensor& fallback) {
    float v = 0.0f;
    if (delrec_max_take((uint32_t)ticket, &v, 10000) != DELREC_OK) v = fallback.max().item<float>();
    note_seen(fallback.data_ptr(), v);
    return v;
}

// L = ceil(1 + max d + max s) + 1 with each sum rounded to fp32 (reference delays.py:26)
int window_length(float d_max, float s_max) {
    const float v = (1.0f + d_max) + s_max;
    return (int)std::ceil((double)v) + 1;
}

void* ptr(const Tensor& t) { return t.defined() ? t.data_ptr() : nullptr; }

size_t workspace_bytes(int kind, int T, int B, int N, int L, int flags) {
    size_t n = 0;
    check(delrec_query_workspace(kind, T, B, N, L, flags, &n), "delrec_query_workspace");
    return n;
}

delrec_lif make_lif(double tau, double vth, int64_t surrogate, double gamma, double alpha, bool detach) {
    delrec_lif k{};
    k.tau = (float)tau;
    k.decay = (float)(1.0 - 1.0 / tau);
    k.v_threshold = (float)vth;
    k.v_reset = 0.0f;
    k.soft_reset = 0;
    k.decay_input = 0;
    k.detach_reset = detach ? 1 : 0;
    k.surrogate = (int32_t)surrogate;
    k.gamma = (float)gamma;
    k.alpha = (float)alpha;
    return k;
}

struct AxonalCommon : public torch::autograd::Function<AxonalCommon> {
    static Tensor forward(AutogradContext* ctx, Tensor x, Tensor W, Tensor d, c10::optional<Tensor> bias,
                          c10::optional<Tensor> drop, double sigma, double tau, double vth, int64_t surrogate,
                          double gamma, double alpha, bool detach) {
        TORCH_CHECK(x.is_cuda() && x.dim() == 3, "axonal_common: x must be a (T, B, N) GPU tensor");
        const int T = (int)x.size(0), B = (int)x.size(1), N = (int)x.size(2);
        TORCH_CHECK(N <= 256, "axonal_common: N <= 256");
        const auto f32 = x.options().dtype(at::kFloat);
        Tensor xc = x.to(at::kFloat).contiguous();
        const bool w_bf16 = W.scalar_type() == at::kBFloat16;
        Tensor Wc = w_bf16 ? W.contiguous() : W.to(at::kFloat).contiguous();
        Tensor dc = d.to(at::kFloat).contiguous();
        Tensor bc = bias && bias->defined() ? bias->to(at::kFloat).contiguous() : Tensor();
        Tensor mc = drop && drop->defined() ? drop->to(at::kFloat).contiguous() : Tensor();
        Tensor y = at::empty({T, B, N}, f32), u = at::empty({T, B, N}, f32), z = at::empty({T, B, N}, f32);
        Tensor bits = at::empty({B, (T + 31) / 32, N}, x.options().dtype(at::kInt));
        hipStream_t stream = c10::hip::getCurrentHIPStream(x.get_device()).stream();


        delrec_axonal_fwd_args a{};
        a.T = T; a.B = B; a.N = N; a.L = 0;
        a.x = (const float*)xc.data_ptr(); a.W = Wc.data_ptr(); a.w_bf16 = w_bf16 ? 1 : 0;
        a.bias = (const float*)ptr(bc); a.d = (const float*)dc.data_ptr(); a.s = nullptr;
        a.s_uniform = (float)(1.0 + sigma); a.drop = (const float*)ptr(mc); a.taps = DELREC_TAPS_SOFT;
        a.lif = make_lif(tau, vth, surrogate, gamma, alpha, detach);
        a.y = (float*)y.data_ptr(); a.u = (float*)u.data_ptr(); a.rec = nullptr; a.z = (float*)z.data_ptr();
        a.bits = (uint32_t*)bits.data_ptr();
        a.workspace = nullptr; a.workspace_bytes = 0;
        uint32_t ticket = 0;
        a.dmax_ticket = &ticket;
        check(delrec_axonal_fwd(&a, stream), "delrec_axonal_fwd");

        ctx->save_for_backward({u, z, bits, Wc, dc, bc, mc});
        ctx->saved_data["T"] = (int64_t)T;
        ctx->saved_data["B"] = (int64_t)B;
        ctx->saved_data["N"] = (int64_t)N;
        ctx->saved_data["ticket"] = (int64_t)ticket;
        ctx->saved_data["sigma"] = sigma;
        ctx->saved_data["tau"] = tau;
        ctx->saved_data["vth"] = vth;
        ctx->saved_data["surrogate"] = surrogate;
        ctx->saved_data["gamma"] = gamma;
        ctx->saved_data["alpha"] = alpha;
        ctx->saved_data["detach"] = detach;
        ctx->saved_data["w_dtype"] = (int64_t)W.scalar_type();
        return y;
    }

    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        auto saved = ctx->get_saved_variables();
        Tensor u = saved[0], z = saved[1], bits = saved[2], Wc = saved[3], dc = saved[4], bc = saved[5],
               mc = saved[6];
        const int T = (int)ctx->saved_data["T"].toInt(), B = (int)ctx->saved_data["B"].toInt(),
                  N = (int)ctx->saved_data["N"].toInt();
        const double sigma = ctx->saved_data["sigma"].toDouble();
        const float d_max = take_max(ctx->saved_data["ticket"].toInt(), dc);
        // NaN: a NaN delay, or a window the forward could not hold (it wrote NaN outputs)
        if (!(d_max == d_max))
            throw std::runtime_error("axonal_common backward: the delay window exceeds the 256 lags the "
                                     "forward holds without a window length, or a delay is NaN");
        const int L = std::max(window_length(d_max, (float)(1.0 + sigma)), 2);
        const bool w_bf16 = Wc.scalar_type() == at::kBFloat16;
        const auto f32 = u.options();
        Tensor gy = grads[0].to(at::kFloat).contiguous();
        Tensor dx = at::empty({T, B, N}, f32);
        const bool need_W = ctx->needs_input_grad(1), need_d = ctx->needs_input_grad(2),
                   need_b = bc.defined() && ctx->needs_input_grad(3);
        Tensor dW = need_W ? at::empty({N, N}, f32) : Tensor();
        Tensor dd = need_d ? at::empty({N}, f32) : Tensor();
        Tensor db = need_b ? at::empty({N}, f32) : Tensor();
        const size_t wsb = workspace_bytes(DELREC_WS_AXONAL_BWD, T, B, N, L, w_bf16 ? 1 : 0);
        Tensor ws = at::empty({(int64_t)std::max<size_t>(wsb, 1)}, u.options().dtype(at::kByte));
        hipStream_t stream = c10::hip::getCurrentHIPStream(u.get_device()).stream();

        delrec_axonal_bwd_args a{};
        a.T = T; a.B = B; a.N = N; a.L = L;
        a.gy = (const float*)gy.data_ptr(); a.u = (const float*)u.data_ptr();
        a.bits = (const uint32_t*)bits.data_ptr(); a.z = (const float*)z.data_ptr();
        a.W = Wc.data_ptr(); a.w_bf16 = w_bf16 ? 1 : 0; a.d = (const float*)dc.data_ptr(); a.s = nullptr;
        a.s_uniform = (float)(1.0 + sigma); a.drop = (const float*)ptr(mc); a.mode = DELREC_BWD_SOFT;
        a.lag = nullptr;
        a.lif = make_lif(ctx->saved_data["tau"].toDouble(), ctx->saved_data["vth"].toDouble(),
                         ctx->saved_data["surrogate"].toInt(), ctx->saved_data["gamma"].toDouble(),
                         ctx->saved_data["alpha"].toDouble(), ctx->saved_data["detach"].toBool());
        a.dx = (float*)dx.data_ptr(); a.dW = (float*)ptr(dW); a.db = (float*)ptr(db); a.dd = (float*)ptr(dd);
        a.ds = nullptr;
        a.workspace = ws.data_ptr(); a.workspace_bytes = ws.numel();
        check(delrec_axonal_bwd(&a, stream), "delrec_axonal_bwd");

        const auto w_dtype = (at::ScalarType)ctx->saved_data["w_dtype"].toInt();
        if (dW.defined() && w_dtype != at::kFloat) dW = dW.to(w_dtype);
        // x, W, d, bias, drop, then the 7 scalars
        return {dx, dW, dd, db, Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor()};
    }
};

Tensor axonal_common(Tensor x, Tensor W, Tensor d, c10::optional<Tensor> bias, c10::optional<Tensor> drop,
                     double sigma, double tau, double vth, int64_t surrogate, double gamma, double alpha,
                     bool detach) {
    return AxonalCommon::apply(x, W, d, bias, drop, sigma, tau, vth, surrogate, gamma, alpha, detach);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "C++ autograd Function of the axonal delayed-LIF layer (common regime)";
    m.def("axonal_common", &axonal_common, "axonal layer forward (autograd)", py::arg("x"), py::arg("W"),
          py::arg("d"), py::arg("bias"), py::arg("drop"), py::arg("sigma"), py::arg("tau"), py::arg("vth"),
          py::arg("surrogate"), py::arg("gamma"), py::arg("alpha"), py::arg("detach"));
    m.def("seen_dmax", &seen_dmax, "largest delay the last backward on this delay tensor took (NaN: none)",
          py::arg("d"));
    m.def("forget_dmax", &forget_dmax, "drop the recorded largest delay of this delay storage", py::arg("d"));
}
