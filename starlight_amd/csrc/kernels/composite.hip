// Composite operators built from the primitive launchers:
//  * SwiGlu (reference/swiglu.rs:40-84): gate and up projections, silu(g)*u,
//    then the down projection. The reference avoids an [rows, inter]
//    temporary by accumulating rank-1 updates; on the GPU the intermediates
//    go to the device workspace (row chunks when they do not fit), which
//    turns the three products into plain streaming GEMV/GEMMs: for a few
//    rows the gate/up GEMV's epilogue forms h = silu(g)*u; for many rows
//    gate and up are one q-GEMM launch and the down projection's activation
//    split forms silu(g)*u as it reads them.
//  * RmsNormMatMul (reference/fused.rs:41-90): the normalised rows go to the
//    workspace, then one matmul.
#include "common.h"
#include "kernels.h"

namespace slhip {

hipError_t launch_linear(const float* a, const WeightRef& w, float* out, uint64_t rows, uint64_t n,
                         uint64_t k, const Workspace& ws, hipStream_t s) {
    if (w.quantized()) return launch_qmatmul(a, w.quant, out, rows, ws, s);
    return launch_matmul(a, w.dense, out, 1, 1, 1, rows, k, n, true, s);
}

// Rows per chunk of launch_swiglu with a workspace of ws_floats: its g and
// u intermediates take half of the workspace, the projections' own scratch
// the other half.
uint64_t swiglu_chunk_rows(uint64_t ws_floats, uint64_t inter) {
    const uint64_t budget = ws_floats / 2;
    return budget > 64 && inter != 0 ? (budget - 64) / (2 * inter) : 0;
}

hipError_t launch_swiglu(const float* x, const WeightRef& gate, const WeightRef& up, const WeightRef& down,
                         float* out, uint64_t rows, uint64_t hidden, uint64_t inter, const Workspace& ws,
                         hipStream_t s, const float* resid, float* out2, bool out_dead, const float* gamma,
                         float eps) {
    if (rows == 0) return hipSuccess;
    const uint64_t budget = ws.floats / 2;
    uint64_t chunk = swiglu_chunk_rows(ws.floats, inter);
    if (chunk == 0) return hipErrorOutOfMemory;
    if (chunk > rows) chunk = rows;
    const uint64_t u_off = (chunk * inter + 63) / 64 * 64;
    float* g = ws.data;
    float* u = ws.data + u_off;
    const Workspace rest = ws.after(budget);
    const QuantWeight* gate_up[2] = {&gate.quant, &up.quant};
    if (gamma != nullptr) {
        // the norm exists only inside the gate/up split: every chunk (the
        // full ones and the last) must take the q-GEMM route
        const uint64_t tail = rows % chunk;
        const auto takes = [&](uint64_t rc) {
            return rc > 16 && qgemm_mfma_takes(x, gate_up, 2, rc, rest);
        };
        if (!gate.quantized() || !up.quantized() || !qgemm_norm_takes(hidden, gamma) || !takes(chunk) ||
            (tail != 0 && !takes(tail)))
            return hipErrorNotSupported;
    }
    if (rows <= 16 && gate.quantized() && up.quantized() && gamma == nullptr) {
        // gate and up tiles in one launch with the silu * up epilogue
        QgemvFused f{};
        f.a = x;
        f.w[0] = &gate.quant;
        f.w[1] = &up.quant;
        f.out[0] = g;
        f.nseg = 2;
        f.m = rows;
        f.epilogue = kFusedPair;
        hipError_t e = launch_qgemv_fused(f, s);
        if (e == hipSuccess) {
            e = launch_linear(g, down, out, rows, hidden, inter, rest, s);
            if (e == hipSuccess && out2 != nullptr) e = launch_add(resid, out, out2, rows * hidden, s);
            return e;
        }
        if (e != hipErrorNotSupported) return e;
    }
    float* gu_out[2] = {g, u};
    for (uint64_t r0 = 0; r0 < rows; r0 += chunk) {
        const uint64_t rc = rows - r0 < chunk ? rows - r0 : chunk;
        const float* xr = x + r0 * hidden;
        hipError_t e;
        if (gate.quantized() && up.quantized() && rc > 16 && qgemm_mfma_takes(xr, gate_up, 2, rc, rest)) {
            // many rows: gate and up in one launch over one activation split
            e = launch_qgemm_multi(xr, gate_up, gu_out, 2, rc, rest, s, nullptr, nullptr, nullptr, gamma, eps);
        } else {
            // (never with gamma: the check above covers every chunk)
            if (gamma != nullptr) return hipErrorInvalidValue;
            e = launch_linear(xr, gate, g, rc, inter, hidden, rest, s);
            if (e == hipSuccess) e = launch_linear(xr, up, u, rc, inter, hidden, rest, s);
        }
        if (e != hipSuccess) return e;
        float* const out_r = out + r0 * hidden;
        const float* const resid_r = resid != nullptr ? resid + r0 * hidden : nullptr;
        float* const out2_r = out2 != nullptr ? out2 + r0 * hidden : nullptr;
        const QuantWeight* dw[1] = {&down.quant};
        if (down.quantized() && rc > 16 && qgemm_mfma_takes(g, dw, 1, rc, rest)) {
            // many rows: silu(g) * u formed by the down projection's
            // activation split (no h pass), the residual in its epilogue
            float* outs[1] = {out_dead && out2_r != nullptr ? nullptr : out_r};
            float* out2s[1] = {out2_r};
            e = launch_qgemm_multi(g, dw, outs, 1, rc, rest, s, u, &resid_r, out2s);
        } else {
            e = launch_silu_mul(g, u, g, rc * inter, s);
            if (e == hipSuccess) e = launch_linear(g, down, out_r, rc, hidden, inter, rest, s);
            if (e == hipSuccess && out2_r != nullptr) e = launch_add(resid_r, out_r, out2_r, rc * hidden, s);
        }
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_rms_norm_matmul(const float* x, const float* weight, const WeightRef& w, float* out,
                                  uint64_t rows, uint64_t hidden, uint64_t out_features, float eps,
                                  const Workspace& ws, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    const uint64_t budget = ws.floats / 2;
    uint64_t chunk = budget / hidden;
    if (chunk == 0) return hipErrorOutOfMemory;
    if (chunk > rows) chunk = rows;
    float* y = ws.data;
    if (rows <= 16 && w.quantized()) {
        // the normalisation runs as the GEMV's prologue
        QgemvFused f{};
        f.a = x;
        f.gamma = weight;
        f.eps = eps;
        f.w[0] = &w.quant;
        f.out[0] = out;
        f.nseg = 1;
        f.m = rows;
        f.epilogue = kFusedPlain;
        hipError_t e = launch_qgemv_fused(f, s);
        if (e != hipErrorNotSupported) return e;
    }
    const QuantWeight* wq[1] = {&w.quant};
    for (uint64_t r0 = 0; r0 < rows; r0 += chunk) {
        const uint64_t rc = rows - r0 < chunk ? rows - r0 : chunk;
        const float* xr = x + r0 * hidden;
        float* outs[1] = {out + r0 * out_features};
        hipError_t e;
        if (w.quantized() && rc > 16 && qgemm_norm_takes(hidden, weight) &&
            qgemm_mfma_takes(xr, wq, 1, rc, ws.after(budget))) {
            // many rows: the norm inside the q-GEMM's activation split
            e = launch_qgemm_multi(xr, wq, outs, 1, rc, ws.after(budget), s, nullptr, nullptr, nullptr, weight, eps);
        } else {
            e = launch_rms_norm(xr, weight, y, rc, hidden, eps, s);
            if (e == hipSuccess) e = launch_linear(y, w, outs[0], rc, out_features, hidden, ws.after(budget), s);
        }
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace slhip
