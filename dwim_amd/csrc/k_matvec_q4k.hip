// Q4_K products of a batch of n tokens, routed by size (dwim gpu/cpu.rs:110-149
// is the product, gpu/mod.rs:259 the add, gpu/mod.rs:274-285 the SwiGLU):
// fewer than kGemmTokens tokens go to the int8 matrix-core matrix-vector
// kernels (k_mv_q4k_mfma.hip: one token, or up to four at a time reading the
// weights once), larger batches to the f16 matrix-core GEMM (k_gemm_q4k.hip).
#include "runtime.h"

// Batches of at least kGemmTokens go through the f16 matrix-core GEMM.
constexpr size_t kGemmTokens = 16;

hipError_t launch_matvec_q4k(dwim_dev *dev, const dwim_weight *w, float *out, const float *x, size_t n, int add) {
    if (n >= kGemmTokens) return launch_gemm_q4k(dev, w, out, x, n, add);
    return launch_mv_q4k_mfma_tokens(dev, &w, &out, &add, 1, 0, x, n, nullptr, 0.0f, nullptr);
}

hipError_t launch_matvec_q4k_multi(dwim_dev *dev, const dwim_weight *const *ws, float *const *outs, int count,
                                   const float *x, size_t n, const float *norm, float eps, float *xn_out) {
    if (count < 1 || count > 4) return hipErrorInvalidValue;
    for (int j = 0; j < count; j++)
        if (ws[j]->cols != ws[0]->cols || ws[j]->fmt != DWIM_Q4_K) return hipErrorInvalidValue;
    if (n < kGemmTokens) return launch_mv_q4k_mfma_tokens(dev, ws, outs, nullptr, count, 0, x, n, norm, eps, xn_out);
    {
        hipError_t e = norm ? gemm_prepare_rms(dev, x, norm, eps, n, ws[0]->cols, xn_out)
                            : gemm_prepare(dev, x, n, ws[0]->cols);
        for (int j = 0; j < count && e == hipSuccess; j++) e = gemm_run(dev, ws[j], outs[j], n, kGemmStore);
        return e;
    }
}

hipError_t launch_swiglu_q4k(dwim_dev *dev, const dwim_weight *gate, const dwim_weight *up, float *out, const float *x,
                             size_t n, const float *norm, float eps) {
    if (gate->rows != up->rows || gate->cols != up->cols) return hipErrorInvalidValue;
    if (n < kGemmTokens) {
        const dwim_weight *ws[2] = {gate, up};
        float *outs[2] = {out, nullptr};
        return launch_mv_q4k_mfma_tokens(dev, ws, outs, nullptr, 2, 1, x, n, norm, eps, nullptr);
    }
    {
        // x normalized, split once; gate·x into out, then out = silu(out)·(up·x)
        const size_t cols = gate->cols;
        hipError_t e = norm ? gemm_prepare_rms(dev, x, norm, eps, n, cols, nullptr) : gemm_prepare(dev, x, n, cols);
        if (e == hipSuccess) e = gemm_run(dev, gate, out, n, kGemmStore);
        if (e == hipSuccess) e = gemm_run(dev, up, out, n, kGemmSiluGate);
        return e;
    }
}

hipError_t launch_ffn_q4k(dwim_dev *dev, const dwim_weight *gate, const dwim_weight *up, const dwim_weight *down,
                          float *x, size_t n, const float *norm, float eps, float *g, float *u) {
    if (n < kGemmTokens || gate->fmt != DWIM_Q4_K || down->fmt != DWIM_Q4_K || down->cols != gate->rows)
        return hipErrorInvalidValue;
    hipError_t e = gemm_prepare_rms(dev, x, norm, eps, n, gate->cols, nullptr);
    if (e == hipSuccess) e = gemm_run_swiglu_pair(dev, gate, up, g, u, n);
    if (e == hipSuccess) e = gemm_run(dev, down, x, n, kGemmAdd);
    return e;
}
