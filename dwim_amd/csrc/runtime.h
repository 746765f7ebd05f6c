// Internal structures of the HIP backend and the kernel launchers the C ABI
// calls.  Everything here is gfx950 (CDNA4): 64-lane wavefronts, 160 KB of LDS
// per CU, 256 CUs in 8 XCDs.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>

#include "dwim_hip.h"
#include "planes.h"

struct dwim_dev {
    int index = 0;
    hipStream_t stream = nullptr;
    std::string name;
    int cus = 256;
    // Device scratch the library owns: attention split-K partials, argmax
    // results.  Grown on demand, freed with the device.
    float *partials = nullptr;
    size_t partials_cap = 0;  // floats
    // the address on this device of k_attention.hip's file-scope scratch
    // array (dwim_attention_noalloc), taken when the device is opened
    float *attn_scratch = nullptr;
    uint32_t *argmax_buf = nullptr;
    size_t argmax_cap = 0;
    uint32_t *tokens = nullptr;  // token ids for the embedding lookup
    size_t tokens_cap = 0;
    void *planes = nullptr;  // one token's int8 activation planes (planes_scratch_bytes())
    size_t prepared = 0;     // width of the planes dwim_prepare wrote (0: none, or replaced)
    void *split = nullptr;   // the f16 hi/lo parts of a batch's activations (k_gemm_q4k)
    size_t split_cap = 0;    // bytes
    size_t split_n = 0, split_cols = 0;  // the batch the split holds
    float *work = nullptr;   // normalized activations / a product's second result
    size_t work_cap = 0;     // floats
    float *gemm_parts = nullptr;  // a k-split batch product's partial results (k_gemm_q4k)
    size_t gemm_parts_cap = 0;    // floats
    void *kvx = nullptr;          // a batch attention's expanded key/value cache (k_attention.hip)
    size_t kvx_cap = 0;           // bytes
    float *dn_work = nullptr;     // a batch delta rule's per-chunk matrices (k_delta_net.hip)
    size_t dn_work_cap = 0;       // floats
    // Split one-token Q4_K products (k_mv_q4k_mfma.hip): the partial sums of
    // up to mv_tiles_cap 16-row tiles (4 parts × 32 floats each) and a counter
    // per tile, zero between launches.
    float *mv_partials = nullptr;
    unsigned *mv_counters = nullptr;
    unsigned mv_tiles_cap = 0;
    // several-token products (k_mv_q4k_stream.hip): partial sums of the
    // tiles that workgroups share, [tile][part][slot][token][32]
    float *mv_stream = nullptr;
    size_t mv_stream_cap = 0;  // floats
    // The open handle and every live buffer, weight and cache hold a
    // reference: the device (its stream) outlives whatever was made on it,
    // whichever order a binding frees them in.
    int refs = 1;
};

void dwim_dev_release(dwim_dev *dev);
// frees everything a device holds, whatever its reference count
void dwim_dev_release_resources(dwim_dev *dev);

struct dwim_buf {
    dwim_dev *dev;
    float *data;
    size_t len, cap;
};

// Device layouts of a weight matrix (`upload` re-lays the host formats):
//   BF16  q: u16 [rows][cols]
//   Q4_0  q: u8 [rows][cols/2] (the reference's nibble order), s: u16 [rows][cols/32]
//   Q8_0  q: i8 [rows][cols],                                    s: u16 [rows][cols/32]
//   Q4_K  q: 64-row tiles of blocks as layout.h describes (rows padded to 64)
//   Q6_K  q: ql u8 [rows][nb][128], s: qh u8 [rows][nb][64], s2: i8 scales [rows][nb][16],
//         s3: f16 d [rows][nb]
// with nb = cols/256 blocks per row.  Splitting each K-quant block into
// streams keeps every lane's 16-byte load aligned and each stream contiguous.
struct dwim_weight {
    dwim_dev *dev;
    int fmt;
    size_t rows, cols;
    void *q = nullptr, *s = nullptr, *s2 = nullptr, *s3 = nullptr;
};

// A key or value cache of `len` activations: the reference's Q8 (q: int8
// values, s: an f16 scale per block of 32), or with f16 set, f16 values (q
// holds their 2·len bytes, s is null).
struct dwim_cache {
    dwim_dev *dev;
    int8_t *q;
    uint16_t *s;
    size_t len;
    bool f16 = false;
};

// ---- errors ----
int dwim_fail(const std::string &msg);
#define DWIM_HIP(call)                                                                        \
    do {                                                                                      \
        hipError_t e_ = (call);                                                               \
        if (e_ != hipSuccess) return dwim_fail(std::string(#call) + ": " + hipGetErrorString(e_)); \
    } while (0)
#define DWIM_CHECK(cond, msg)                      \
    do {                                           \
        if (!(cond)) return dwim_fail(msg);        \
    } while (0)

// ---- launchers (each returns hipGetLastError() of its launch) ----
hipError_t launch_fill_zero(hipStream_t s, float *x, size_t n);
hipError_t launch_add(hipStream_t s, float *x, const float *y, size_t n);
hipError_t launch_silu_mul(hipStream_t s, float *g, const float *u, size_t n);
hipError_t launch_sigmoid_mul(hipStream_t s, float *x, const float *g, size_t n);
hipError_t launch_rmsnorm(hipStream_t s, float *out, const float *x, const float *w, size_t rows,
                          size_t dim, float eps);
hipError_t launch_l2norm(hipStream_t s, float *x, size_t rows, size_t dim, float eps);
hipError_t launch_rope(hipStream_t s, float *x, const float *table, size_t n, size_t pos,
                       size_t n_heads, size_t head_dim, size_t rot_dim);
hipError_t launch_store(hipStream_t s, int8_t *cq, uint16_t *cs, const float *src, size_t blocks);
hipError_t launch_store_f16(hipStream_t s, uint16_t *c, const float *src, size_t n);
hipError_t launch_matvec(dwim_dev *dev, const dwim_weight *w, float *out, const float *x, size_t n,
                         int add);
hipError_t launch_matvec_q4k(dwim_dev *dev, const dwim_weight *w, float *out, const float *x, size_t n,
                             int add);
// Up to four Q4_K matrices of one row length over the same x in one launch,
// x first RMS-normalized by `norm` (when given; the normalized rows are also
// written to xn_out when that is given).
hipError_t launch_matvec_q4k_multi(dwim_dev *dev, const dwim_weight *const *ws, float *const *outs, int count,
                                   const float *x, size_t n, const float *norm, float eps, float *xn_out);
// out = silu(gate·x) · (up·x) for Q4_K gate and up, x optionally RMS-normalized
hipError_t launch_swiglu_q4k(dwim_dev *dev, const dwim_weight *gate, const dwim_weight *up, float *out,
                             const float *x, size_t n, const float *norm, float eps);
// One token on the int8 matrix cores (planes.h): launch_planes writes x's
// planes (RMS-normalized by `norm` when given, the normalized x also to
// xn_out when given) into plane area `area` (0 or 1) of the device;
// launch_mv_q4k_mfma then runs up to four matrices over that area
// (outs[j] += or = W_j·x by adds[j]), or gate and up as a SwiGLU pair
// (swiglu = 1, count = 2, the result in outs[0]).
// handover = 1 with a norm: the planes of x·norm and each group's Σx²
// (planes.h), for a product launched with MvExtra::rms.
size_t planes_scratch_bytes();
planes::View planes_area(dwim_dev *dev, int area, size_t cols);
hipError_t launch_planes(dwim_dev *dev, const float *x, size_t cols, const float *norm, float eps, float *xn_out,
                         int area, int handover = 0);
// Optional parts of a one-token product: rms, the input planes are x·w with
// Σx² per group and every result is scaled by 1/sqrt(Σx²/cols + eps);
// emit_area >= 0 (one matrix or a SwiGLU pair, rows whole 256-blocks), the
// planes of outs[0] (after the add or the SwiGLU) go to that area, of
// outs[0]·emit_norm with Σ outs[0]² per group when emit_norm is given (and
// outs[0]·emit_norm in f32 to emit_xw when that is given).
struct MvExtra {
    int rms = 0;
    float eps = 0.0f;
    int emit_area = -1;
    const float *emit_norm = nullptr;
    float *emit_xw = nullptr;
    // the input planes hold heads of head_dim columns unnormalized, each
    // scaled here by 1/sqrt(Σ head_ss[head][0..3] / head_dim + head_eps)
    const float *head_ss = nullptr;
    size_t head_dim = 0;
    float head_eps = 0.0f;
    // given: the same launch also computes bf16_out = bf16 · bf16_x (a small
    // bf16 matrix against f32 x, in workgroups of its own)
    const dwim_weight *bf16 = nullptr;
    const float *bf16_x = nullptr;
    float *bf16_out = nullptr;
};
hipError_t launch_mv_q4k_mfma(dwim_dev *dev, const dwim_weight *const *ws, float *const *outs, const int *adds,
                              int count, int swiglu, int area, const MvExtra *extra = nullptr);
// n tokens (rows of x, [n][cols]) on the int8 matrix cores, in launches of
// up to four tokens that share the weight loads: the planes of each token
// (RMS-normalized by `norm` when given, the normalized rows to xn_out when
// that is given) in the batch areas, then outs[j] ([n][rows_j]) += or = W_j·x
// by adds[j], or a SwiGLU pair into outs[0] as launch_mv_q4k_mfma.
// Plane areas: 0 and 1 for one token's products (each reads one and writes
// the other); kBatchArea + t for token t of a 2..4-token launch, and a
// second such set at kBatchArea2, so that a batch product that reads one set
// hands its results' planes on in the other.
constexpr int kBatchArea = 2;
constexpr int kBatchArea2 = kBatchArea + 4;
// Optional parts of a 2..4-token product (one launch), as MvExtra's for one
// token: in_area >= 0, the tokens' planes are already in areas in_area + t
// (written by the product before, per 16 or per 32 activations) and nothing
// is made from x; rms, those planes are x·w with Σx² per group, every
// token's results scaled by 1/sqrt(Σx²/cols + eps); emit_area >= 0 (one
// matrix or a SwiGLU pair, rows
// whole 256-blocks), token t's planes of outs[0] (after the add or the
// SwiGLU) go to area emit_area + t, of outs[0]·emit_norm with Σ outs[0]² per
// group when emit_norm is given (and outs[0]·emit_norm in f32 to emit_xw,
// [nt][rows], when that is given).
struct StreamExtra {
    int in_area = -1;
    int rms = 0;
    float eps = 0.0f;
    // given: the planes hold heads of 128 columns unnormalized (a DeltaNet
    // output gate), each scaled here by 1/sqrt(Σ head_ss[t][head][0..7] /
    // 128 + head_eps)
    const float *head_ss = nullptr;
    float head_eps = 0.0f;
    // given: the same launch also writes bf16_out ([nt][rows]) = bf16 ·
    // bf16_x ([nt][cols], f32), each token's results RMS-scaled with the
    // products' (a small bf16 matrix)
    const dwim_weight *bf16 = nullptr;
    const float *bf16_x = nullptr;
    float *bf16_out = nullptr;
    int emit_area = -1;
    const float *emit_norm = nullptr;
    float *emit_xw = nullptr;
};
// 2..4 tokens whose planes (per 16 or per 32 activations) are at xq[t],
// xstat[t]: outs[j] ([nt][rows_j]) += or = W_j·x, or a SwiGLU pair into
// outs[0], every weight read once (k_mv_q4k_stream.hip); se's rms and emit
// parts apply (its in_area is the caller's)
hipError_t run_mv_stream(dwim_dev *dev, const dwim_weight *const *ws, float *const *outs, const int *adds, int count,
                         int swiglu, size_t nt, const int8_t *const *xq, const float *const *xstat,
                         const StreamExtra *se = nullptr);
// (gate_z given: the input is the DeltaNet output gate silu(gate_z)·
// rmsnorm(x)·norm over heads of 128, made with the planes; xn_out unused)
// (se given: n <= 4, one launch with se's parts)
hipError_t launch_mv_q4k_mfma_tokens(dwim_dev *dev, const dwim_weight *const *ws, float *const *outs, const int *adds,
                                     int count, int swiglu, const float *x, size_t n, const float *norm, float eps,
                                     float *xn_out, const float *gate_z = nullptr, const StreamExtra *se = nullptr);
// The planes of nt <= 4 rows of x ([nt][cols]) in the batch areas, one launch;
// views[t] is token t's (pair: per-32 scales)
hipError_t launch_planes_batch(dwim_dev *dev, const float *x, size_t cols, size_t nt, int pair, planes::View *views);
// A Q6_K weight times one token's planes in plane area `area` (the output
// head; k_mv_q6k_mfma.hip).
hipError_t launch_mv_q6k_mfma(dwim_dev *dev, const dwim_weight *w, float *out, int area);
// A Q6_K weight times n tokens (rows of x), out [n][rows], in launches of up
// to four tokens that read the weights once (a verify batch through the head)
hipError_t launch_mv_q6k_tokens(dwim_dev *dev, const dwim_weight *w, float *out, const float *x, size_t n);
hipError_t launch_swiglu(dwim_dev *dev, const dwim_weight *gate, const dwim_weight *up, float *out,
                         float *scratch, const float *x, size_t n);
hipError_t launch_attention(dwim_dev *dev, float *out, const float *q, const dwim_cache *k,
                            const dwim_cache *v, size_t n, size_t pos, size_t n_heads,
                            size_t head_dim, size_t n_kv_heads);
hipError_t launch_conv(hipStream_t s, float *q, float *k, float *v, float *state_out,
                       const float *x, const float *state, const float *w, size_t n, size_t q_dim,
                       size_t k_dim, size_t v_dim);
// An RMS scale 1/sqrt(Σ ss / cols + eps) over `groups` partial sums of
// squares (planes.h), for an operation whose input arrived as x·w unscaled.
struct Rms {
    const float *ss = nullptr;
    unsigned groups = 0;
    float cols = 1.0f;
    float eps = 0.0f;
};
// with rms, the gate logits (alpha, beta) are scaled by it first; with
// unit_keys (keys of unit length), 64 tokens and more take the chunked form;
// with state_in (fewer tokens only), the state is read from there and the
// updated one written to `state`
// A batch of up to 16 tokens through a DeltaNet mixer's conv, l2 norms and
// delta rule in one launch (k_delta_net.hip): qkv raw [n][2·nk·D + nv·D],
// the conv state carried from conv_state to conv_state_out, the gate logits
// [n][2·nv] final (no RMS scale), the state read from state_in (null: state)
// and written to state, o to out [n][nv·D] (null: not written).
// Where k_gdn_tokens also writes the recurrent state and the conv state
// after each token t < min(n - 1, kMaxSteps) (null: not kept), so that a
// rewind keeping t + 1 tokens of a verified batch takes them as they are.
constexpr int kMaxSteps = 8;
struct GdnSteps {
    float *state[kMaxSteps];
    float *conv[kMaxSteps];
};
// And given (n <= 4): the mixer's output gate silu(z)·o·norm_w of each
// token (z [n][nv·D]), unnormalized, as token t's planes in the plane area
// at planes + t·kAreaBytes, and each 16 columns' Σo² to head_ss
// [n][nv][D / 16]: the consuming product applies each head's RMS norm.
struct GdnGate {
    const float *z = nullptr;
    const float *norm_w = nullptr;
    int8_t *planes = nullptr;
    float *head_ss = nullptr;
};
hipError_t launch_gdn_tokens(dwim_dev *dev, float *out, const float *qkv, const float *conv_state,
                             float *conv_state_out, const float *conv_w, const float *gates, const float *decay,
                             float *state, const float *state_in, size_t n, size_t n_k_heads, size_t n_v_heads,
                             size_t head_dim, float eps, const GdnSteps *steps = nullptr,
                             const GdnGate *gate = nullptr);
hipError_t launch_delta_net(dwim_dev *dev, float *out, const float *q, const float *k,
                            const float *v, const float *gates, const float *decay, float *state,
                            size_t n, size_t n_k_heads, size_t n_v_heads, size_t head_dim, const Rms *rms = nullptr,
                            bool unit_keys = false, const float *state_in = nullptr);
hipError_t launch_embed(hipStream_t s, float *out, const dwim_weight *w, const uint32_t *tokens,
                        size_t n);
// first index of each row's maximum, into the first `rows` words of scratch
// (argmax_scratch_words(rows) words)
size_t argmax_scratch_words(size_t rows);
hipError_t launch_argmax(hipStream_t s, const float *logits, size_t rows, size_t cols, uint32_t *scratch);
hipError_t launch_synthetic_q4_k(hipStream_t s, uint8_t *tiled, size_t rows, size_t cols,
                                 uint64_t seed, float c);
hipError_t launch_synthetic_q6_k(hipStream_t s, uint8_t *ql, uint8_t *qh, int8_t *sc,
                                 uint16_t *d, size_t rows, size_t cols, uint64_t seed, float c);
hipError_t launch_synthetic_bf16(hipStream_t s, uint16_t *q, size_t rows, size_t cols,
                                 uint64_t seed, float c);

// ---- fused launches of the model host (k_fused.hip, k_attention.hip) ----
hipError_t launch_conv_l2(hipStream_t s, float *q, float *k, float *v, float *state_out, const float *x,
                          const float *state, const float *w, size_t n, size_t qd, size_t kd, size_t vd, size_t dim,
                          float eps);
// z = silu(z) · rmsnorm(att, w) per dim-row of the n·total values; area >= 0
// (one token): the result's planes into that plane area too
hipError_t launch_gated_norm(dwim_dev *dev, float *z, const float *att, const float *w, size_t n, size_t total,
                             size_t dim, float eps, int area);
hipError_t launch_qk_prep(hipStream_t s, float *q, float *k, const float *v, const float *q_norm,
                          const float *k_norm, const float *table, size_t n, size_t pos, size_t heads,
                          size_t kv_heads, size_t head_dim, size_t rot, float eps, dwim_cache *kc, dwim_cache *vc);
// attention, then out *= sigmoid(gate) when gate is given, and (one token,
// area >= 0) out's planes into that plane area
// Grows a device scratch buffer (cap in elements of `elem` bytes) to `need`,
// after whatever is queued; a model reserves each buffer's largest size when
// it is built, so that no forward pass allocates.
hipError_t dev_grow(dwim_dev *dev, void **ptr, size_t *cap, size_t need, size_t elem);
size_t delta_net_work_floats(size_t n, size_t n_v_heads);
hipError_t delta_net_reserve(dwim_dev *dev, size_t n, size_t n_v_heads);
size_t gemm_split_bytes(size_t n, size_t cols);
size_t argmax_scratch_words(size_t rows);
size_t gemm_parts_floats(size_t n, size_t rows, size_t cols);
hipError_t gemm_reserve(dwim_dev *dev, size_t split_bytes, size_t parts_floats);
size_t attention_partials_floats(size_t n, size_t pos, size_t n_heads, size_t head_dim);
hipError_t attention_reserve(dwim_dev *dev, size_t floats);
size_t attention_kvx_bytes(size_t len, size_t n_kv_heads);
hipError_t attention_kvx_reserve(dwim_dev *dev, size_t bytes);
hipError_t attention_scratch_init(dwim_dev *dev);
hipError_t launch_attention_gated(dwim_dev *dev, float *out, const float *q, const dwim_cache *k,
                                  const dwim_cache *v, size_t n, size_t pos, size_t n_heads, size_t head_dim,
                                  size_t n_kv_heads, const float *gate, int area);

// One token through a gated-DeltaNet mixer (k_gdn.hip): conv + SiLU of qkv
// with its state carried to conv_state_out, l2 norms and the delta rule on
// `state`, over 4 workgroups a head, from gate logits ab = W_ab ·
// x·attn_norm computed beforehand (not yet RMS-scaled), the RMS norm of o
// left to the product that reads the planes (area): each quarter's Σo² to
// head_ss ([nv][4] floats), its columns' silu(z)·o·norm_w unnormalized as
// planes.
hipError_t launch_gdn_split(dwim_dev *dev, const float *qkv, const float *conv_state, float *conv_state_out,
                            const float *conv_w, const float *ab, const Rms &rms, const float *decay, float *state,
                            const float *z, const float *norm_w, float eps, size_t nk, size_t nv, size_t head_dim,
                            float *head_ss, int area);

// ---- batches of tokens (k_gemm_q4k.hip) ----
// out (+)= w · x for n tokens on the f16 matrix cores (x's hi/lo parts are
// written to the device's split scratch first)
hipError_t launch_gemm_q4k(dwim_dev *dev, const dwim_weight *w, float *out, const float *x, size_t n, int add);
// The same in two steps, so that products of one x share its split:
// gemm_prepare writes x's parts ([n][cols]) to the device's split scratch,
// gemm_run multiplies a weight of that many columns by them, out by the mode.
enum GemmMode { kGemmStore = 0, kGemmAdd = 1, kGemmSiluGate = 2 /* out = silu(out)·(w·x) */ };
hipError_t gemm_prepare(dwim_dev *dev, const float *x, size_t n, size_t cols);
// gemm_prepare of rmsnorm(x)·norm (the values launch_rmsnorm gives, in one
// pass over x), the normalized rows also to xn_out when given
hipError_t gemm_prepare_rms(dwim_dev *dev, const float *x, const float *norm, float eps, size_t n, size_t cols,
                            float *xn_out);
// gemm_prepare of silu(z)·rmsnorm(att)·norm per head of dim (the values
// launch_gated_norm gives; z is not written)
hipError_t gemm_prepare_gated(dwim_dev *dev, const float *z, const float *att, const float *norm, float eps, size_t n,
                              size_t total, size_t dim);
hipError_t gemm_run(dwim_dev *dev, const dwim_weight *w, float *out, size_t n, int mode);
// out (+)= w · x for a bf16 matrix of up to 96 rows over the prepared split
// (the DeltaNet gate projection of a batch), on the f16 matrix cores
hipError_t gemm_run_bf16(dwim_dev *dev, const dwim_weight *w, float *out, size_t n, int add);
// gate and up over the prepared split in one launch, g and u written plain;
// then the split of silu(g)·u prepared for the down product
hipError_t gemm_run_swiglu_pair(dwim_dev *dev, const dwim_weight *gate, const dwim_weight *up, float *g, float *u,
                                size_t n);
// the FFN of a batch (n >= 16 tokens, Q4_K): x += down · (silu(gate·xn) · (up·xn)),
// xn = rmsnorm(x)·norm; g and u hold n·rows floats each
hipError_t launch_ffn_q4k(dwim_dev *dev, const dwim_weight *gate, const dwim_weight *up, const dwim_weight *down,
                          float *x, size_t n, const float *norm, float eps, float *g, float *u);
// the device's work scratch, grown to at least `floats`
float *dev_work(dwim_dev *dev, size_t floats);
