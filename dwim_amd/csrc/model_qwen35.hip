// The qwen35 hybrid model (dwim inference/qwen35/mod.rs) as a host program
// over the C ABI of include/dwim_hip.h: the same buffers, the same operations
// in the same order as `Model::forward_batch` / `Pass::layer` /
// `Pass::drafter`, so that what the reference's token loop asks of its
// `Device` is exactly what runs here.  It is the stand-in for the reference's
// Rust caller (no Rust toolchain here) and the driver of the model benchmark.
//
// Weights are random (dwim_model_synthetic): every tensor is drawn from its own
// stream, seeded from the model seed and the tensor's GGUF-style name, and the
// matrices are generated and quantized on the device.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <array>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "quant_math.h"
#include "runtime.h"

namespace {

#define TRY(call)                   \
    do {                            \
        if ((call) != 0) return 1;  \
    } while (0)

constexpr size_t kConvKernel = 4;
constexpr size_t kMaxDrafts = 8;  // MAX_DRAFTS (qwen35/mod.rs:26)

// FNV-1a of a tensor's name, the key of its value stream
uint64_t fnv1a(const std::string &s) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (unsigned char c : s) {
        h ^= c;
        h *= 0x100000001b3ull;
    }
    return h;
}

struct Layer {
    bool attention = false;
    dwim_buf *attn_norm = nullptr, *mlp_norm = nullptr;
    dwim_weight *gate = nullptr, *up = nullptr, *down = nullptr;
    // full attention
    dwim_weight *q = nullptr, *qgate = nullptr, *k = nullptr, *v = nullptr, *o = nullptr;
    dwim_buf *q_norm = nullptr, *k_norm = nullptr;
    size_t cache = 0;
    // linear attention
    dwim_weight *qkv = nullptr, *z = nullptr, *ab = nullptr, *out = nullptr;
    dwim_buf *conv = nullptr, *decay = nullptr, *norm = nullptr;
    size_t slot = 0;
};

struct Draft {
    dwim_buf *embed_norm = nullptr, *hidden_norm = nullptr, *norm = nullptr;
    dwim_weight *embed_proj = nullptr, *hidden_proj = nullptr;
    Layer layer;
};

// Sequence (qwen35/mod.rs:1351-1374): a sequence's own state
struct Sequence {
    size_t id = 0;
    std::vector<dwim_cache *> k_cache, v_cache;
    std::vector<std::array<dwim_buf *, 2>> conv_state;
    bool parity = false;
    std::vector<dwim_buf *> ssm_state;
    size_t max_len = 0;
    dwim_buf *hidden = nullptr;
    bool carry = false;
    // a batch being verified: its tokens and the position of the first
    std::vector<uint32_t> verified;
    size_t verified_at = 0;
};

}  // namespace

struct dwim_model {
    dwim_dev *dev = nullptr;
    dwim_qwen35_config c{};
    uint64_t seed = 0;
    std::vector<Layer> layers;
    dwim_buf *norm = nullptr;
    dwim_weight *head = nullptr, *embd = nullptr;
    bool has_draft = false;
    bool fuse = true;  // fused decode launches where the formats allow
    Draft draft;
    // State (qwen35/mod.rs:1298-1344): per-token buffers for `most` tokens
    size_t most = 0;
    std::array<size_t, 11> widths{};
    dwim_buf *x = nullptr, *xb = nullptr, *xh = nullptr, *q = nullptr, *gate = nullptr, *k = nullptr,
             *v = nullptr, *att = nullptr, *qkv = nullptr, *z = nullptr, *ab = nullptr;
    dwim_buf *up = nullptr, *gate_ffn = nullptr, *logits = nullptr, *rope = nullptr, *drafted = nullptr;
    // the one-token DeltaNet step's Σo² per head quarter ([v_heads][4])
    dwim_buf *head_ss = nullptr;
    // a 2..4-token batch's DeltaNet output gate's Σo² per 16 columns
    // ([4][v_heads][8])
    dwim_buf *batch_hss = nullptr;
    // device-fed greedy decoding: the picks, and where the step running
    // reads its token and writes its pick (null outside decode_greedy)
    uint32_t *picks = nullptr;
    size_t picks_cap = 0;
    const uint32_t *embed_from = nullptr;
    uint32_t *argmax_to = nullptr;
    Sequence seq;
    std::map<size_t, Sequence> parked;  // the sequences not running
    // verifying: the linear layers' states run through the batch, and their
    // inputs, apart from the real ones (with a drafter only)
    std::vector<dwim_buf *> ssm_scratch, qkv_saved, ab_saved;
    // verifying in one launch a layer: the states after each of the batch's
    // first tokens (step t: after token t), which a rewind takes as they are
    std::vector<dwim_buf *> ssm_step[kMaxSteps], conv_step[kMaxSteps];
    // the mark: linear layers' states and the carried hidden state
    std::vector<dwim_buf *> mark_conv, mark_ssm;
    dwim_buf *mark_hidden = nullptr;
    bool mark_carry = false;
    long marked = -1;  // the id of the sequence marked, or -1
    size_t caches = 0, slots = 0;
    // everything allocated, freed with the model
    std::vector<dwim_buf *> bufs;
    std::vector<dwim_weight *> weights;
    std::vector<dwim_cache *> cache_list;

    size_t q_dim() const { return c.heads * c.head_dim; }
    size_t kv_dim() const { return c.kv_heads * c.head_dim; }
    size_t k_dim() const { return c.k_heads * c.state_dim; }
    size_t v_dim() const { return c.v_heads * c.state_dim; }
    size_t conv_width() const { return (kConvKernel - 1) * (2 * k_dim() + v_dim()); }
    size_t ssm_width() const { return c.v_heads * c.state_dim * c.state_dim; }
    bool is_attention(size_t layer) const { return (layer + 1) % c.full_attention_interval == 0; }

    // ---- allocation
    int buf(size_t len, dwim_buf **out) {
        TRY(dwim_alloc(dev, len, out));
        bufs.push_back(*out);
        return 0;
    }
    int vec(const std::string &name, size_t len, float sigma, float offset, dwim_buf **out) {
        std::vector<float> v(len);
        const uint64_t s = dq::splitmix(seed, fnv1a(name));
        dwim_synthetic_values(s, 0, len, sigma, v.data());
        for (auto &e : v) e = e + offset;
        TRY(buf(len, out));
        return dwim_write(dev, *out, v.data(), len);
    }
    // values u ∈ [0, 1) from the tensor's stream: (hash >> 40) / 2^24
    int uniform_vec(const std::string &name, size_t len, float scale, float offset, dwim_buf **out) {
#pragma clang fp contract(off)
        std::vector<float> v(len);
        const uint64_t s = dq::splitmix(seed, fnv1a(name));
        for (size_t i = 0; i < len; i++) {
            const float u = (float)(dq::splitmix(s, i) >> 40) * (1.0f / 16777216.0f);
            v[i] = u * scale + offset;
        }
        TRY(buf(len, out));
        return dwim_write(dev, *out, v.data(), len);
    }
    int mat(const std::string &name, int fmt, size_t rows, size_t cols, float sigma, dwim_weight **out) {
        TRY(dwim_upload_synthetic(dev, fmt, rows, cols, dq::splitmix(seed, fnv1a(name)), sigma, out));
        weights.push_back(*out);
        return 0;
    }

    int load_layer(size_t i, bool attention, int fmt, Layer &l) {
        const std::string p = "blk." + std::to_string(i) + ".";
        const size_t H = c.hidden;
        const float s = 0.02f;
        l.attention = attention;
        TRY(vec(p + "attn_norm", H, 0.1f, 1.0f, &l.attn_norm));
        if (attention) {
            TRY(mat(p + "attn_q", fmt, q_dim(), H, s, &l.q));
            TRY(mat(p + "attn_q_gate", fmt, q_dim(), H, s, &l.qgate));
            TRY(mat(p + "attn_k", fmt, kv_dim(), H, s, &l.k));
            TRY(mat(p + "attn_v", fmt, kv_dim(), H, s, &l.v));
            TRY(mat(p + "attn_output", fmt, H, q_dim(), s, &l.o));
            TRY(vec(p + "attn_q_norm", c.head_dim, 0.1f, 1.0f, &l.q_norm));
            TRY(vec(p + "attn_k_norm", c.head_dim, 0.1f, 1.0f, &l.k_norm));
            l.cache = caches++;
        } else {
            TRY(mat(p + "attn_qkv", fmt, 2 * k_dim() + v_dim(), H, s, &l.qkv));
            TRY(mat(p + "attn_gate", fmt, v_dim(), H, s, &l.z));
            TRY(mat(p + "ssm_ab", DWIM_BF16, 2 * c.v_heads, H, s, &l.ab));
            TRY(vec(p + "ssm_conv1d", (2 * k_dim() + v_dim()) * kConvKernel, 0.3f, 0.0f, &l.conv));
            // decay: a ∈ [-1, -0.1) for every value head, then dt_bias ∈ [-4, 4)
            dwim_buf *a = nullptr, *dt = nullptr;
            TRY(uniform_vec(p + "ssm_a", c.v_heads, -0.9f, -0.1f, &a));
            TRY(uniform_vec(p + "ssm_dt.bias", c.v_heads, 8.0f, -4.0f, &dt));
            TRY(buf(2 * c.v_heads, &l.decay));
            TRY(dwim_copy(dev, l.decay, 0, a, 0, c.v_heads));
            TRY(dwim_copy(dev, l.decay, c.v_heads, dt, 0, c.v_heads));
            TRY(vec(p + "ssm_norm", c.state_dim, 0.1f, 1.0f, &l.norm));
            TRY(mat(p + "ssm_out", fmt, H, v_dim(), s, &l.out));
            l.slot = slots++;
        }
        TRY(vec(p + "post_attention_norm", H, 0.1f, 1.0f, &l.mlp_norm));
        TRY(mat(p + "ffn_gate", fmt, c.intermediate, H, s, &l.gate));
        TRY(mat(p + "ffn_up", fmt, c.intermediate, H, s, &l.up));
        TRY(mat(p + "ffn_down", fmt, H, c.intermediate, s, &l.down));
        return 0;
    }

    int zeroed(size_t len, dwim_buf **out) { return buf(len, out); }  // dwim_alloc zeroes

    int new_sequence(Sequence &s, size_t id, size_t max_len) {
        s.id = id;
        s.max_len = max_len;
        for (size_t i = 0; i < caches; i++) {
            dwim_cache *kc, *vc;
            TRY(dwim_alloc_cache(dev, max_len * kv_dim(), &kc));
            cache_list.push_back(kc);
            TRY(dwim_alloc_cache(dev, max_len * kv_dim(), &vc));
            cache_list.push_back(vc);
            s.k_cache.push_back(kc);
            s.v_cache.push_back(vc);
        }
        for (size_t i = 0; i < slots; i++) {
            std::array<dwim_buf *, 2> pair{};
            TRY(zeroed(conv_width(), &pair[0]));
            TRY(zeroed(conv_width(), &pair[1]));
            s.conv_state.push_back(pair);
            dwim_buf *st;
            TRY(zeroed(ssm_width(), &st));
            s.ssm_state.push_back(st);
        }
        TRY(buf((most + 1) * c.hidden, &s.hidden));
        return 0;
    }

    // State::batch (qwen35/mod.rs:1476-1497)
    int batch(size_t n) {
        if (n > most) return dwim_fail("a batch of " + std::to_string(n) + " tokens is more than " + std::to_string(most));
        dwim_buf *b[11] = {x, xb, xh, q, gate, k, v, att, qkv, z, ab};
        for (int i = 0; i < 11; i++) TRY(dwim_resize(dev, b[i], n * widths[i]));
        TRY(dwim_resize(dev, up, n * c.intermediate));
        TRY(dwim_resize(dev, gate_ffn, n * c.intermediate));
        return 0;
    }

    int normalize(dwim_buf *out, dwim_buf *in, dwim_buf *weight, size_t rows) {
        return dwim_normalize(dev, out, in, weight, rows * c.hidden, c.eps);
    }

    // The fused path: Q4_K matrices with rows of whole 256-blocks, heads the
    // fused kernels take.  One token goes through the int8 matrix cores, the
    // activations of each product handed over as planes (plane area 0);
    // several tokens through the f32 matrix kernels.
    // a verified batch of n whose linear layers all ran in one launch each,
    // keeping the states after its first tokens
    bool steps_kept(size_t n) const {
        if (!has_draft || n < 2 || n - 1 > (size_t)kMaxSteps || n > 16 || c.state_dim != 128) return false;
        for (const Layer &l : layers)
            if (!l.attention && !fusable(l)) return false;
        return true;
    }

    bool fusable(const Layer &l) const {
        const bool shapes = c.hidden % 256 == 0 && c.hidden <= 10240 && c.intermediate % 256 == 0 &&
                            c.intermediate <= 80 * 256 && (c.state_dim == 128 || c.state_dim == 256) &&
                            c.head_dim % 64 == 0 && c.head_dim <= 256 && q_dim() % 256 == 0 && v_dim() % 256 == 0;
        const bool formats = (l.attention ? (l.q->fmt == DWIM_Q4_K && l.qgate->fmt == DWIM_Q4_K && l.k->fmt == DWIM_Q4_K &&
                                             l.v->fmt == DWIM_Q4_K && l.o->fmt == DWIM_Q4_K)
                                          : (l.qkv->fmt == DWIM_Q4_K && l.z->fmt == DWIM_Q4_K && l.out->fmt == DWIM_Q4_K)) &&
                             l.gate->fmt == DWIM_Q4_K && l.up->fmt == DWIM_Q4_K && l.down->fmt == DWIM_Q4_K;
        return fuse && shapes && formats;
    }
    int projections(const dwim_weight *const *ws, dwim_buf *const *outs, int count, const dwim_buf *norm_w,
                    size_t n, dwim_buf *xn_out) {
        float *o[4];
        for (int i = 0; i < count; i++) o[i] = outs[i]->data;
        DWIM_HIP(launch_matvec_q4k_multi(dev, ws, o, count, x->data, n, norm_w->data, c.eps,
                                         xn_out ? xn_out->data : nullptr));
        return 0;
    }
    // One token through the int8 matrix cores, the activations of each
    // product handed over as planes: a layer's input arrives in area 0 as the
    // planes of x·attn_norm with Σx² per group (written by the previous
    // layer's last product when `handed`, else by launch_planes here); the
    // mixer's output goes to area 1; the residual product x += o·att writes
    // the planes of x·mlp_norm into area 0; the SwiGLU pair writes its
    // result's planes into area 1; and the down product's x += down·h hands
    // the next layer its input in area 0.  The RMS norms become scales the
    // consuming products apply to their results.
    bool handed = false;
    Rms rms0() const {
        const planes::View in = planes_area(dev, 0, c.hidden);
        return Rms{in.ss, (unsigned)(c.hidden / planes::kGroup), (float)c.hidden, c.eps};
    }
    // x += w · (area `area`), handing the planes of x·norm (and x·norm in f32
    // to xw when given) on to area `to`
    // (head_ss given: the planes in `area` are DeltaNet heads whose RMS norm
    // is applied here, from their Σo² per quarter)
    int add_handover(const dwim_weight *w, int area, int to, const dwim_buf *norm, dwim_buf *xw,
                     const dwim_buf *head_ss = nullptr) {
        float *o = x->data;
        const int add = 1;
        MvExtra e;
        e.emit_area = to;
        e.emit_norm = norm ? norm->data : nullptr;
        e.emit_xw = xw ? xw->data : nullptr;
        if (head_ss) {
            e.head_ss = head_ss->data;
            e.head_dim = c.state_dim;
            e.head_eps = c.eps;
        }
        DWIM_HIP(launch_mv_q4k_mfma(dev, &w, &o, &add, 1, 0, area, norm || head_ss ? &e : nullptr));
        return 0;
    }
    // products of the layer input (area 0, RMS-scaled)
    // (bf16 given: the same launch also writes bf16_out = bf16 · xh, the
    // DeltaNet gate logits from x·attn_norm, not yet RMS-scaled)
    int from_input(const dwim_weight *const *ws, dwim_buf *const *outs, int count, const dwim_weight *bf16 = nullptr,
                   dwim_buf *bf16_out = nullptr) {
        float *o[4];
        for (int i = 0; i < count; i++) o[i] = outs[i]->data;
        MvExtra e;
        e.rms = 1;
        e.eps = c.eps;
        if (bf16) {
            e.bf16 = bf16;
            e.bf16_x = xh->data;
            e.bf16_out = bf16_out->data;
        }
        DWIM_HIP(launch_mv_q4k_mfma(dev, ws, o, nullptr, count, 0, 0, &e));
        return 0;
    }

    // 2..4 tokens through a fused layer hand every product's planes to the
    // next as one token does, in the two sets of batch areas: the layer input
    // (planes of x·attn_norm with Σx² per group) arrives in the second set
    // when the previous layer's down product wrote it (batch_in), else is
    // made in the first; the mixer's output is made in the first set; the
    // residual product x += o·att hands x·mlp_norm on in the second; the
    // SwiGLU pair its result in the first; the down product the next
    // layer's input in the second (and, before a DeltaNet layer, x·attn_norm
    // in f32 to xh for its gate rows, which scale by the batch's row scales).
    int batch_in = -1;
    bool batch_hand(const Layer &l, size_t n) const {
        return n >= 2 && n <= 4 && fusable(l) && c.state_dim == 128 &&
               (l.attention || (l.ab->fmt == DWIM_BF16 && l.ab->rows <= 96));
    }
    // products of the layer input (handed over in `in_set`, or made here from
    // x with the norm, the normalized rows to xn_out when given)
    // (bf16 given: the same launch writes bf16_out = bf16 · xh, RMS-scaled
    // like the products, the DeltaNet gate rows)
    int batch_input(const dwim_weight *const *ws, dwim_buf *const *outs, int count, const dwim_buf *norm_w, size_t n,
                    int in_set, dwim_buf *xn_out, const dwim_weight *bf16 = nullptr, dwim_buf *bf16_out = nullptr) {
        float *o[4];
        for (int i = 0; i < count; i++) o[i] = outs[i]->data;
        StreamExtra se;
        se.in_area = in_set;
        se.rms = in_set >= 0;
        se.eps = c.eps;
        if (bf16) {
            se.bf16 = bf16;
            se.bf16_x = xh->data;
            se.bf16_out = bf16_out->data;
        }
        DWIM_HIP(launch_mv_q4k_mfma_tokens(dev, ws, o, nullptr, count, 0, in_set >= 0 ? nullptr : x->data, n,
                                           norm_w->data, c.eps, xn_out ? xn_out->data : nullptr, nullptr, &se));
        return 0;
    }
    // x += w · in, handing x·mlp_norm on in the second set: in's planes made
    // here (of in, or the DeltaNet output gate with gate_z), or (in null)
    // already in the first set, written by the attention merge or (with
    // head_ss) by the DeltaNet step, heads unnormalized
    int batch_residual(const dwim_weight *w, const dwim_buf *in, size_t n, const dwim_buf *norm_w,
                       const dwim_buf *gate_z, const dwim_buf *emit_norm, const dwim_buf *hss = nullptr) {
        float *o = x->data;
        const int add = 1;
        StreamExtra se;
        se.in_area = in ? -1 : kBatchArea;
        se.head_ss = hss ? hss->data : nullptr;
        se.head_eps = c.eps;
        se.emit_area = kBatchArea2;
        se.emit_norm = emit_norm->data;
        DWIM_HIP(launch_mv_q4k_mfma_tokens(dev, &w, &o, &add, 1, 0, in ? in->data : nullptr, n,
                                           norm_w ? norm_w->data : nullptr, c.eps, nullptr,
                                           gate_z ? gate_z->data : nullptr, &se));
        return 0;
    }
    // the SwiGLU pair and the down product over handed-over planes
    int batch_ffn(const Layer &l, size_t n, const Layer *next) {
        {
            const dwim_weight *ws[2] = {l.gate, l.up};
            float *o[2] = {up->data, nullptr};
            StreamExtra se;
            se.in_area = kBatchArea2;
            se.rms = 1;
            se.eps = c.eps;
            se.emit_area = kBatchArea;
            DWIM_HIP(launch_mv_q4k_mfma_tokens(dev, ws, o, nullptr, 2, 1, nullptr, n, nullptr, c.eps, nullptr, nullptr,
                                               &se));
        }
        float *o = x->data;
        const int add = 1;
        StreamExtra se;
        se.in_area = kBatchArea;
        if (next && batch_hand(*next, n)) {
            se.emit_area = kBatchArea2;
            se.emit_norm = next->attn_norm->data;
            se.emit_xw = next->attention ? nullptr : xh->data;
        }
        DWIM_HIP(launch_mv_q4k_mfma_tokens(dev, &l.down, &o, &add, 1, 0, nullptr, n, nullptr, c.eps, nullptr, nullptr,
                                           &se));
        batch_in = se.emit_area;
        return 0;
    }

    // The one-token layer on the handover path (Pass::layer, qwen35/mod.rs:
    // 541-655, in the same order); `next` is the following layer's input
    // norm, to hand its input over, or null.
    int layer_one(const Layer &l, size_t pos, const dwim_buf *next) {
        const float eps = c.eps;
        TRY(dwim_resize(dev, xh, c.hidden));
        // the DeltaNet gate projection takes x·attn_norm in f32 (xh)
        if (!handed) {
            DWIM_HIP(launch_planes(dev, x->data, c.hidden, l.attn_norm->data, eps, l.attention ? nullptr : xh->data, 0, 1));
        }
        handed = false;
        if (l.attention) {
            TRY(dwim_resize(dev, q, q_dim()));
            TRY(dwim_resize(dev, gate, q_dim()));
            TRY(dwim_resize(dev, k, kv_dim()));
            TRY(dwim_resize(dev, v, kv_dim()));
            TRY(dwim_resize(dev, att, q_dim()));
            dwim_cache *kc = seq.k_cache[l.cache], *vc = seq.v_cache[l.cache];
            const dwim_weight *ws[4] = {l.q, l.qgate, l.k, l.v};
            dwim_buf *outs[4] = {q, gate, k, v};
            TRY(from_input(ws, outs, 4));
            DWIM_HIP(launch_qk_prep(dev->stream, q->data, k->data, v->data, l.q_norm->data, l.k_norm->data,
                                    rope->data, 1, pos, c.heads, c.kv_heads, c.head_dim, c.rot_dim, eps, kc, vc));
            DWIM_HIP(launch_attention_gated(dev, att->data, q->data, kc, vc, 1, pos, c.heads, c.head_dim, c.kv_heads,
                                            gate->data, 1));
            TRY(add_handover(l.o, 1, 0, l.mlp_norm, nullptr));
        } else {
            TRY(dwim_resize(dev, q, k_dim()));
            TRY(dwim_resize(dev, k, k_dim()));
            TRY(dwim_resize(dev, v, v_dim()));
            TRY(dwim_resize(dev, att, v_dim()));
            auto &pair = seq.conv_state[l.slot];
            dwim_buf *state = seq.parity ? pair[0] : pair[1];
            dwim_buf *state_out = seq.parity ? pair[1] : pair[0];
            const dwim_weight *ws[2] = {l.qkv, l.z};
            dwim_buf *outs[2] = {qkv, z};
            TRY(dwim_resize(dev, ab, 2 * c.v_heads));
            TRY(from_input(ws, outs, 2, l.ab, ab));
            // conv, delta rule and gated output in one launch of 4
            // workgroups a head, the gate logits (ab) RMS-scaled there; the
            // head's RMS norm of o is applied by the output product (its Σo²
            // in head_ss)
            DWIM_HIP(launch_gdn_split(dev, qkv->data, state->data, state_out->data, l.conv->data, ab->data, rms0(),
                                      l.decay->data, seq.ssm_state[l.slot]->data, z->data, l.norm->data, eps,
                                      c.k_heads, c.v_heads, c.state_dim, head_ss->data, 1));
            TRY(add_handover(l.out, 1, 0, l.mlp_norm, nullptr, head_ss));
        }
        // the FFN: gate/up pair from area 0 (RMS-scaled), its planes to area 1
        const dwim_weight *ws[2] = {l.gate, l.up};
        float *outs[2] = {up->data, nullptr};
        MvExtra e;
        e.rms = 1;
        e.eps = eps;
        e.emit_area = 1;
        DWIM_HIP(launch_mv_q4k_mfma(dev, ws, outs, nullptr, 2, 1, 0, &e));
        TRY(add_handover(l.down, 1, 0, next, next ? xh : nullptr));
        handed = next != nullptr;
        return 0;
    }

    // Pass::layer (qwen35/mod.rs:541-655).  Verifying, the linear layers
    // save their inputs and run a copy of their recurrent state (:606-632).
    int layer(const Layer &l, size_t n, size_t pos, bool verify = false, const Layer *next = nullptr) {
        const float eps = c.eps;
        const bool fused = fusable(l), one = fused && n == 1;
        if (one && !verify) return layer_one(l, pos, next ? next->attn_norm : nullptr);
        handed = false;
        const bool bh = batch_hand(l, n);
        const int in_set = bh ? batch_in : -1;
        batch_in = -1;
        TRY(dwim_resize(dev, xh, n * c.hidden));
        if (!fused) TRY(normalize(xh, x, l.attn_norm, n));
        if (l.attention) {
            TRY(dwim_resize(dev, q, n * q_dim()));
            TRY(dwim_resize(dev, gate, n * q_dim()));
            TRY(dwim_resize(dev, k, n * kv_dim()));
            TRY(dwim_resize(dev, v, n * kv_dim()));
            TRY(dwim_resize(dev, att, n * q_dim()));
            dwim_cache *kc = seq.k_cache[l.cache], *vc = seq.v_cache[l.cache];
            if (fused) {
                const dwim_weight *ws[4] = {l.q, l.qgate, l.k, l.v};
                dwim_buf *outs[4] = {q, gate, k, v};
                if (bh)
                    TRY(batch_input(ws, outs, 4, l.attn_norm, n, in_set, nullptr));
                else
                    TRY(projections(ws, outs, 4, l.attn_norm, n, nullptr));
                DWIM_HIP(launch_qk_prep(dev->stream, q->data, k->data, v->data, l.q_norm->data, l.k_norm->data,
                                        rope->data, n, pos, c.heads, c.kv_heads, c.head_dim, c.rot_dim, eps, kc, vc));
                DWIM_HIP(launch_attention_gated(dev, att->data, q->data, kc, vc, n, pos, c.heads, c.head_dim,
                                                c.kv_heads, gate->data, bh ? kBatchArea : -1));
                if (bh)
                    TRY(batch_residual(l.o, nullptr, n, nullptr, nullptr, l.mlp_norm));
                else
                    TRY(dwim_matmul_add(dev, x, l.o, att, xb));
            } else {
                TRY(dwim_matmul(dev, q, l.q, xh));
                TRY(dwim_matmul(dev, gate, l.qgate, xh));
                TRY(dwim_matmul(dev, k, l.k, xh));
                TRY(dwim_matmul(dev, v, l.v, xh));
                TRY(dwim_rmsnorm(dev, q, l.q_norm, eps));
                TRY(dwim_rmsnorm(dev, k, l.k_norm, eps));
                TRY(dwim_rope(dev, q, rope, pos, c.heads, c.head_dim, c.rot_dim));
                TRY(dwim_rope(dev, k, rope, pos, c.kv_heads, c.head_dim, c.rot_dim));
                TRY(dwim_store(dev, kc, pos * kv_dim(), k));
                TRY(dwim_store(dev, vc, pos * kv_dim(), v));
                TRY(dwim_attention(dev, att, q, kc, vc, pos, c.heads, c.head_dim, c.kv_heads));
                TRY(dwim_sigmoid_mul(dev, att, gate));
                TRY(dwim_matmul_add(dev, x, l.o, att, xb));
            }
        } else {
            TRY(dwim_resize(dev, q, n * k_dim()));
            TRY(dwim_resize(dev, k, n * k_dim()));
            TRY(dwim_resize(dev, v, n * v_dim()));
            TRY(dwim_resize(dev, att, n * v_dim()));
            auto &pair = seq.conv_state[l.slot];
            dwim_buf *state = seq.parity ? pair[0] : pair[1];
            dwim_buf *state_out = seq.parity ? pair[1] : pair[0];
            dwim_buf *ssm = verify ? ssm_scratch[l.slot] : seq.ssm_state[l.slot];
            if (fused) {
                // a verified batch's projections go straight to where rewind
                // reads them, and its state runs from the real one into the
                // scratch (no copies)
                dwim_buf *qkv_in = verify ? qkv_saved[l.slot] : qkv, *ab_in = verify ? ab_saved[l.slot] : ab;
                if (verify) {
                    TRY(dwim_resize(dev, qkv_in, n * (2 * k_dim() + v_dim())));
                    TRY(dwim_resize(dev, ab_in, n * 2 * c.v_heads));
                }
                const dwim_weight *ws[2] = {l.qkv, l.z};
                dwim_buf *outs[2] = {qkv_in, z};
                if (n >= 16 && l.ab->fmt == DWIM_BF16 && l.ab->rows <= 96 && l.qkv->fmt == DWIM_Q4_K) {
                    // the gate projection over the same split as qkv and z
                    TRY(projections(ws, outs, 2, l.attn_norm, n, nullptr));
                    TRY(dwim_resize(dev, ab_in, n * 2 * c.v_heads));
                    DWIM_HIP(gemm_run_bf16(dev, l.ab, ab_in->data, n, 0));
                } else if (bh) {
                    // (the gate rows in the same launch, from xh: x·attn_norm
                    // handed over, RMS-scaled like the products, or the
                    // normalized rows the launch makes)
                    TRY(batch_input(ws, outs, 2, l.attn_norm, n, in_set, xh, l.ab, ab_in));
                } else {
                    TRY(projections(ws, outs, 2, l.attn_norm, n, xh));
                    TRY(dwim_matmul(dev, ab_in, l.ab, xh));
                }
                if (n <= 16 && c.state_dim == 128) {
                    // conv, key norms and delta rule in one launch (verifying:
                    // from the real state into the scratch, the states after
                    // the first tokens kept for a rewind)
                    GdnSteps st{};
                    if (verify && steps_kept(n))
                        for (size_t t = 0; t + 1 < n; t++) {
                            st.state[t] = ssm_step[t][l.slot]->data;
                            st.conv[t] = conv_step[t][l.slot]->data;
                        }
                    // (handing over: its output gate's planes, heads unnormalized)
                    GdnGate gg;
                    if (bh) {
                        gg.z = z->data;
                        gg.norm_w = l.norm->data;
                        gg.planes = planes_area(dev, kBatchArea, v_dim()).q;
                        gg.head_ss = batch_hss->data;
                    }
                    DWIM_HIP(launch_gdn_tokens(dev, att->data, qkv_in->data, state->data, state_out->data,
                                               l.conv->data, ab_in->data, l.decay->data, ssm->data,
                                               verify ? seq.ssm_state[l.slot]->data : nullptr, n, c.k_heads,
                                               c.v_heads, c.state_dim, eps, &st, bh ? &gg : nullptr));
                } else {
                    TRY(dwim_conv_l2norm(dev, q, k, v, state_out, qkv_in, state, l.conv, c.state_dim, eps));
                    if (verify) {
                        DWIM_HIP(launch_delta_net(dev, att->data, q->data, k->data, v->data, ab_in->data,
                                                  l.decay->data, ssm->data, n, c.k_heads, c.v_heads, c.state_dim,
                                                  nullptr, true, seq.ssm_state[l.slot]->data));
                    } else {
                        TRY(dwim_delta_net_unit_keys(dev, att, q, k, v, ab, l.decay, ssm, c.k_heads, c.v_heads,
                                                     c.state_dim));
                    }
                }
                if (n >= 16 && l.out->fmt == DWIM_Q4_K) {
                    // the gated norm made in the out product's split
                    DWIM_HIP(gemm_prepare_gated(dev, z->data, att->data, l.norm->data, eps, n, v_dim(), c.state_dim));
                    DWIM_HIP(gemm_run(dev, l.out, x->data, n, kGemmAdd));
                } else if (bh) {
                    TRY(batch_residual(l.out, nullptr, n, nullptr, nullptr, l.mlp_norm, batch_hss));
                } else if (l.out->fmt == DWIM_Q4_K && c.state_dim == 128) {
                    // the gated norm made with the out product's planes
                    const int add = 1;
                    float *o = x->data;
                    DWIM_HIP(launch_mv_q4k_mfma_tokens(dev, &l.out, &o, &add, 1, 0, att->data, n, l.norm->data, eps,
                                                       nullptr, z->data));
                } else {
                    DWIM_HIP(launch_gated_norm(dev, z->data, att->data, l.norm->data, n, v_dim(), c.state_dim, eps,
                                               -1));
                    TRY(dwim_matmul_add(dev, x, l.out, z, xb));
                }
            } else {
                TRY(dwim_matmul(dev, qkv, l.qkv, xh));
                TRY(dwim_matmul(dev, z, l.z, xh));
                TRY(dwim_matmul(dev, ab, l.ab, xh));
                if (verify) TRY(save_inputs(l.slot, n));
                TRY(dwim_conv(dev, q, k, v, state_out, qkv, state, l.conv));
                TRY(dwim_l2norm(dev, q, c.state_dim, eps));
                TRY(dwim_l2norm(dev, k, c.state_dim, eps));
                TRY(dwim_delta_net(dev, att, q, k, v, ab, l.decay, ssm, c.k_heads, c.v_heads, c.state_dim));
                TRY(dwim_rmsnorm(dev, att, l.norm, eps));
                TRY(dwim_silu_mul(dev, z, att));
                TRY(dwim_matmul_add(dev, x, l.out, z, xb));
            }
        }
        if (fused && n >= 16 && l.down->fmt == DWIM_Q4_K) {
            // gate and up in one launch, the SwiGLU in the down product's split
            TRY(dwim_resize(dev, up, n * c.intermediate));
            TRY(dwim_resize(dev, gate_ffn, n * c.intermediate));
            DWIM_HIP(launch_ffn_q4k(dev, l.gate, l.up, l.down, x->data, n, l.mlp_norm->data, eps, gate_ffn->data,
                                    up->data));
            return 0;
        }
        if (bh) return batch_ffn(l, n, next);
        if (fused) {
            DWIM_HIP(launch_swiglu_q4k(dev, l.gate, l.up, up->data, x->data, n, l.mlp_norm->data, eps));
        } else {
            TRY(normalize(xh, x, l.mlp_norm, n));
            TRY(dwim_swiglu(dev, up, l.gate, l.up, xh, gate_ffn));
        }
        TRY(dwim_matmul_add(dev, x, l.down, up, xb));
        return 0;
    }

    // the verified batch's inputs of linear layer `slot`, and its state
    int save_inputs(size_t slot, size_t n) {
        TRY(dwim_resize(dev, qkv_saved[slot], n * (2 * k_dim() + v_dim())));
        TRY(dwim_resize(dev, ab_saved[slot], n * 2 * c.v_heads));
        TRY(dwim_copy(dev, qkv_saved[slot], 0, qkv, 0, n * (2 * k_dim() + v_dim())));
        TRY(dwim_copy(dev, ab_saved[slot], 0, ab, 0, n * 2 * c.v_heads));
        return dwim_copy(dev, ssm_scratch[slot], 0, seq.ssm_state[slot], 0, ssm_width());
    }

    // Pass::drafter (qwen35/mod.rs:663-698), fed rows of seq.hidden from `first`
    int drafter(size_t rows, size_t pos, size_t first, bool chain, const uint32_t *tokens) {
        if (rows == 0) return 0;
        TRY(batch(rows));
        TRY(dwim_embed(dev, xb, embd, tokens, rows));
        TRY(dwim_rmsnorm(dev, xb, draft.embed_norm, c.eps));
        if (chain)
            TRY(dwim_copy(dev, xh, 0, drafted, 0, c.hidden));
        else
            TRY(dwim_copy(dev, xh, 0, seq.hidden, first * c.hidden, rows * c.hidden));
        TRY(dwim_rmsnorm(dev, xh, draft.hidden_norm, c.eps));
        TRY(dwim_matmul(dev, x, draft.embed_proj, xb));
        TRY(dwim_matmul(dev, xb, draft.hidden_proj, xh));
        TRY(dwim_add(dev, x, xb));
        handed = false;
        batch_in = -1;
        TRY(layer(draft.layer, rows, pos));
        return normalize(xh, x, draft.norm, rows);
    }

    // State::carry_over (qwen35/mod.rs:1466-1473)
    int carry_over(size_t n) {
        const size_t h = c.hidden;
        TRY(dwim_resize(dev, xb, h));
        TRY(dwim_copy(dev, xb, 0, seq.hidden, n * h, h));
        TRY(dwim_copy(dev, seq.hidden, 0, xb, 0, h));
        seq.carry = true;
        return 0;
    }

    int finish() {
        float one;
        TRY(dwim_resize(dev, xb, 1));
        return dwim_read(dev, xb, &one, 1);
    }

    // forward_batch (qwen35/mod.rs:425-496).  With `logits_out` the logits
    // after the last token are read back, or verifying, after every token;
    // with `greedy` the first index of each row's maximum is taken on the
    // device.
    int forward_batch(const uint32_t *tokens, size_t n, size_t pos, bool verify, bool wanted, float *logits_out,
                      uint32_t *greedy) {
        TRY(batch(n));
        if (embed_from) {
            DWIM_HIP(launch_embed(dev->stream, x->data, embd, embed_from, n));
        } else {
            TRY(dwim_embed(dev, x, embd, tokens, n));
        }
        handed = false;
        batch_in = -1;
        for (size_t i = 0; i < layers.size(); i++)
            TRY(layer(layers[i], n, pos, verify, i + 1 < layers.size() ? &layers[i + 1] : nullptr));
        if (!verify) seq.parity = !seq.parity;
        const size_t h = c.hidden;
        if (!has_draft) {
            if (!wanted) return finish();
            if (n == 1 && head->fmt == DWIM_Q6_K && h % 256 == 0 && h <= planes::kMaxCols) {
                // the output norm inside the head's planes (one launch
                // instead of a copy, an RMS norm and the planes)
                DWIM_HIP(launch_planes(dev, x->data, h, norm->data, c.eps, nullptr, 0, 0));
                TRY(dwim_resize(dev, logits, c.vocab));
                DWIM_HIP(launch_mv_q6k_mfma(dev, head, logits->data, 0));
                return read_logits(logits_out, greedy);
            }
            TRY(dwim_resize(dev, xb, h));
            TRY(dwim_resize(dev, xh, h));
            TRY(dwim_copy(dev, xb, 0, x, (n - 1) * h, h));
            TRY(normalize(xh, xb, norm, 1));
            TRY(dwim_resize(dev, logits, c.vocab));
            TRY(dwim_matmul(dev, logits, head, xh));
            return read_logits(logits_out, greedy);
        }
        TRY(normalize(xh, x, norm, n));
        TRY(dwim_copy(dev, seq.hidden, h, xh, 0, n * h));
        if (verify) {
            seq.verified.assign(tokens, tokens + n);
            seq.verified_at = pos;
            TRY(dwim_resize(dev, logits, n * c.vocab));
            TRY(dwim_matmul(dev, logits, head, xh));
            return read_logits(logits_out, greedy, n);
        }
        if (wanted) {
            TRY(dwim_resize(dev, xb, h));
            TRY(dwim_copy(dev, xb, 0, xh, (n - 1) * h, h));
            TRY(dwim_resize(dev, logits, c.vocab));
            TRY(dwim_matmul(dev, logits, head, xb));
        }
        const size_t first = seq.carry ? 0 : 1;
        TRY(drafter(n - first, pos + first - 1, first, false, tokens + first));
        TRY(carry_over(n));
        if (wanted) return read_logits(logits_out, greedy);
        return finish();
    }

    int read_logits(float *logits_out, uint32_t *greedy, size_t rows = 1) {
        if (argmax_to) {
            // the pick stays on the device, where the next step's embedding reads it
            DWIM_HIP(launch_argmax(dev->stream, logits->data, rows, c.vocab, argmax_to));
            return 0;
        }
        if (greedy) TRY(dwim_argmax(dev, logits, rows, greedy));
        if (logits_out) TRY(dwim_read(dev, logits, logits_out, rows * c.vocab));
        if (!greedy && !logits_out) return finish();
        return 0;
    }

    // LanguageModel::forward (qwen35/mod.rs:1021-1038)
    int forward(const uint32_t *tokens, size_t n, size_t pos, float *logits_out, uint32_t *greedy) {
        if (n == 0) return dwim_fail("no tokens to run");
        if (pos + n > seq.max_len) return dwim_fail("tokens past the end of the cache");
        const size_t batches = (n + most - 1) / most;
        for (size_t i = 0; i < batches; i++) {
            const size_t m = std::min(most, n - i * most);
            const bool last = i + 1 == batches;
            TRY(forward_batch(tokens + i * most, m, pos + i * most, false, last, last ? logits_out : nullptr,
                              last ? greedy : nullptr));
        }
        return 0;
    }

    // Greedy decoding of `steps` tokens from `token` at `pos`, as the reply
    // loop runs it token by token (inference/local.rs:162-240, each step
    // LanguageModel::forward of the token picked, qwen35/mod.rs:1021-1038,
    // then qwen35::argmax).  Each step's pick stays on the device: the argmax
    // writes it into `picks` and the next step's embedding reads it there, so
    // the host queues every step without waiting and reads the picks back
    // once.  picks[0] is the first token; step i's argmax writes picks[i+1]
    // and uses the words after it as its partials, which step i+1's pick then
    // overwrites, in stream order.  A drafting model runs the steps one by
    // one (its drafter takes the token ids on the host).
    int decode_greedy(uint32_t token, size_t pos, size_t steps, uint32_t *out) {
        if (steps == 0) return 0;
        if (token >= embd->rows) return dwim_fail("decode: token " + std::to_string(token) + " is past the table");
        if (pos + steps > seq.max_len) return dwim_fail("tokens past the end of the cache");
        if (has_draft) {
            for (size_t i = 0; i < steps; i++) {
                TRY(forward(&token, 1, pos + i, nullptr, &token));
                out[i] = token;
            }
            return 0;
        }
        if (c.vocab > embd->rows) return dwim_fail("decode: the head picks tokens past the embedding table");
        const size_t words = steps + 1 + argmax_scratch_words(1);
        DWIM_HIP(dev_grow(dev, (void **)&picks, &picks_cap, words, 4));
        DWIM_HIP(hipMemcpyAsync(picks, &token, 4, hipMemcpyHostToDevice, dev->stream));
        // the pageable source is read before the call returns; waiting here
        // keeps that so whatever the runtime does with small copies
        DWIM_HIP(hipStreamSynchronize(dev->stream));
        int err = 0;
        for (size_t i = 0; i < steps && !err; i++) {
            embed_from = picks + i;
            argmax_to = picks + i + 1;
            err = forward_batch(nullptr, 1, pos + i, false, true, nullptr, nullptr);
        }
        embed_from = argmax_to = nullptr;
        TRY(err);
        DWIM_HIP(hipMemcpyAsync(out, picks + 1, steps * 4, hipMemcpyDeviceToHost, dev->stream));
        DWIM_HIP(hipStreamSynchronize(dev->stream));
        return 0;
    }

    // LanguageModel::draft (qwen35/mod.rs:1045-1071): the drafter at the
    // position before `token`, fed the hidden state carried over, then on
    // its own output, `k` times; each draft the head's greedy pick, taken on
    // the device.  Returns how many were drafted.
    size_t draft_tokens(uint32_t token, size_t pos, size_t k, uint32_t *drafts, int *status) {
        *status = 0;
        if (!has_draft) return 0;
        k = std::min(k, kMaxDrafts);
        k = std::min(k, seq.max_len > pos + 1 ? seq.max_len - (pos + 1) : (size_t)0);
        if (!seq.carry || !seq.verified.empty() || pos == 0 || k == 0) return 0;
        uint32_t next = token;
        for (size_t i = 0; i < k; i++) {
            if (drafter(1, pos - 1 + i, 0, i > 0, &next) || dwim_copy(dev, drafted, 0, xh, 0, c.hidden) ||
                dwim_resize(dev, logits, c.vocab) || dwim_matmul(dev, logits, head, xh) ||
                dwim_argmax(dev, logits, 1, &next)) {
                *status = 1;
                return i;
            }
            drafts[i] = next;
        }
        return k;
    }

    // LanguageModel::verify (qwen35/mod.rs:1073-1091)
    int verify(const uint32_t *tokens, size_t n, size_t pos, float *logits_out, uint32_t *greedy) {
        if (!has_draft) return dwim_fail("the model does not draft");
        if (!seq.verified.empty() || !seq.carry) return dwim_fail("a batch is being verified, or none was run before");
        if (n == 0 || n > kMaxDrafts + 1)
            return dwim_fail("a batch of " + std::to_string(n) + " tokens is not one to verify");
        if (pos + n > seq.max_len) return dwim_fail("tokens past the end of the cache");
        return forward_batch(tokens, n, pos, true, true, logits_out, greedy);
    }

    // LanguageModel::rewind (qwen35/mod.rs:1099-1169): commits the first
    // `keep` tokens of the batch being verified.  All kept, the states the
    // batch ran through become the real ones; fewer, the real ones run
    // through the tokens kept from the inputs saved.  Then the drafter
    // catches up on the tokens kept.
    int rewind(size_t keep) {
        const size_t n = seq.verified.size();
        if (n == 0 || keep == 0 || keep > n)
            return dwim_fail("keeping " + std::to_string(keep) + " tokens of a batch of " + std::to_string(n) +
                             " being verified");
        const std::vector<uint32_t> tokens = std::move(seq.verified);
        seq.verified.clear();
        if (keep == n) {
            for (size_t slot = 0; slot < slots; slot++) std::swap(seq.ssm_state[slot], ssm_scratch[slot]);
        } else if (steps_kept(n)) {
            // the states after token keep - 1, as the batch left them (the
            // same arithmetic as running the kept tokens again)
            for (const Layer &l : layers) {
                if (l.attention) continue;
                auto &pair = seq.conv_state[l.slot];
                dwim_buf *&conv_out = seq.parity ? pair[1] : pair[0];
                std::swap(seq.ssm_state[l.slot], ssm_step[keep - 1][l.slot]);
                std::swap(conv_out, conv_step[keep - 1][l.slot]);
            }
        } else {
            TRY(batch(keep));
            TRY(dwim_resize(dev, q, keep * k_dim()));
            TRY(dwim_resize(dev, k, keep * k_dim()));
            TRY(dwim_resize(dev, v, keep * v_dim()));
            TRY(dwim_resize(dev, att, keep * v_dim()));
            for (const Layer &l : layers) {
                if (l.attention) continue;
                auto &pair = seq.conv_state[l.slot];
                dwim_buf *state = seq.parity ? pair[0] : pair[1];
                dwim_buf *state_out = seq.parity ? pair[1] : pair[0];
                if (fusable(l)) {
                    // as the batch ran: conv and key norms in one launch, the
                    // saved inputs read where they lie
                    TRY(dwim_resize(dev, qkv_saved[l.slot], keep * (2 * k_dim() + v_dim())));
                    TRY(dwim_resize(dev, ab_saved[l.slot], keep * 2 * c.v_heads));
                    if (keep <= 16 && c.state_dim == 128) {
                        // conv, key norms and delta rule in one launch
                        DWIM_HIP(launch_gdn_tokens(dev, nullptr, qkv_saved[l.slot]->data, state->data,
                                                   state_out->data, l.conv->data, ab_saved[l.slot]->data,
                                                   l.decay->data, seq.ssm_state[l.slot]->data, nullptr, keep,
                                                   c.k_heads, c.v_heads, c.state_dim, c.eps));
                        continue;
                    }
                    TRY(dwim_conv_l2norm(dev, q, k, v, state_out, qkv_saved[l.slot], state, l.conv, c.state_dim,
                                         c.eps));
                    TRY(dwim_delta_net_unit_keys(dev, att, q, k, v, ab_saved[l.slot], l.decay,
                                                 seq.ssm_state[l.slot], c.k_heads, c.v_heads, c.state_dim));
                    continue;
                }
                TRY(dwim_copy(dev, qkv, 0, qkv_saved[l.slot], 0, keep * (2 * k_dim() + v_dim())));
                TRY(dwim_copy(dev, ab, 0, ab_saved[l.slot], 0, keep * 2 * c.v_heads));
                TRY(dwim_conv(dev, q, k, v, state_out, qkv, state, l.conv));
                TRY(dwim_l2norm(dev, q, c.state_dim, c.eps));
                TRY(dwim_l2norm(dev, k, c.state_dim, c.eps));
                TRY(dwim_delta_net(dev, att, q, k, v, ab, l.decay, seq.ssm_state[l.slot], c.k_heads, c.v_heads,
                                   c.state_dim));
            }
        }
        seq.parity = !seq.parity;
        TRY(drafter(keep, seq.verified_at - 1, 0, false, tokens.data()));
        TRY(carry_over(keep));
        return finish();
    }

    // LanguageModel::mark (qwen35/mod.rs:1176-1203): the linear layers'
    // states and the carried hidden state, copied aside on the device
    int mark() {
        if (!seq.verified.empty()) return dwim_fail("a batch is being verified");
        for (size_t slot = 0; slot < slots; slot++) {
            TRY(dwim_copy(dev, mark_conv[slot], 0, seq.conv_state[slot][seq.parity ? 0 : 1], 0, conv_width()));
            TRY(dwim_copy(dev, mark_ssm[slot], 0, seq.ssm_state[slot], 0, ssm_width()));
        }
        if (seq.carry) TRY(dwim_copy(dev, mark_hidden, 0, seq.hidden, 0, c.hidden));
        mark_carry = seq.carry;
        marked = (long)seq.id;
        return 0;
    }

    // LanguageModel::rewind_to_mark (qwen35/mod.rs:1207-1228)
    int rewind_to_mark() {
        if (marked != (long)seq.id) return dwim_fail("no mark to rewind to");
        if (!seq.verified.empty()) return dwim_fail("a batch is being verified");
        for (size_t slot = 0; slot < slots; slot++) {
            TRY(dwim_copy(dev, seq.conv_state[slot][0], 0, mark_conv[slot], 0, conv_width()));
            TRY(dwim_copy(dev, seq.ssm_state[slot], 0, mark_ssm[slot], 0, ssm_width()));
        }
        seq.parity = true;
        if (mark_carry) TRY(dwim_copy(dev, seq.hidden, 0, mark_hidden, 0, c.hidden));
        seq.carry = mark_carry;
        return 0;
    }

    // LanguageModel::add_sequence (qwen35/mod.rs:1258-1272)
    int add_sequence(size_t *id) {
        const size_t next = parked.size() + 1;
        Sequence s;
        TRY(new_sequence(s, next, seq.max_len));
        parked.emplace(next, std::move(s));
        *id = next;
        return dwim_sync(dev);
    }

    // LanguageModel::select_sequence (qwen35/mod.rs:1275-1290): nothing copied
    int select_sequence(size_t id) {
        if (seq.id == id) return 0;
        if (!seq.verified.empty()) return dwim_fail("a batch is being verified");
        auto it = parked.find(id);
        if (it == parked.end()) return dwim_fail("no sequence " + std::to_string(id));
        Sequence next = std::move(it->second);
        parked.erase(it);
        const size_t old = seq.id;
        parked.emplace(old, std::move(seq));
        seq = std::move(next);
        return 0;
    }

    // LanguageModel::save (qwen35/mod.rs:905-947): the "dwimstat" layout of
    // version 3, all little-endian: magic, version u32, then seven u64 (len,
    // attention caches, linear slots, kv_dim, conv width, ssm width, hidden
    // or 0 without a drafter); every key cache's first len·kv_dim activations
    // as read_cache gives them, then every value cache's; per linear slot its
    // conv state (the buffer the next batch reads) and its recurrent state as
    // f32; with a drafter, the hidden state carried over.  `bytes` is 0 when
    // there is no state to save (a batch being verified, or a drafter with
    // nothing carried over), as the reference returns None.
    size_t state_bytes(size_t len) const {
        size_t b = 8 + 4 + 7 * 8 + 2 * caches * (len * kv_dim() + len * kv_dim() / 32 * 2);
        b += slots * (conv_width() + ssm_width()) * 4;
        if (has_draft) b += c.hidden * 4;
        return b;
    }
    int save(size_t len, uint8_t *out, size_t cap, size_t *bytes) {
        *bytes = 0;
        if (!seq.verified.empty() || (has_draft && !seq.carry)) return 0;
        if (len > seq.max_len || (len * kv_dim()) % 32 != 0)
            return dwim_fail("save: " + std::to_string(len) + " positions do not fit the context");
        const size_t need = state_bytes(len);
        if (!out) {
            *bytes = need;
            return 0;
        }
        if (cap < need) return dwim_fail("save: a buffer of " + std::to_string(cap) + " bytes can't hold " +
                                         std::to_string(need));
        uint8_t *p = out;
        memcpy(p, "dwimstat", 8);
        p += 8;
        const uint32_t version = 3;
        memcpy(p, &version, 4);
        p += 4;
        const uint64_t header[7] = {len, caches, slots, kv_dim(), conv_width(), ssm_width(),
                                    has_draft ? c.hidden : 0};
        memcpy(p, header, sizeof header);
        p += sizeof header;
        const size_t cache_len = len * kv_dim(), cache_bytes = cache_len + cache_len / 32 * 2;
        for (int kv = 0; kv < 2; kv++)
            for (size_t i = 0; i < caches; i++) {
                TRY(dwim_read_cache(dev, kv ? seq.v_cache[i] : seq.k_cache[i], cache_len, p, cache_bytes));
                p += cache_bytes;
            }
        for (size_t slot = 0; slot < slots; slot++) {
            TRY(dwim_read(dev, seq.conv_state[slot][seq.parity ? 0 : 1], (float *)p, conv_width()));
            p += conv_width() * 4;
            TRY(dwim_read(dev, seq.ssm_state[slot], (float *)p, ssm_width()));
            p += ssm_width() * 4;
        }
        if (has_draft) {
            // the carried row, through xb (the first c.hidden of seq.hidden)
            TRY(dwim_resize(dev, xb, c.hidden));
            TRY(dwim_copy(dev, xb, 0, seq.hidden, 0, c.hidden));
            TRY(dwim_read(dev, xb, (float *)p, c.hidden));
            p += c.hidden * 4;
        }
        *bytes = (size_t)(p - out);
        return 0;
    }

    // LanguageModel::restore (qwen35/mod.rs:949-1017), with its checks and
    // messages; the conv state goes to the first buffer of each pair, read
    // next with the parity set.
    int restore(const uint8_t *state, size_t bytes, size_t *len_out) {
        size_t at = 0;
        auto take = [&](size_t n, const uint8_t **ptr) -> int {
            if (at + n > bytes) return dwim_fail("the saved state is cut short");
            *ptr = state + at;
            at += n;
            return 0;
        };
        const uint8_t *ptr;
        TRY(take(8, &ptr));
        if (memcmp(ptr, "dwimstat", 8) != 0) return dwim_fail("not a saved state");
        TRY(take(4, &ptr));
        uint32_t version;
        memcpy(&version, ptr, 4);
        if (version != 3) return dwim_fail("a saved state of another version");
        uint64_t header[7];
        TRY(take(sizeof header, &ptr));
        memcpy(header, ptr, sizeof header);
        const uint64_t want[6] = {caches, slots, kv_dim(), conv_width(), ssm_width(), has_draft ? c.hidden : 0};
        if (memcmp(header + 1, want, sizeof want) != 0) return dwim_fail("a saved state of another model");
        const size_t len = header[0];
        if (len > seq.max_len)
            return dwim_fail("a saved state of " + std::to_string(len) + " tokens does not fit in the context");
        if ((len * kv_dim()) % 32 != 0) return dwim_fail("a saved state of another model");
        // every section is checked for length before any is written
        const size_t cache_len = len * kv_dim(), cache_bytes = cache_len + cache_len / 32 * 2;
        const size_t need = 2 * caches * cache_bytes + slots * (conv_width() + ssm_width()) * 4 +
                            (has_draft ? c.hidden * 4 : 0);
        if (bytes - at < need) return dwim_fail("the saved state is cut short");
        for (int kv = 0; kv < 2; kv++)
            for (size_t i = 0; i < caches; i++) {
                TRY(take(cache_bytes, &ptr));
                TRY(dwim_write_cache(dev, kv ? seq.v_cache[i] : seq.k_cache[i], ptr, cache_bytes));
            }
        for (size_t slot = 0; slot < slots; slot++) {
            TRY(take(conv_width() * 4, &ptr));
            TRY(dwim_write(dev, seq.conv_state[slot][0], (const float *)ptr, conv_width()));
            TRY(take(ssm_width() * 4, &ptr));
            TRY(dwim_write(dev, seq.ssm_state[slot], (const float *)ptr, ssm_width()));
        }
        seq.parity = true;
        seq.verified.clear();
        if (marked == (long)seq.id) marked = -1;
        if (has_draft) {
            TRY(take(c.hidden * 4, &ptr));
            TRY(dwim_resize(dev, xb, c.hidden));
            TRY(dwim_write(dev, xb, (const float *)ptr, c.hidden));
            TRY(dwim_copy(dev, seq.hidden, 0, xb, 0, c.hidden));
            seq.carry = true;
        }
        *len_out = len;
        return dwim_sync(dev);
    }

    // Every device scratch buffer a forward pass can grow, at its largest for
    // this model, now: a forward pass then never frees and allocates (which
    // would wait for the device) in the middle of its launches.
    int reserve(size_t max_len, int fmt) {
        const size_t small = std::min(most, (size_t)15);  // the decode attention's most tokens
        DWIM_HIP(attention_reserve(
            dev, attention_partials_floats(small, max_len > small ? max_len - small : 0, c.heads, c.head_dim)));
        DWIM_HIP(delta_net_reserve(dev, most, c.v_heads));
        if (c.head_dim == 256 && most >= 16) DWIM_HIP(attention_kvx_reserve(dev, attention_kvx_bytes(max_len, c.kv_heads)));
        if (fmt == DWIM_Q4_K) {
            const size_t H = c.hidden, I = c.intermediate;
            const size_t shapes[][2] = {{q_dim(), H}, {kv_dim(), H}, {H, q_dim()}, {2 * k_dim() + v_dim(), H},
                                        {v_dim(), H}, {H, v_dim()}, {I, H}, {H, I}, {H, H}};
            size_t split = 0, parts = 0, cols_max = 0;
            for (auto &rc : shapes) {
                cols_max = std::max(cols_max, rc[1]);
                for (size_t n = 16; n <= most; n++) {
                    split = std::max(split, gemm_split_bytes(n, rc[1]));
                    parts = std::max(parts, gemm_parts_floats(n, rc[0], rc[1]));
                }
            }
            DWIM_HIP(gemm_reserve(dev, split, parts));
            if (!dev_work(dev, most * cols_max)) return dwim_fail("reserving the normalized activations failed");
        }
        DWIM_HIP(dev_grow(dev, (void **)&dev->tokens, &dev->tokens_cap, most, 4));
        DWIM_HIP(dev_grow(dev, (void **)&dev->argmax_buf, &dev->argmax_cap, argmax_scratch_words(kMaxDrafts + 1), 4));
        return 0;
    }

    // LanguageModel::reset (qwen35/mod.rs:1230-1246)
    int reset() {
        std::vector<float> zeros(std::max(conv_width(), ssm_width()), 0.0f);
        for (size_t s = 0; s < slots; s++) {
            for (dwim_buf *b : seq.conv_state[s]) TRY(dwim_write(dev, b, zeros.data(), conv_width()));
            TRY(dwim_write(dev, seq.ssm_state[s], zeros.data(), ssm_width()));
        }
        seq.parity = false;
        seq.carry = false;
        seq.verified.clear();
        if (marked == (long)seq.id) marked = -1;
        return 0;
    }

    ~dwim_model() {
        if (picks) {
            (void)hipStreamSynchronize(dev->stream);
            (void)hipFree(picks);
        }
        for (auto *b : bufs) dwim_free_buffer(b);
        for (auto *w : weights) dwim_free_weight(w);
        for (auto *cc : cache_list) dwim_free_cache(cc);
    }
};

// rope_table (qwen35/mod.rs:1504-1515): cos, sin of pos·theta^(-2i/rot)
static void rope_table(std::vector<float> &t, size_t max_len, size_t rot, float theta) {
    const size_t half = rot / 2;
    t.resize(max_len * rot);
    for (size_t pos = 0; pos < max_len; pos++)
        for (size_t i = 0; i < half; i++) {
            const float freq = 1.0f / powf(theta, (float)(2 * i) / (float)rot);
            const float a = (float)pos * freq;
            t[(pos * half + i) * 2] = cosf(a);
            t[(pos * half + i) * 2 + 1] = sinf(a);
        }
}

extern "C" int dwim_model_synthetic(dwim_dev *dev, const dwim_qwen35_config *cfg, uint64_t seed, int body_format,
                                    int head_format, size_t max_len, dwim_model **out) {
    *out = nullptr;
    const dwim_qwen35_config &c = *cfg;
    if (c.full_attention_interval == 0 || c.k_heads == 0 || c.v_heads % c.k_heads != 0 || c.head_dim % 32 != 0 ||
        max_len == 0)
        return dwim_fail("model: an inconsistent configuration");
    std::unique_ptr<dwim_model> m(new dwim_model());
    m->dev = dev;
    m->c = c;
    m->seed = seed;
    m->most = dwim_batch(dev);
    for (size_t i = 0; i < c.layers; i++) {
        m->layers.emplace_back();
        if (m->load_layer(i, m->is_attention(i), body_format, m->layers.back())) return 1;
    }
    if (m->vec("output_norm", c.hidden, 0.1f, 1.0f, &m->norm)) return 1;
    if (m->mat("output", head_format, c.vocab, c.hidden, 0.02f, &m->head)) return 1;
    if (m->mat("token_embd", body_format, c.vocab, c.hidden, 1.0f, &m->embd)) return 1;
    if (c.drafter) {
        m->has_draft = true;
        const std::string p = "blk." + std::to_string(c.layers) + ".";
        if (m->vec(p + "enorm", c.hidden, 0.1f, 1.0f, &m->draft.embed_norm) ||
            m->vec(p + "hnorm", c.hidden, 0.1f, 1.0f, &m->draft.hidden_norm) ||
            m->mat(p + "eh_proj.embed", body_format, c.hidden, c.hidden, 0.02f, &m->draft.embed_proj) ||
            m->mat(p + "eh_proj.hidden", body_format, c.hidden, c.hidden, 0.02f, &m->draft.hidden_proj) ||
            m->load_layer(c.layers, true, body_format, m->draft.layer) ||
            m->vec(p + "shared_head_norm", c.hidden, 0.1f, 1.0f, &m->draft.norm))
            return 1;
    }
    // State::new (qwen35/mod.rs:1416-1460)
    const size_t q_dim = m->q_dim(), kv_dim = m->kv_dim(), k_dim = m->k_dim(), v_dim = m->v_dim();
    m->widths = {c.hidden,
                 c.hidden,
                 c.hidden,
                 std::max(q_dim, k_dim),
                 q_dim,
                 std::max(kv_dim, k_dim),
                 std::max(kv_dim, v_dim),
                 std::max(q_dim, v_dim),
                 2 * k_dim + v_dim,
                 v_dim,
                 2 * c.v_heads};
    dwim_buf **b[11] = {&m->x, &m->xb, &m->xh, &m->q, &m->gate, &m->k, &m->v, &m->att, &m->qkv, &m->z, &m->ab};
    for (int i = 0; i < 11; i++)
        if (m->buf(m->most * m->widths[i], b[i])) return 1;
    if (m->buf(m->most * c.intermediate, &m->up) || m->buf(m->most * c.intermediate, &m->gate_ffn) ||
        m->buf((c.drafter ? kMaxDrafts + 1 : 1) * c.vocab, &m->logits) || m->buf(c.hidden, &m->drafted) ||
        m->buf(4 * c.v_heads, &m->head_ss) || m->buf(4 * c.v_heads * 8, &m->batch_hss))
        return 1;
    std::vector<float> table;
    rope_table(table, max_len, c.rot_dim, c.rope_theta);
    if (m->buf(table.size(), &m->rope) || dwim_write(dev, m->rope, table.data(), table.size())) return 1;
    for (size_t i = 0; i < m->slots; i++) {
        dwim_buf *mc, *ms;
        if (m->buf(m->conv_width(), &mc) || m->buf(m->ssm_width(), &ms)) return 1;
        m->mark_conv.push_back(mc);
        m->mark_ssm.push_back(ms);
        if (c.drafter) {
            // verify batches hold at most MAX_DRAFTS + 1 tokens
            dwim_buf *sc, *qs, *as;
            if (m->buf(m->ssm_width(), &sc) || m->buf((kMaxDrafts + 1) * (2 * k_dim + v_dim), &qs) ||
                m->buf((kMaxDrafts + 1) * 2 * c.v_heads, &as))
                return 1;
            m->ssm_scratch.push_back(sc);
            m->qkv_saved.push_back(qs);
            m->ab_saved.push_back(as);
            if (c.state_dim == 128)
                for (int t = 0; t < kMaxSteps; t++) {
                    dwim_buf *ss, *cs;
                    if (m->buf(m->ssm_width(), &ss) || m->buf(m->conv_width(), &cs)) return 1;
                    m->ssm_step[t].push_back(ss);
                    m->conv_step[t].push_back(cs);
                }
        }
    }
    if (m->buf(c.hidden, &m->mark_hidden)) return 1;
    if (m->new_sequence(m->seq, 0, max_len)) return 1;
    if (m->reserve(max_len, body_format)) return 1;
    if (dwim_sync(dev)) return 1;
    *out = m.release();
    return 0;
}

extern "C" void dwim_model_free(dwim_model *m) { delete m; }

extern "C" size_t dwim_model_batch(const dwim_model *m) { return m->most; }

extern "C" int dwim_model_forward(dwim_model *m, const uint32_t *tokens, size_t n, size_t pos, float *logits) {
    return m->forward(tokens, n, pos, logits, nullptr);
}

extern "C" int dwim_model_forward_greedy(dwim_model *m, const uint32_t *tokens, size_t n, size_t pos, uint32_t *next) {
    return m->forward(tokens, n, pos, nullptr, next);
}

extern "C" int dwim_model_decode_greedy(dwim_model *m, uint32_t token, size_t pos, size_t steps, uint32_t *out) {
    return m->decode_greedy(token, pos, steps, out);
}

extern "C" int dwim_model_reset(dwim_model *m) { return m->reset(); }

extern "C" int dwim_model_draft(dwim_model *m, uint32_t token, size_t pos, size_t k, uint32_t *drafts, size_t *count) {
    int status = 0;
    *count = m->draft_tokens(token, pos, k, drafts, &status);
    return status;
}

extern "C" int dwim_model_verify(dwim_model *m, const uint32_t *tokens, size_t n, size_t pos, float *logits,
                                 uint32_t *greedy) {
    return m->verify(tokens, n, pos, logits, greedy);
}

extern "C" int dwim_model_rewind(dwim_model *m, size_t keep) { return m->rewind(keep); }

extern "C" int dwim_model_logits(dwim_model *m, const dwim_buf **out) {
    *out = m->logits;
    return 0;
}

extern "C" int dwim_model_mark(dwim_model *m) { return m->mark(); }

extern "C" int dwim_model_rewind_to_mark(dwim_model *m) { return m->rewind_to_mark(); }

extern "C" int dwim_model_add_sequence(dwim_model *m, size_t *id) { return m->add_sequence(id); }

extern "C" int dwim_model_select_sequence(dwim_model *m, size_t id) { return m->select_sequence(id); }

extern "C" int dwim_model_save(dwim_model *m, size_t len, uint8_t *out, size_t cap, size_t *bytes) {
    return m->save(len, out, cap, bytes);
}

extern "C" int dwim_model_restore(dwim_model *m, const uint8_t *state, size_t bytes, size_t *len) {
    return m->restore(state, bytes, len);
}
