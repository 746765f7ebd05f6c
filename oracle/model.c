/*
 * Oracle: the qwen35 forward pass (dwim inference/qwen35/mod.rs) over the
 * oracle's CPU operations, for the same random-initialised model the product
 * builds (dwim_model_synthetic): every tensor drawn from its own stream, keyed
 * by the model seed and the tensor's name, quantized by the oracle's own
 * quantizers.  TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Restated from qwen35/mod.rs: forward_batch :425-496 (verify = false),
 * Pass::layer :541-655, Pass::drafter :663-698, State::carry_over
 * :1466-1473, rope_table :1504-1515, LanguageModel::forward :1021-1038,
 * draft :1045-1071, verify :1073-1091, rewind :1099-1169, mark and
 * rewind_to_mark :1176-1228, reset :1230-1246.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* ---- the synthetic value streams (restated from the product's generator
 * definition: SplitMix64 at position i of a stream; the centred sum of the
 * hash's four 16-bit fields times sigma·sqrt(3)/65536) ---- */
static uint64_t splitmix(uint64_t seed, uint64_t i) {
    uint64_t z = seed + (i + 1) * 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

void or_synthetic_values(uint64_t seed, uint64_t first, size_t n, float sigma, float *out) {
    float c = sigma * (1.7320508075688772f / 65536.0f);
    for (size_t k = 0; k < n; k++) {
        uint64_t h = splitmix(seed, first + k);
        int32_t s = (int32_t)(h & 0xffff) + (int32_t)((h >> 16) & 0xffff) + (int32_t)((h >> 32) & 0xffff) +
                    (int32_t)(h >> 48);
        out[k] = (float)(s - 131070) * c;
    }
}

static uint64_t fnv1a(const char *s) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (; *s; s++) {
        h ^= (unsigned char)*s;
        h *= 0x100000001b3ull;
    }
    return h;
}

static uint64_t tensor_seed(uint64_t model_seed, const char *name) { return splitmix(model_seed, fnv1a(name)); }

/* ---- the model ---- */
typedef struct {
    or_weight w;
    void *quants;
    uint16_t *scales;
} owned_weight;

typedef struct {
    int attention;
    float *attn_norm, *mlp_norm;
    owned_weight gate, up, down;
    owned_weight q, qgate, k, v, o;
    float *q_norm, *k_norm;
    size_t cache;
    owned_weight qkv, z, ab, out;
    float *conv, *decay, *norm;
    size_t slot;
} layer_t;

struct or_model {
    or_qwen35_config c;
    uint64_t seed;
    layer_t *layers;
    float *norm;
    owned_weight head, embd;
    int has_draft;
    float *enorm, *hnorm, *dnorm;
    owned_weight eproj, hproj;
    layer_t dlayer;
    size_t most, caches, slots, max_len;
    /* buffers, sized for `most` tokens */
    float *x, *xb, *xh, *q, *gate, *k, *v, *att, *qkv, *z, *ab, *up, *gate_ffn, *logits, *rope, *drafted;
    /* the sequence */
    int8_t **kq, **vq;
    uint16_t **ks, **vs;
    float **conv_state[2];
    float **ssm_state;
    int parity;
    float *hidden;
    int carry;
    /* a batch being verified: its tokens, where it started, and the linear
     * layers' inputs and states run through it apart from the real ones */
    uint32_t verified[OR_MAX_DRAFTS + 1];
    size_t n_verified, verified_at;
    float **ssm_scratch, **qkv_saved, **ab_saved;
    /* the mark */
    float **mark_conv, **mark_ssm, *mark_hidden;
    int marked, mark_carry;
};

static float *vec(struct or_model *m, const char *name, size_t len, float sigma, float offset) {
    float *v = malloc(len * sizeof(float));
    or_synthetic_values(tensor_seed(m->seed, name), 0, len, sigma, v);
    for (size_t i = 0; i < len; i++) v[i] = v[i] + offset;
    return v;
}

static float *uniform_vec(struct or_model *m, const char *name, size_t len, float scale, float offset) {
    float *v = malloc(len * sizeof(float));
    uint64_t s = tensor_seed(m->seed, name);
    for (size_t i = 0; i < len; i++) {
        float u = (float)(splitmix(s, i) >> 40) * (1.0f / 16777216.0f);
        v[i] = u * scale + offset;
    }
    return v;
}

static owned_weight mat(struct or_model *m, const char *name, int fmt, size_t rows, size_t cols, float sigma) {
    owned_weight o;
    memset(&o, 0, sizeof o);
    o.w.fmt = fmt;
    o.w.rows = rows;
    o.w.cols = cols;
    uint64_t s = tensor_seed(m->seed, name);
    if (fmt == OR_BF16) o.quants = malloc(rows * cols * 2);
    else if (fmt == OR_Q4_K || fmt == OR_Q6_K) o.quants = malloc(rows * (cols / 256) * (fmt == OR_Q4_K ? 144 : 210));
    else if (fmt == OR_Q4_0 || fmt == OR_Q8_0) {
        o.scales = malloc(rows * (cols / 32) * 2);
        o.quants = malloc(fmt == OR_Q4_0 ? rows * cols / 2 : rows * cols);
    }
    /* rows are independent streams of values: generated and quantized in parallel */
#pragma omp parallel
    {
        float *row = malloc(cols * sizeof(float));
#pragma omp for schedule(static)
        for (size_t r = 0; r < rows; r++) {
            or_synthetic_values(s, r * cols, cols, sigma, row);
            switch (fmt) {
            case OR_BF16:
                for (size_t i = 0; i < cols; i++) ((uint16_t *)o.quants)[r * cols + i] = or_to_bf16(row[i]);
                break;
            case OR_Q4_K: or_quantize_q4_k_row(row, cols, (uint8_t *)o.quants + r * (cols / 256) * 144); break;
            case OR_Q6_K: or_quantize_q6_k_row(row, cols, (uint8_t *)o.quants + r * (cols / 256) * 210); break;
            case OR_Q4_0:
                or_quantize_q4_0_row(row, cols, o.scales + r * (cols / 32), (uint8_t *)o.quants + r * cols / 2);
                break;
            case OR_Q8_0:
                or_quantize_q8_0_row(row, cols, o.scales + r * (cols / 32), (int8_t *)o.quants + r * cols);
                break;
            }
        }
        free(row);
    }
    o.w.quants = o.quants;
    o.w.scales = o.scales;
    return o;
}

static void free_weight(owned_weight *o) {
    free(o->quants);
    free(o->scales);
}

static size_t q_dim(struct or_model *m) { return m->c.heads * m->c.head_dim; }
static size_t kv_dim(struct or_model *m) { return m->c.kv_heads * m->c.head_dim; }
static size_t k_dim(struct or_model *m) { return m->c.k_heads * m->c.state_dim; }
static size_t v_dim(struct or_model *m) { return m->c.v_heads * m->c.state_dim; }
static size_t conv_width(struct or_model *m) { return 3 * (2 * k_dim(m) + v_dim(m)); }
static size_t ssm_width(struct or_model *m) { return m->c.v_heads * m->c.state_dim * m->c.state_dim; }

static void load_layer(struct or_model *m, size_t i, int attention, int fmt, layer_t *l) {
    char p[64], n[128];
    snprintf(p, sizeof p, "blk.%zu.", i);
    size_t H = m->c.hidden;
    float s = 0.02f;
    memset(l, 0, sizeof *l);
    l->attention = attention;
#define NAME(x) (snprintf(n, sizeof n, "%s%s", p, x), n)
    l->attn_norm = vec(m, NAME("attn_norm"), H, 0.1f, 1.0f);
    if (attention) {
        l->q = mat(m, NAME("attn_q"), fmt, q_dim(m), H, s);
        l->qgate = mat(m, NAME("attn_q_gate"), fmt, q_dim(m), H, s);
        l->k = mat(m, NAME("attn_k"), fmt, kv_dim(m), H, s);
        l->v = mat(m, NAME("attn_v"), fmt, kv_dim(m), H, s);
        l->o = mat(m, NAME("attn_output"), fmt, H, q_dim(m), s);
        l->q_norm = vec(m, NAME("attn_q_norm"), m->c.head_dim, 0.1f, 1.0f);
        l->k_norm = vec(m, NAME("attn_k_norm"), m->c.head_dim, 0.1f, 1.0f);
        l->cache = m->caches++;
    } else {
        l->qkv = mat(m, NAME("attn_qkv"), fmt, 2 * k_dim(m) + v_dim(m), H, s);
        l->z = mat(m, NAME("attn_gate"), fmt, v_dim(m), H, s);
        l->ab = mat(m, NAME("ssm_ab"), OR_BF16, 2 * m->c.v_heads, H, s);
        l->conv = vec(m, NAME("ssm_conv1d"), (2 * k_dim(m) + v_dim(m)) * 4, 0.3f, 0.0f);
        float *a = uniform_vec(m, NAME("ssm_a"), m->c.v_heads, -0.9f, -0.1f);
        float *dt = uniform_vec(m, NAME("ssm_dt.bias"), m->c.v_heads, 8.0f, -4.0f);
        l->decay = malloc(2 * m->c.v_heads * sizeof(float));
        memcpy(l->decay, a, m->c.v_heads * sizeof(float));
        memcpy(l->decay + m->c.v_heads, dt, m->c.v_heads * sizeof(float));
        free(a);
        free(dt);
        l->norm = vec(m, NAME("ssm_norm"), m->c.state_dim, 0.1f, 1.0f);
        l->out = mat(m, NAME("ssm_out"), fmt, H, v_dim(m), s);
        l->slot = m->slots++;
    }
    l->mlp_norm = vec(m, NAME("post_attention_norm"), H, 0.1f, 1.0f);
    l->gate = mat(m, NAME("ffn_gate"), fmt, m->c.intermediate, H, s);
    l->up = mat(m, NAME("ffn_up"), fmt, m->c.intermediate, H, s);
    l->down = mat(m, NAME("ffn_down"), fmt, H, m->c.intermediate, s);
#undef NAME
}

static void free_layer(layer_t *l) {
    free(l->attn_norm);
    free(l->mlp_norm);
    free_weight(&l->gate);
    free_weight(&l->up);
    free_weight(&l->down);
    if (l->attention) {
        free_weight(&l->q); free_weight(&l->qgate); free_weight(&l->k); free_weight(&l->v); free_weight(&l->o);
        free(l->q_norm);
        free(l->k_norm);
    } else {
        free_weight(&l->qkv); free_weight(&l->z); free_weight(&l->ab); free_weight(&l->out);
        free(l->conv); free(l->decay); free(l->norm);
    }
}

or_model *or_model_synthetic(const or_qwen35_config *cfg, uint64_t seed, int body_fmt, int head_fmt, size_t max_len,
                             size_t batch) {
    struct or_model *m = calloc(1, sizeof *m);
    m->c = *cfg;
    m->seed = seed;
    m->most = batch;
    m->max_len = max_len;
    const or_qwen35_config *c = &m->c;
    m->layers = calloc(c->layers, sizeof(layer_t));
    for (size_t i = 0; i < c->layers; i++)
        load_layer(m, i, (i + 1) % c->full_attention_interval == 0, body_fmt, &m->layers[i]);
    m->norm = vec(m, "output_norm", c->hidden, 0.1f, 1.0f);
    m->head = mat(m, "output", head_fmt, c->vocab, c->hidden, 0.02f);
    m->embd = mat(m, "token_embd", body_fmt, c->vocab, c->hidden, 1.0f);
    if (c->drafter) {
        char p[64], n[128];
        snprintf(p, sizeof p, "blk.%zu.", c->layers);
        m->has_draft = 1;
#define NAME(x) (snprintf(n, sizeof n, "%s%s", p, x), n)
        m->enorm = vec(m, NAME("enorm"), c->hidden, 0.1f, 1.0f);
        m->hnorm = vec(m, NAME("hnorm"), c->hidden, 0.1f, 1.0f);
        m->eproj = mat(m, NAME("eh_proj.embed"), body_fmt, c->hidden, c->hidden, 0.02f);
        m->hproj = mat(m, NAME("eh_proj.hidden"), body_fmt, c->hidden, c->hidden, 0.02f);
        load_layer(m, c->layers, 1, body_fmt, &m->dlayer);
        m->dnorm = vec(m, NAME("shared_head_norm"), c->hidden, 0.1f, 1.0f);
#undef NAME
    }
    size_t most = m->most, H = c->hidden;
    size_t qd = q_dim(m), kvd = kv_dim(m), kd = k_dim(m), vd = v_dim(m);
#define MAX(a, b) ((a) > (b) ? (a) : (b))
    m->x = calloc(most * H, 4);
    m->xb = calloc(most * H, 4);
    m->xh = calloc(most * H, 4);
    m->q = calloc(most * MAX(qd, kd), 4);
    m->gate = calloc(most * qd, 4);
    m->k = calloc(most * MAX(kvd, kd), 4);
    m->v = calloc(most * MAX(kvd, vd), 4);
    m->att = calloc(most * MAX(qd, vd), 4);
    m->qkv = calloc(most * (2 * kd + vd), 4);
    m->z = calloc(most * vd, 4);
    m->ab = calloc(most * 2 * c->v_heads, 4);
    m->up = calloc(most * c->intermediate, 4);
    m->gate_ffn = calloc(most * c->intermediate, 4);
    m->logits = calloc((OR_MAX_DRAFTS + 1) * c->vocab, 4);
    m->drafted = calloc(H, 4);
    m->rope = malloc(max_len * c->rot_dim * 4);
    or_rope_table(m->rope, max_len, c->rot_dim, c->rope_theta);
    m->kq = calloc(m->caches, sizeof(void *));
    m->vq = calloc(m->caches, sizeof(void *));
    m->ks = calloc(m->caches, sizeof(void *));
    m->vs = calloc(m->caches, sizeof(void *));
    for (size_t i = 0; i < m->caches; i++) {
        m->kq[i] = calloc(max_len * kvd, 1);
        m->vq[i] = calloc(max_len * kvd, 1);
        m->ks[i] = calloc(max_len * kvd / 32, 2);
        m->vs[i] = calloc(max_len * kvd / 32, 2);
    }
    for (int p = 0; p < 2; p++) {
        m->conv_state[p] = calloc(m->slots, sizeof(float *));
        for (size_t i = 0; i < m->slots; i++) m->conv_state[p][i] = calloc(conv_width(m), 4);
    }
    m->ssm_state = calloc(m->slots, sizeof(float *));
    for (size_t i = 0; i < m->slots; i++) m->ssm_state[i] = calloc(ssm_width(m), 4);
    float ***per_slot[] = {&m->ssm_scratch, &m->qkv_saved, &m->ab_saved, &m->mark_conv, &m->mark_ssm};
    size_t widths[] = {ssm_width(m), (OR_MAX_DRAFTS + 1) * (2 * kd + vd), (OR_MAX_DRAFTS + 1) * 2 * c->v_heads,
                       conv_width(m), ssm_width(m)};
    for (int j = 0; j < 5; j++) {
        *per_slot[j] = calloc(m->slots, sizeof(float *));
        for (size_t i = 0; i < m->slots; i++) (*per_slot[j])[i] = calloc(widths[j], 4);
    }
    m->mark_hidden = calloc(H, 4);
    m->hidden = calloc((most + 1) * H, 4);
#undef MAX
    return m;
}

void or_model_free(or_model *m) {
    for (size_t i = 0; i < m->c.layers; i++) free_layer(&m->layers[i]);
    free(m->layers);
    if (m->has_draft) {
        free_layer(&m->dlayer);
        free(m->enorm); free(m->hnorm); free(m->dnorm);
        free_weight(&m->eproj); free_weight(&m->hproj);
    }
    free(m->norm);
    free_weight(&m->head);
    free_weight(&m->embd);
    float *bufs[] = {m->x, m->xb, m->xh, m->q, m->gate, m->k, m->v, m->att, m->qkv, m->z, m->ab, m->up,
                     m->gate_ffn, m->logits, m->drafted, m->rope, m->hidden};
    for (size_t i = 0; i < sizeof bufs / sizeof *bufs; i++) free(bufs[i]);
    for (size_t i = 0; i < m->caches; i++) {
        free(m->kq[i]); free(m->vq[i]); free(m->ks[i]); free(m->vs[i]);
    }
    free(m->kq); free(m->vq); free(m->ks); free(m->vs);
    for (int p = 0; p < 2; p++) {
        for (size_t i = 0; i < m->slots; i++) free(m->conv_state[p][i]);
        free(m->conv_state[p]);
    }
    for (size_t i = 0; i < m->slots; i++) free(m->ssm_state[i]);
    free(m->ssm_state);
    float **per_slot[] = {m->ssm_scratch, m->qkv_saved, m->ab_saved, m->mark_conv, m->mark_ssm};
    for (int j = 0; j < 5; j++) {
        for (size_t i = 0; i < m->slots; i++) free(per_slot[j][i]);
        free(per_slot[j]);
    }
    free(m->mark_hidden);
    free(m);
}

/* dequantized row r of a weight (the host lookup of qwen35 Pass::embed) */
static void weight_row(const or_weight *w, size_t r, float *out) {
    size_t cols = w->cols;
    switch (w->fmt) {
    case OR_BF16:
        for (size_t i = 0; i < cols; i++) out[i] = or_bf16(((const uint16_t *)w->quants)[r * cols + i]);
        break;
    case OR_Q4_0:
        or_dequantize_q4_0_row(w->scales + r * (cols / 32), (const uint8_t *)w->quants + r * cols / 2, cols, out);
        break;
    case OR_Q8_0:
        or_dequantize_q8_0_row(w->scales + r * (cols / 32), (const int8_t *)w->quants + r * cols, cols, out);
        break;
    case OR_Q4_K: or_dequantize_q4_k_row((const uint8_t *)w->quants + r * (cols / 256) * 144, cols, out); break;
    case OR_Q6_K: or_dequantize_q6_k_file((const uint8_t *)w->quants + r * (cols / 256) * 210, cols, out); break;
    }
}

static void embed(struct or_model *m, float *out, const uint32_t *tokens, size_t n) {
    for (size_t t = 0; t < n; t++) weight_row(&m->embd.w, tokens[t], out + t * m->c.hidden);
}

/* Device::normalize's default (gpu/mod.rs:295-305): copy then rmsnorm */
static void normalize(struct or_model *m, float *out, const float *x, const float *w, size_t rows) {
    size_t len = rows * m->c.hidden;
    memcpy(out, x, len * 4);
    or_rmsnorm(out, len, w, m->c.hidden, m->c.eps);
}

static void matmul_add(float *x, const or_weight *w, const float *in, size_t n, float *scratch) {
    or_matmul(scratch, w, in, n);
    or_add(x, scratch, n * w->rows);
}

static void layer(struct or_model *m, const layer_t *l, size_t n, size_t pos, int verify) {
    const or_qwen35_config *c = &m->c;
    float eps = c->eps;
    size_t H = c->hidden;
    normalize(m, m->xh, m->x, l->attn_norm, n);
    if (l->attention) {
        size_t qd = q_dim(m), kvd = kv_dim(m);
        or_matmul(m->q, &l->q.w, m->xh, n);
        or_matmul(m->gate, &l->qgate.w, m->xh, n);
        or_matmul(m->k, &l->k.w, m->xh, n);
        or_matmul(m->v, &l->v.w, m->xh, n);
        or_rmsnorm(m->q, n * qd, l->q_norm, c->head_dim, eps);
        or_rmsnorm(m->k, n * kvd, l->k_norm, c->head_dim, eps);
        or_rope(m->q, n * qd, m->rope, pos, c->heads, c->head_dim, c->rot_dim);
        or_rope(m->k, n * kvd, m->rope, pos, c->kv_heads, c->head_dim, c->rot_dim);
        or_store(m->kq[l->cache], m->ks[l->cache], pos * kvd, m->k, n * kvd);
        or_store(m->vq[l->cache], m->vs[l->cache], pos * kvd, m->v, n * kvd);
        or_attention(m->att, m->q, n, m->kq[l->cache], m->ks[l->cache], m->vq[l->cache], m->vs[l->cache], pos,
                     c->heads, c->head_dim, c->kv_heads);
        or_sigmoid_mul(m->att, m->gate, n * qd);
        matmul_add(m->x, &l->o.w, m->att, n, m->xb);
    } else {
        size_t kd = k_dim(m), vd = v_dim(m);
        or_matmul(m->qkv, &l->qkv.w, m->xh, n);
        or_matmul(m->z, &l->z.w, m->xh, n);
        or_matmul(m->ab, &l->ab.w, m->xh, n);
        if (verify) {
            memcpy(m->qkv_saved[l->slot], m->qkv, n * (2 * kd + vd) * 4);
            memcpy(m->ab_saved[l->slot], m->ab, n * 2 * c->v_heads * 4);
            memcpy(m->ssm_scratch[l->slot], m->ssm_state[l->slot], ssm_width(m) * 4);
        }
        float *state = m->parity ? m->conv_state[0][l->slot] : m->conv_state[1][l->slot];
        float *state_out = m->parity ? m->conv_state[1][l->slot] : m->conv_state[0][l->slot];
        or_conv(m->q, kd, m->k, kd, m->v, vd, state_out, m->qkv, n, state, l->conv);
        or_l2norm(m->q, n * kd, c->state_dim, eps);
        or_l2norm(m->k, n * kd, c->state_dim, eps);
        or_delta_net(m->att, m->q, m->k, m->v, m->ab, l->decay,
                     verify ? m->ssm_scratch[l->slot] : m->ssm_state[l->slot], n, c->k_heads, c->v_heads,
                     c->state_dim);
        or_rmsnorm(m->att, n * vd, l->norm, c->state_dim, eps);
        or_silu_mul(m->z, m->att, n * vd);
        matmul_add(m->x, &l->out.w, m->z, n, m->xb);
    }
    normalize(m, m->xh, m->x, l->mlp_norm, n);
    or_matmul(m->up, &l->gate.w, m->xh, n);
    or_matmul(m->gate_ffn, &l->up.w, m->xh, n);
    or_silu_mul(m->up, m->gate_ffn, n * c->intermediate);
    matmul_add(m->x, &l->down.w, m->up, n, m->xb);
    (void)H;
}

static void drafter(struct or_model *m, size_t rows, size_t pos, size_t first, int chain, const uint32_t *tokens) {
    const or_qwen35_config *c = &m->c;
    size_t H = c->hidden;
    if (rows == 0) return;
    embed(m, m->xb, tokens, rows);
    or_rmsnorm(m->xb, rows * H, m->enorm, H, c->eps);
    if (chain) memcpy(m->xh, m->drafted, H * 4);
    else memcpy(m->xh, m->hidden + first * H, rows * H * 4);
    or_rmsnorm(m->xh, rows * H, m->hnorm, H, c->eps);
    or_matmul(m->x, &m->eproj.w, m->xb, rows);
    or_matmul(m->xb, &m->hproj.w, m->xh, rows);
    or_add(m->x, m->xb, rows * H);
    layer(m, &m->dlayer, rows, pos, 0);
    normalize(m, m->xh, m->x, m->dnorm, rows);
}

static void carry_over(struct or_model *m, size_t n) {
    size_t H = m->c.hidden;
    memcpy(m->xb, m->hidden + n * H, H * 4);
    memcpy(m->hidden, m->xb, H * 4);
    m->carry = 1;
}

/* returns 1 when logits were computed; verifying, the logits of every token */
static int forward_batch(struct or_model *m, const uint32_t *tokens, size_t n, size_t pos, int verify, int wanted) {
    const or_qwen35_config *c = &m->c;
    size_t H = c->hidden;
    embed(m, m->x, tokens, n);
    for (size_t i = 0; i < c->layers; i++) layer(m, &m->layers[i], n, pos, verify);
    if (!verify) m->parity = !m->parity;
    if (!m->has_draft) {
        if (!wanted) return 0;
        memcpy(m->xb, m->x + (n - 1) * H, H * 4);
        normalize(m, m->xh, m->xb, m->norm, 1);
        or_matmul(m->logits, &m->head.w, m->xh, 1);
        return 1;
    }
    normalize(m, m->xh, m->x, m->norm, n);
    memcpy(m->hidden + H, m->xh, n * H * 4);
    if (verify) {
        memcpy(m->verified, tokens, n * sizeof *tokens);
        m->n_verified = n;
        m->verified_at = pos;
        or_matmul(m->logits, &m->head.w, m->xh, n);
        return 1;
    }
    if (wanted) {
        memcpy(m->xb, m->xh + (n - 1) * H, H * 4);
        or_matmul(m->logits, &m->head.w, m->xb, 1);
    }
    size_t first = m->carry ? 0 : 1;
    drafter(m, n - first, pos + first - 1, first, 0, tokens + first);
    carry_over(m, n);
    return wanted;
}

void or_model_forward(or_model *m, const uint32_t *tokens, size_t n, size_t pos, float *logits) {
    size_t batches = (n + m->most - 1) / m->most;
    for (size_t i = 0; i < batches; i++) {
        size_t k = n - i * m->most < m->most ? n - i * m->most : m->most;
        forward_batch(m, tokens + i * m->most, k, pos + i * m->most, 0, i + 1 == batches);
    }
    if (logits) memcpy(logits, m->logits, m->c.vocab * 4);
}

/* LanguageModel::draft (qwen35/mod.rs:1045-1071) */
size_t or_model_draft(or_model *m, uint32_t token, size_t pos, size_t k, uint32_t *drafts) {
    if (!m->has_draft || !m->carry || m->n_verified || pos == 0) return 0;
    if (k > OR_MAX_DRAFTS) k = OR_MAX_DRAFTS;
    if (pos + 1 + k > m->max_len) k = m->max_len > pos + 1 ? m->max_len - pos - 1 : 0;
    uint32_t next = token;
    for (size_t i = 0; i < k; i++) {
        drafter(m, 1, pos - 1 + i, 0, i > 0, &next);
        memcpy(m->drafted, m->xh, m->c.hidden * 4);
        or_matmul(m->logits, &m->head.w, m->xh, 1);
        next = or_argmax(m->logits, m->c.vocab);
        drafts[i] = next;
    }
    return k;
}

/* Test hook: the logits of the last single-token head product (after a
 * draft, those of its last draft: qwen35/mod.rs:1064-1066). */
void or_model_last_logits(const or_model *m, float *out) { memcpy(out, m->logits, m->c.vocab * 4); }

/* LanguageModel::verify (qwen35/mod.rs:1073-1091): logits [n][vocab] */
void or_model_verify(or_model *m, const uint32_t *tokens, size_t n, size_t pos, float *logits) {
    forward_batch(m, tokens, n, pos, 1, 1);
    memcpy(logits, m->logits, n * m->c.vocab * 4);
}

/* LanguageModel::rewind (qwen35/mod.rs:1099-1169) */
void or_model_rewind(or_model *m, size_t keep) {
    const or_qwen35_config *c = &m->c;
    size_t n = m->n_verified, kd = k_dim(m), vd = v_dim(m);
    uint32_t tokens[OR_MAX_DRAFTS + 1];
    memcpy(tokens, m->verified, n * sizeof *tokens);
    m->n_verified = 0;
    if (keep == n) {
        for (size_t i = 0; i < m->slots; i++) {
            float *t = m->ssm_state[i];
            m->ssm_state[i] = m->ssm_scratch[i];
            m->ssm_scratch[i] = t;
        }
    } else {
        for (size_t li = 0; li < c->layers; li++) {
            const layer_t *l = &m->layers[li];
            if (l->attention) continue;
            memcpy(m->qkv, m->qkv_saved[l->slot], keep * (2 * kd + vd) * 4);
            memcpy(m->ab, m->ab_saved[l->slot], keep * 2 * c->v_heads * 4);
            float *state = m->parity ? m->conv_state[0][l->slot] : m->conv_state[1][l->slot];
            float *state_out = m->parity ? m->conv_state[1][l->slot] : m->conv_state[0][l->slot];
            or_conv(m->q, kd, m->k, kd, m->v, vd, state_out, m->qkv, keep, state, l->conv);
            or_l2norm(m->q, keep * kd, c->state_dim, c->eps);
            or_l2norm(m->k, keep * kd, c->state_dim, c->eps);
            or_delta_net(m->att, m->q, m->k, m->v, m->ab, l->decay, m->ssm_state[l->slot], keep, c->k_heads,
                         c->v_heads, c->state_dim);
        }
    }
    m->parity = !m->parity;
    if (m->has_draft) {
        drafter(m, keep, m->verified_at - 1, 0, 0, tokens);
        carry_over(m, keep);
    }
}

/* LanguageModel::mark and rewind_to_mark (qwen35/mod.rs:1176-1228) */
void or_model_mark(or_model *m) {
    for (size_t i = 0; i < m->slots; i++) {
        memcpy(m->mark_conv[i], m->conv_state[m->parity ? 0 : 1][i], conv_width(m) * 4);
        memcpy(m->mark_ssm[i], m->ssm_state[i], ssm_width(m) * 4);
    }
    if (m->carry) memcpy(m->mark_hidden, m->hidden, m->c.hidden * 4);
    m->mark_carry = m->carry;
    m->marked = 1;
}

int or_model_rewind_to_mark(or_model *m) {
    if (!m->marked || m->n_verified) return 1;
    for (size_t i = 0; i < m->slots; i++) {
        memcpy(m->conv_state[0][i], m->mark_conv[i], conv_width(m) * 4);
        memcpy(m->ssm_state[i], m->mark_ssm[i], ssm_width(m) * 4);
    }
    m->parity = 1;
    if (m->mark_carry) memcpy(m->hidden, m->mark_hidden, m->c.hidden * 4);
    m->carry = m->mark_carry;
    return 0;
}

void or_model_reset(or_model *m) {
    for (size_t i = 0; i < m->slots; i++) {
        memset(m->conv_state[0][i], 0, conv_width(m) * 4);
        memset(m->conv_state[1][i], 0, conv_width(m) * 4);
        memset(m->ssm_state[i], 0, ssm_width(m) * 4);
    }
    m->parity = 0;
    m->carry = 0;
    m->n_verified = 0;
    m->marked = 0;
}

/* Test hook: zeroes every product that writes into the residual stream (each
 * layer's ffn_down, attn_output and ssm_out), so that the logits reduce to the
 * head applied to the normalized embedding of the last token. */
static void zero_weight(owned_weight *o) {
    const or_weight *w = &o->w;
    size_t bytes = 0;
    switch (w->fmt) {
    case OR_BF16: bytes = w->rows * w->cols * 2; break;
    case OR_Q4_K: bytes = w->rows * (w->cols / 256) * 144; break;
    case OR_Q6_K: bytes = w->rows * (w->cols / 256) * 210; break;
    case OR_Q4_0: bytes = w->rows * w->cols / 2; break;
    case OR_Q8_0: bytes = w->rows * w->cols; break;
    }
    memset(o->quants, 0, bytes);
    if (o->scales) memset(o->scales, 0, w->rows * (w->cols / 32) * 2);
}

void or_model_zero_residual_writes(or_model *m) {
    for (size_t i = 0; i < m->c.layers; i++) {
        layer_t *l = &m->layers[i];
        zero_weight(&l->down);
        zero_weight(l->attention ? &l->o : &l->out);
    }
}

/* LanguageModel::save (qwen35/mod.rs:905-947), "dwimstat" version 3.  Returns
 * the bytes written (or needed, with out null); 0 for the reference's None. */
size_t or_model_save(or_model *m, size_t len, uint8_t *out) {
    if (m->n_verified || (m->has_draft && !m->carry)) return 0;
    size_t kvd = kv_dim(m), cl = len * kvd, cb = cl + cl / 32 * 2;
    size_t need = 8 + 4 + 56 + 2 * m->caches * cb + m->slots * (conv_width(m) + ssm_width(m)) * 4 +
                  (m->has_draft ? m->c.hidden * 4 : 0);
    if (!out) return need;
    uint8_t *p = out;
    memcpy(p, "dwimstat", 8);
    p += 8;
    uint32_t version = 3;
    memcpy(p, &version, 4);
    p += 4;
    uint64_t header[7] = {len, m->caches, m->slots, kvd, conv_width(m), ssm_width(m), m->has_draft ? m->c.hidden : 0};
    memcpy(p, header, sizeof header);
    p += sizeof header;
    for (int kv = 0; kv < 2; kv++)
        for (size_t i = 0; i < m->caches; i++) {
            memcpy(p, kv ? m->vq[i] : m->kq[i], cl);
            memcpy(p + cl, kv ? m->vs[i] : m->ks[i], cl / 32 * 2);
            p += cb;
        }
    for (size_t i = 0; i < m->slots; i++) {
        memcpy(p, m->conv_state[m->parity ? 0 : 1][i], conv_width(m) * 4);
        p += conv_width(m) * 4;
        memcpy(p, m->ssm_state[i], ssm_width(m) * 4);
        p += ssm_width(m) * 4;
    }
    if (m->has_draft) {
        memcpy(p, m->hidden, m->c.hidden * 4);
        p += m->c.hidden * 4;
    }
    return (size_t)(p - out);
}

/* LanguageModel::restore (qwen35/mod.rs:949-1017): returns 0 and *len, or an
 * error code: 1 cut short, 2 not a state, 3 another version, 4 another model,
 * 5 too long for the context. */
int or_model_restore(or_model *m, const uint8_t *state, size_t bytes, size_t *len) {
    if (bytes < 8) return 1;
    if (memcmp(state, "dwimstat", 8) != 0) return 2;
    if (bytes < 12) return 1;
    uint32_t version;
    memcpy(&version, state + 8, 4);
    if (version != 3) return 3;
    if (bytes < 68) return 1;
    uint64_t header[7];
    memcpy(header, state + 12, sizeof header);
    uint64_t want[6] = {m->caches, m->slots, kv_dim(m), conv_width(m), ssm_width(m), m->has_draft ? m->c.hidden : 0};
    if (memcmp(header + 1, want, sizeof want) != 0) return 4;
    size_t n = header[0];
    if (n > m->max_len) return 5;
    size_t cl = n * kv_dim(m), cb = cl + cl / 32 * 2;
    size_t need = 68 + 2 * m->caches * cb + m->slots * (conv_width(m) + ssm_width(m)) * 4 +
                  (m->has_draft ? m->c.hidden * 4 : 0);
    if (bytes < need) return 1;
    const uint8_t *p = state + 68;
    for (int kv = 0; kv < 2; kv++)
        for (size_t i = 0; i < m->caches; i++) {
            memcpy(kv ? m->vq[i] : m->kq[i], p, cl);
            memcpy(kv ? m->vs[i] : m->ks[i], p + cl, cl / 32 * 2);
            p += cb;
        }
    for (size_t i = 0; i < m->slots; i++) {
        memcpy(m->conv_state[0][i], p, conv_width(m) * 4);
        p += conv_width(m) * 4;
        memcpy(m->ssm_state[i], p, ssm_width(m) * 4);
        p += ssm_width(m) * 4;
    }
    m->parity = 1;
    m->n_verified = 0;
    m->marked = 0;
    if (m->has_draft) {
        memcpy(m->hidden, p, m->c.hidden * 4);
        m->carry = 1;
    }
    *len = n;
    return 0;
}
