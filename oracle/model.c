/*
 * Oracle restatement of the mivi-model decode step and the mivi-kv cache
 * (TEST INFRASTRUCTURE ONLY).
 *
 * Follows crates/mivi-model/src/{gguf,loader,model,ssm,transformer,ffn}.rs and
 * crates/mivi-kv/src/cache.rs. The GGUF image is borrowed, like the
 * reference's mmap (weights.rs:22-32).
 */
#include "oracle.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* GGUF parsing: gguf.rs:106-197, value types gguf.rs:264-310 */

typedef struct {
    char name[128];
    size_t dims[4];
    uint32_t n_dims;
    int32_t type;
    uint64_t offset;
} gg_tensor;

typedef struct {
    const uint8_t* p;
    size_t len, pos;
    int fail;
} cur_t;

static uint64_t rd_u(cur_t* c, int n) {
    if (c->pos + (size_t)n > c->len) { c->fail = 1; return 0; }
    uint64_t v = 0;
    for (int i = 0; i < n; i++) v |= (uint64_t)c->p[c->pos + i] << (8 * i);
    c->pos += (size_t)n;
    return v;
}

/* metadata values we keep: numeric as double + "is numeric/usize" flag */
typedef struct {
    char key[96];
    int kind;          /* 0 none, 1 usize-able, 2 f32-able, 3 array */
    uint64_t u;
    double f;
    size_t arr_len;    /* number of string elements for arrays of strings */
    size_t arr_max_pos;/* max positive usize element of a numeric array */
    int arr_numeric;
    int is_u32;
} gg_meta;

typedef struct {
    size_t data_offset;
    gg_meta* meta;
    size_t n_meta;
    gg_tensor* tens;
    size_t n_tens;
} gguf_t;

static int skip_value(cur_t* c, uint32_t t, gg_meta* m, int top);

static int read_str(cur_t* c, char* dst, size_t cap) {
    uint64_t n = rd_u(c, 8);
    if (c->fail || n > 1024 * 1024 || c->pos + n > c->len) { c->fail = 1; return 0; }
    if (dst) {
        size_t k = n < cap - 1 ? (size_t)n : cap - 1;
        memcpy(dst, c->p + c->pos, k);
        dst[k] = 0;
    }
    c->pos += (size_t)n;
    return 1;
}

/* Reads one value of type t; fills m (if top-level) with the numeric view
 * that GgufValue::as_usize / as_f32 would give (gguf.rs:59-84). */
static int skip_value(cur_t* c, uint32_t t, gg_meta* m, int top) {
    switch (t) {
    case 0: case 1: case 2: case 3: case 4: case 5: case 10: case 11: {
        int sz = (t == 0 || t == 1) ? 1 : (t == 2 || t == 3) ? 2 : (t == 4 || t == 5) ? 4 : 8;
        uint64_t v = rd_u(c, sz);
        int is_signed = (t == 1 || t == 3 || t == 5 || t == 11);
        int64_t sv = 0;
        if (is_signed) {
            sv = (int64_t)(v << (64 - 8 * sz)) >> (64 - 8 * sz);
        }
        if (m) {
            if (top) { m->is_u32 = (t == 4); }
            if (!is_signed || sv >= 0) {
                uint64_t uv = is_signed ? (uint64_t)sv : v;
                if (top) { m->kind = 1; m->u = uv; }
                else if (uv > 0 && uv > m->arr_max_pos) m->arr_max_pos = uv;
                if (!top) m->arr_numeric = 1;
            }
        }
        return !c->fail;
    }
    case 6: {
        uint32_t v = (uint32_t)rd_u(c, 4);
        float f;
        memcpy(&f, &v, 4);
        if (m && top) { m->kind = 2; m->f = f; }
        return !c->fail;
    }
    case 12: {
        uint64_t v = rd_u(c, 8);
        double f;
        memcpy(&f, &v, 8);
        if (m && top) { m->kind = 2; m->f = (double)(float)f; }
        return !c->fail;
    }
    case 7: rd_u(c, 1); return !c->fail;
    case 8:
        if (m && !top) m->arr_len++;
        return read_str(c, NULL, 0);
    case 9: {
        uint32_t et = (uint32_t)rd_u(c, 4);
        uint64_t n = rd_u(c, 8);
        if (c->fail || n > 10000000ull) { c->fail = 1; return 0; }
        if (m && top) { m->kind = 3; m->arr_len = 0; m->arr_max_pos = 0; }
        for (uint64_t i = 0; i < n; i++)
            if (!skip_value(c, et, top ? m : NULL, 0)) return 0;
        return 1;
    }
    default: c->fail = 1; return 0;
    }
}

static int gguf_parse(const uint8_t* p, size_t len, gguf_t* g, char* eb, size_t el) {
    memset(g, 0, sizeof(*g));
    cur_t c = {p, len, 0, 0};
    if (len < 16) { snprintf(eb, el, "file too small"); return 1; }
    uint32_t magic = (uint32_t)rd_u(&c, 4);
    if (magic != 0x46554747u) { snprintf(eb, el, "invalid magic 0x%X", magic); return 1; }
    uint32_t ver = (uint32_t)rd_u(&c, 4);
    if (ver != 2 && ver != 3) { snprintf(eb, el, "unsupported version %u", ver); return 1; }
    uint64_t nt = rd_u(&c, 8), nm = rd_u(&c, 8);
    if (nt > 50000 || nm > 100000) { snprintf(eb, el, "counts exceed limits"); return 1; }
    g->meta = (gg_meta*)calloc(nm ? nm : 1, sizeof(gg_meta));
    g->tens = (gg_tensor*)calloc(nt ? nt : 1, sizeof(gg_tensor));
    for (uint64_t i = 0; i < nm; i++) {
        gg_meta* m = &g->meta[g->n_meta++];
        if (!read_str(&c, m->key, sizeof(m->key))) break;
        uint32_t t = (uint32_t)rd_u(&c, 4);
        if (!skip_value(&c, t, m, 1)) break;
    }
    for (uint64_t i = 0; i < nt && !c.fail; i++) {
        gg_tensor* t = &g->tens[g->n_tens++];
        read_str(&c, t->name, sizeof(t->name));
        t->n_dims = (uint32_t)rd_u(&c, 4);
        for (uint32_t d = 0; d < t->n_dims; d++) {
            uint64_t v = rd_u(&c, 8);
            if (d < 4) t->dims[d] = (size_t)v;
        }
        t->type = (int32_t)rd_u(&c, 4);
        t->offset = rd_u(&c, 8);
    }
    if (c.fail) { snprintf(eb, el, "malformed gguf"); return 1; }
    size_t align = 32;
    for (size_t i = 0; i < g->n_meta; i++)
        if (!strcmp(g->meta[i].key, "general.alignment") && g->meta[i].is_u32) align = (size_t)g->meta[i].u;
    g->data_offset = (c.pos + align - 1) & ~(align - 1);
    return 0;
}

static const gg_meta* meta_get(const gguf_t* g, const char* k) {
    for (size_t i = 0; i < g->n_meta; i++)
        if (!strcmp(g->meta[i].key, k)) return &g->meta[i];
    return NULL;
}
static const gg_tensor* tensor_get(const gguf_t* g, const char* n) {
    for (size_t i = 0; i < g->n_tens; i++)
        if (!strcmp(g->tens[i].name, n)) return &g->tens[i];
    return NULL;
}

/* gguf.rs:200-253 */
static int tensor_data(const gguf_t* g, size_t len, const gg_tensor* t, size_t* off, size_t* nbytes) {
    size_t bs, ts, n = 1;
    if (!or_block_size(t->type, &bs) || !or_type_size(t->type, &ts)) return 1;
    for (uint32_t d = 0; d < t->n_dims && d < 4; d++) n *= t->dims[d];
    size_t blocks = (n + bs - 1) / bs;
    size_t start = g->data_offset + (size_t)t->offset;
    size_t bl = blocks * ts;
    if (start + bl > len) return 1;
    *off = start;
    *nbytes = bl;
    return 0;
}

/* ------------------------------------------------------------------ */

typedef struct {
    int32_t type;
    size_t offset, len;
} qt_t; /* weights.rs:6-13 */

typedef struct {
    float* norm;
    qt_t gate, up, down;
} ffn_w;

typedef struct {
    int is_attn;
    float* norm;            /* attn_norm or ssm_norm */
    float* q_norm;          /* optional */
    float* k_norm;
    size_t qk_norm_len;
    qt_t wq, wk, wv, wo;
    qt_t in_proj, out_proj;
    float* conv;
    size_t conv_len;
    ffn_w ffn;
} layer_w;

struct or_model {
    const uint8_t* img;
    size_t img_len;
    or_model_info cfg;
    qt_t embd, head;
    float* out_norm;
    layer_w* layers;
    /* RunState, arena.rs:25-62 */
    float *x, *xb, *xb2, *hb, *hb2, *q, *k, *v, *attn_out, *logits, *conv_states, *sc_in;
    /* KvCache, cache.rs:41-56 */
    int kv_prec;
    size_t* layer_map;
    void *kc, *vc;
    size_t kv_row_bytes;
    /* RopeCache */
    float *rcos, *rsin;
};

static float* load_vec(const gguf_t* g, const uint8_t* img, size_t len, const char* name, size_t* n_out) {
    const gg_tensor* t = tensor_get(g, name);
    if (!t) return NULL;
    size_t off, nb, n = 1;
    if (tensor_data(g, len, t, &off, &nb)) return NULL;
    for (uint32_t d = 0; d < t->n_dims && d < 4; d++) n *= t->dims[d];
    float* v = (float*)calloc(n ? n : 1, sizeof(float));
    if (or_dequantize_slice(t->type, img + off, nb, v, n, NULL)) { free(v); return NULL; }
    if (n_out) *n_out = n;
    return v;
}

static int load_qt(const gguf_t* g, size_t len, const char* name, qt_t* q) {
    const gg_tensor* t = tensor_get(g, name);
    if (!t) return 1;
    if (tensor_data(g, len, t, &q->offset, &q->len)) return 1;
    q->type = t->type;
    return 0;
}

static int errf(char* eb, size_t el, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    if (eb && el) vsnprintf(eb, el, fmt, ap);
    va_end(ap);
    return 1;
}

static void meta_usize(const gguf_t* g, const char* k2, const char* k1, size_t* dst) {
    const gg_meta* m = meta_get(g, k2);
    if (m && m->kind == 1) *dst = (size_t)m->u;
    m = meta_get(g, k1);
    if (m && m->kind == 1) *dst = (size_t)m->u;
}
static void meta_f32(const gguf_t* g, const char* k2, const char* k1, float* dst) {
    const gg_meta* m = meta_get(g, k2);
    if (m && m->kind == 2) *dst = (float)m->f;
    m = meta_get(g, k1);
    if (m && m->kind == 2) *dst = (float)m->f;
}

void or_model_destroy(or_model* m) {
    if (!m) return;
    if (m->layers) {
        for (size_t i = 0; i < m->cfg.n_layers; i++) {
            layer_w* L = &m->layers[i];
            free(L->norm); free(L->q_norm); free(L->k_norm); free(L->conv); free(L->ffn.norm);
        }
    }
    free(m->layers); free(m->out_norm);
    free(m->x); free(m->xb); free(m->xb2); free(m->hb); free(m->hb2); free(m->q); free(m->k);
    free(m->v); free(m->attn_out); free(m->logits); free(m->conv_states); free(m->sc_in);
    free(m->layer_map); free(m->kc); free(m->vc); free(m->rcos); free(m->rsin);
    free(m);
}

/* model.rs:105-233 with loader.rs:44-177 and :359-415 */
int or_model_create(const uint8_t* img, size_t len, size_t max_ctx, int kv_precision,
                    or_model** out, char* eb, size_t el) {
    gguf_t g;
    *out = NULL;
    if (gguf_parse(img, len, &g, eb, el)) { free(g.meta); free(g.tens); return 1; }
    or_model* m = (or_model*)calloc(1, sizeof(or_model));
    m->img = img;
    m->img_len = len;
    or_model_info* c = &m->cfg;
    /* ModelConfig::default, config.rs:123-159 */
    c->dim = 1024; c->hidden_dim = 4608; c->n_layers = 16; c->n_heads = 16; c->n_kv_heads = 8;
    c->vocab_size = 65536; c->max_seq_len = 128000; c->rope_base = 1000000.0f;
    c->rms_norm_eps = 1e-5f; c->ssm_conv_kernel = 3;
    meta_usize(&g, "lfm2.context_length", "lfm.context_length", &c->max_seq_len);
    meta_usize(&g, "lfm2.embedding_length", "lfm.embedding_length", &c->dim);
    meta_usize(&g, "lfm2.feed_forward_length", "lfm.feed_forward_length", &c->hidden_dim);
    meta_usize(&g, "lfm2.block_count", "lfm.block_count", &c->n_layers);
    meta_usize(&g, "lfm2.attention.head_count", "lfm.attention.head_count", &c->n_heads);
    const char* kvk[2] = {"lfm2.attention.head_count_kv", "lfm.attention.head_count_kv"};
    for (int i = 0; i < 2; i++) {
        const gg_meta* mm = meta_get(&g, kvk[i]);
        if (!mm) continue;
        if (mm->kind == 3) {
            if (mm->arr_max_pos > 0) c->n_kv_heads = (size_t)mm->arr_max_pos;
        } else if (mm->kind == 1) {
            c->n_kv_heads = (size_t)mm->u;
        }
    }
    meta_f32(&g, "lfm2.rope.freq_base", "lfm.rope.freq_base", &c->rope_base);
    meta_f32(&g, "lfm2.attention.layer_norm_rms_epsilon", "lfm.attention.layer_norm_rms_epsilon",
             &c->rms_norm_eps);
    meta_usize(&g, "lfm2.ssm.conv_kernel", "lfm.ssm.conv_kernel", &c->ssm_conv_kernel);
    char nm[160], nm2[160];
    for (size_t i = 0; i < c->n_layers; i++) {
        snprintf(nm, sizeof nm, "blk.%zu.ssm_conv.weight", i);
        snprintf(nm2, sizeof nm2, "blk.%zu.shortconv.conv.weight", i);
        const gg_tensor* t = tensor_get(&g, nm);
        if (!t) t = tensor_get(&g, nm2);
        if (t) {
            size_t tot = 1;
            for (uint32_t d = 0; d < t->n_dims && d < 4; d++) tot *= t->dims[d];
            if (c->dim > 0 && tot >= c->dim && tot % c->dim == 0) { c->ssm_conv_kernel = tot / c->dim; break; }
        }
    }
    const gg_meta* tok = meta_get(&g, "tokenizer.ggml.tokens");
    if (tok && tok->kind == 3 && tok->arr_len > 0) c->vocab_size = tok->arr_len;
    c->head_dim = c->n_heads ? c->dim / c->n_heads : 64;
    c->kv_dim = c->n_kv_heads * c->head_dim;
    if (!c->dim || !c->n_heads || !c->n_kv_heads || c->dim % c->n_heads || c->n_heads % c->n_kv_heads ||
        !c->n_layers) {
        errf(eb, el, "invalid config");
        goto fail;
    }
    size_t ctx_cap = max_ctx ? max_ctx : 16384;
    if (ctx_cap > 65536) ctx_cap = 65536;
    if (c->max_seq_len > ctx_cap) c->max_seq_len = ctx_cap;

    m->layers = (layer_w*)calloc(c->n_layers, sizeof(layer_w));
    size_t n_attn = 0;
    for (size_t i = 0; i < c->n_layers; i++) {
        layer_w* L = &m->layers[i];
        char a[160], b[160], d3[160];
        snprintf(a, sizeof a, "blk.%zu.ssm_in.weight", i);
        snprintf(b, sizeof b, "blk.%zu.shortconv.in_proj.weight", i);
        snprintf(d3, sizeof d3, "blk.%zu.shortconv.conv.weight", i);
        L->is_attn = !(tensor_get(&g, a) || tensor_get(&g, b) || tensor_get(&g, d3));
#define LN(s) (snprintf(nm, sizeof nm, "blk.%zu." s ".weight", i), nm)
        if (L->is_attn) {
            n_attn++;
            if (!(L->norm = load_vec(&g, img, len, LN("attn_norm"), NULL))) { errf(eb, el, "missing %s", nm); goto fail; }
            L->q_norm = load_vec(&g, img, len, LN("attn_q_norm"), &L->qk_norm_len);
            L->k_norm = load_vec(&g, img, len, LN("attn_k_norm"), NULL);
            if (load_qt(&g, len, LN("attn_q"), &L->wq) || load_qt(&g, len, LN("attn_k"), &L->wk) ||
                load_qt(&g, len, LN("attn_v"), &L->wv) || load_qt(&g, len, LN("attn_output"), &L->wo)) {
                errf(eb, el, "missing %s", nm);
                goto fail;
            }
        } else {
            L->norm = load_vec(&g, img, len, LN("ssm_norm"), NULL);
            if (!L->norm) L->norm = load_vec(&g, img, len, LN("attn_norm"), NULL);
            if (!L->norm) { errf(eb, el, "missing ssm norm layer %zu", i); goto fail; }
            if (load_qt(&g, len, LN("ssm_in"), &L->in_proj) && load_qt(&g, len, LN("shortconv.in_proj"), &L->in_proj)) {
                errf(eb, el, "missing in_proj layer %zu", i);
                goto fail;
            }
            if (load_qt(&g, len, LN("ssm_out"), &L->out_proj) && load_qt(&g, len, LN("shortconv.out_proj"), &L->out_proj)) {
                errf(eb, el, "missing out_proj layer %zu", i);
                goto fail;
            }
            L->conv = load_vec(&g, img, len, LN("ssm_conv"), &L->conv_len);
            if (!L->conv) L->conv = load_vec(&g, img, len, LN("shortconv.conv"), &L->conv_len);
        }
        if (!(L->ffn.norm = load_vec(&g, img, len, LN("ffn_norm"), NULL)) ||
            load_qt(&g, len, LN("ffn_gate"), &L->ffn.gate) || load_qt(&g, len, LN("ffn_up"), &L->ffn.up) ||
            load_qt(&g, len, LN("ffn_down"), &L->ffn.down)) {
            errf(eb, el, "missing ffn layer %zu", i);
            goto fail;
        }
#undef LN
    }
    c->n_attn_layers = (int32_t)n_attn;
    if (load_qt(&g, len, "token_embd.weight", &m->embd) && load_qt(&g, len, "model.embed_tokens.weight", &m->embd)) {
        errf(eb, el, "missing token_embd.weight");
        goto fail;
    }
    m->out_norm = load_vec(&g, img, len, "output_norm.weight", NULL);
    if (!m->out_norm) m->out_norm = load_vec(&g, img, len, "token_embd_norm.weight", NULL);
    if (!m->out_norm) m->out_norm = load_vec(&g, img, len, "token_embd_norm", NULL);
    if (load_qt(&g, len, "output.weight", &m->head) && load_qt(&g, len, "lm_head.weight", &m->head))
        m->head = m->embd;

    size_t D = c->dim, H = c->hidden_dim;
    m->x = calloc(D, 4); m->xb = calloc(D, 4); m->xb2 = calloc(D, 4);
    m->hb = calloc(H, 4); m->hb2 = calloc(H, 4); m->q = calloc(D, 4);
    m->k = calloc(c->kv_dim, 4); m->v = calloc(c->kv_dim, 4); m->attn_out = calloc(D, 4);
    m->logits = calloc(c->vocab_size, 4);
    m->conv_states = calloc(c->n_layers * D * (c->ssm_conv_kernel ? c->ssm_conv_kernel : 1), 4);
    m->sc_in = calloc(3 * D, 4);

    /* cache.rs:95-219 */
    m->kv_prec = kv_precision;
    m->layer_map = (size_t*)malloc(c->n_layers * sizeof(size_t));
    size_t ci = 0;
    for (size_t i = 0; i < c->n_layers; i++) m->layer_map[i] = m->layers[i].is_attn ? ci++ : (size_t)-1;
    if (kv_precision == OR_KV_Q8_0) m->kv_row_bytes = ((c->kv_dim + 31) / 32) * 34;
    else m->kv_row_bytes = c->kv_dim * 4;
    size_t kvb = n_attn * c->max_seq_len * m->kv_row_bytes;
    m->kc = calloc(kvb ? kvb : 1, 1);
    m->vc = calloc(kvb ? kvb : 1, 1);
    if (!m->kc || !m->vc) { errf(eb, el, "kv allocation failed"); goto fail; }

    /* model.rs:194-212 */
    int yarn = c->max_seq_len > 4096;
    float scale = (float)c->max_seq_len / 4096.0f;
    c->yarn = yarn;
    c->yarn_scale = yarn ? scale : 1.0f;
    size_t half = c->head_dim / 2;
    m->rcos = (float*)malloc(c->max_seq_len * half * 4);
    m->rsin = (float*)malloc(c->max_seq_len * half * 4);
    or_rope_table(m->rcos, m->rsin, c->head_dim, c->max_seq_len, c->rope_base, yarn ? 2 : 0, scale,
                  4096, 32.0f, 1.0f);
    free(g.meta);
    free(g.tens);
    *out = m;
    return 0;
fail:
    free(g.meta);
    free(g.tens);
    or_model_destroy(m);
    return 1;
}

void or_model_info_get(const or_model* m, or_model_info* info) { *info = m->cfg; }

void or_model_reset(or_model* m) {
    const or_model_info* c = &m->cfg;
    memset(m->x, 0, c->dim * 4); memset(m->xb, 0, c->dim * 4); memset(m->xb2, 0, c->dim * 4);
    memset(m->hb, 0, c->hidden_dim * 4); memset(m->hb2, 0, c->hidden_dim * 4);
    memset(m->q, 0, c->dim * 4); memset(m->k, 0, c->kv_dim * 4); memset(m->v, 0, c->kv_dim * 4);
    memset(m->attn_out, 0, c->dim * 4); memset(m->logits, 0, c->vocab_size * 4);
    memset(m->conv_states, 0, c->n_layers * c->dim * (c->ssm_conv_kernel ? c->ssm_conv_kernel : 1) * 4);
    memset(m->sc_in, 0, 3 * c->dim * 4);
}

const float* or_model_logits(const or_model* m) { return m->logits; }
const float* or_model_hidden(const or_model* m) { return m->x; }
size_t or_model_kv_bytes(const or_model* m) {
    return (size_t)m->cfg.n_attn_layers * m->cfg.max_seq_len * m->kv_row_bytes;
}
void* or_model_k_cache(or_model* m) { return m->kc; }
void* or_model_v_cache(or_model* m) { return m->vc; }
float* or_model_conv_states(or_model* m) { return m->conv_states; }
size_t or_model_conv_len(const or_model* m) {
    return m->cfg.n_layers * m->cfg.dim * (m->cfg.ssm_conv_kernel ? m->cfg.ssm_conv_kernel : 1);
}

/* ffn.rs:24-37 (no LoRA adapters) */
static int linear(or_model* m, float* out, size_t out_len, const qt_t* w, const float* in,
                  size_t in_len, size_t rows, size_t cols) {
    return or_quantized_matvec(out, out_len, w->type, m->img + w->offset, w->len, in, in_len, rows, cols, NULL);
}

/* ffn.rs:56-108 */
static int ffn(or_model* m, const ffn_w* w) {
    const or_model_info* c = &m->cfg;
    or_rms_norm(m->xb, m->x, w->norm, c->dim, c->rms_norm_eps);
    if (linear(m, m->hb, c->hidden_dim, &w->gate, m->xb, c->dim, c->hidden_dim, c->dim)) return 1;
    if (linear(m, m->hb2, c->hidden_dim, &w->up, m->xb, c->dim, c->hidden_dim, c->dim)) return 1;
    or_swiglu(m->hb, m->hb2, c->hidden_dim);
    if (linear(m, m->xb, c->dim, &w->down, m->hb, c->hidden_dim, c->dim, c->hidden_dim)) return 1;
    or_vec_add(m->x, m->xb, c->dim);
    return 0;
}

/* ssm.rs:51-167 */
static int ssm(or_model* m, size_t layer) {
    const or_model_info* c = &m->cfg;
    const layer_w* w = &m->layers[layer];
    size_t D = c->dim, K = c->ssm_conv_kernel;
    if (K == 0) return 0;
    or_rms_norm(m->xb, m->x, w->norm, D, c->rms_norm_eps);
    if (linear(m, m->sc_in, 3 * D, &w->in_proj, m->xb, D, 3 * D, D)) return 1;
    const float *B = m->sc_in, *C = m->sc_in + D, *X = m->sc_in + 2 * D;
    for (size_t d = 0; d < D; d++) m->xb2[d] = B[d] * X[d];
    size_t lo = layer * D * K;
    int full = w->conv && w->conv_len >= D * K;
    int shared = w->conv && w->conv_len >= K;
    float* st = m->conv_states;
    if (K == 3 && full) {
        for (size_t d = 0; d < D; d++) {
            size_t co = lo + d * 3, wo = d * 3;
            float s0 = st[co + 1], s1 = st[co + 2], s2 = m->xb2[d];
            st[co] = s0; st[co + 1] = s1; st[co + 2] = s2;
            float conv = w->conv[wo] * s0 + w->conv[wo + 1] * s1 + w->conv[wo + 2] * s2;
            m->xb2[d] = C[d] * conv;
        }
    } else {
        for (size_t d = 0; d < D; d++) {
            size_t co = lo + d * K, wo = d * K;
            float conv = 0.0f;
            for (size_t k = 0; k + 1 < K; k++) st[co + k] = st[co + k + 1];
            st[co + K - 1] = m->xb2[d];
            if (full) {
                for (size_t k = 0; k < K; k++) conv += w->conv[wo + k] * st[co + k];
            } else if (shared) {
                for (size_t k = 0; k < K; k++) conv += w->conv[k] * st[co + k];
            } else {
                float dw = 1.0f / (float)K;
                for (size_t k = 0; k < K; k++) conv += dw * st[co + k];
            }
            m->xb2[d] = C[d] * conv;
        }
    }
    if (linear(m, m->xb, D, &w->out_proj, m->xb2, D, D, D)) return 1;
    or_vec_add(m->x, m->xb, D);
    return ffn(m, &w->ffn);
}

static uint16_t f2h(float f) { return or_f32_to_f16(f); }

/* cache.rs:395-461 (F32, Q8_0); OR_KV_F16RT stores fp16-rounded values in
 * the F32 layout to model a half-precision cache (not a reference mode). */
static int kv_store(or_model* m, size_t layer, size_t pos) {
    const or_model_info* c = &m->cfg;
    if (layer >= c->n_layers || m->layer_map[layer] == (size_t)-1) return 1;
    if (pos >= c->max_seq_len) return 1;
    size_t cl = m->layer_map[layer];
    size_t off = (cl * c->max_seq_len + pos) * m->kv_row_bytes;
    if (m->kv_prec == OR_KV_Q8_0) {
        size_t nb = (c->kv_dim + 31) / 32;
        for (size_t b = 0; b < nb; b++) {
            float kb[32] = {0}, vb[32] = {0};
            size_t s = b * 32, e = s + 32 < c->kv_dim ? s + 32 : c->kv_dim;
            memcpy(kb, m->k + s, (e - s) * 4);
            memcpy(vb, m->v + s, (e - s) * 4);
            or_quantize_q8_0_block(kb, (uint8_t*)m->kc + off + b * 34);
            or_quantize_q8_0_block(vb, (uint8_t*)m->vc + off + b * 34);
        }
    } else {
        float* kd = (float*)((uint8_t*)m->kc + off);
        float* vd = (float*)((uint8_t*)m->vc + off);
        for (size_t i = 0; i < c->kv_dim; i++) {
            if (m->kv_prec == OR_KV_F16RT) {
                kd[i] = or_f16_to_f32(f2h(m->k[i]));
                vd[i] = or_f16_to_f32(f2h(m->v[i]));
            } else {
                kd[i] = m->k[i];
                vd[i] = m->v[i];
            }
        }
    }
    return 0;
}

static int g_serial_attention = 0;
void or_set_serial_attention(int on) { g_serial_attention = on != 0; }

/* transformer.rs:134-167 online-softmax step (shared by both precisions) */
static inline void online_step(float score, const float* v, float* out, size_t hd, float* rmax, float* rsum) {
    if (score > -INFINITY) {
        if (score > *rmax || *rmax == -INFINITY) {
            float alpha = *rmax == -INFINITY ? 0.0f : expf(*rmax - score);
            *rsum = *rsum * alpha + 1.0f;
            for (size_t i = 0; i < hd; i++) out[i] = out[i] * alpha + v[i];
            *rmax = score;
        } else {
            float beta = expf(score - *rmax);
            *rsum += beta;
            or_vec_fmadd(out, beta, v, hd);
        }
    }
}

/* transformer.rs:114-301 over one layer's cache rows (row stride `rb`
 * bytes, precision `prec`), positions 0..seq-1 */
static void gqa_attention_rows(const float* q, const uint8_t* kc, const uint8_t* vc, size_t rb, int prec,
                               size_t nh, size_t nkv, size_t hd, size_t seq, float* attn_out) {
    size_t hpk = nh / (nkv ? nkv : 1);
    if (hpk < 1) hpk = 1;
    float scale = 1.0f / sqrtf((float)hd);
    /* query heads are independent (each keeps its own running max, sum and
     * output, in token order), so long caches spread them over the threads
     * unless the reference's serial loop over heads (transformer.rs:128) is
     * asked for (or_set_serial_attention) */
    int nt = seq * nh >= 65536 && !g_serial_attention ? or_get_threads() : 1;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
    for (size_t h = 0; h < nh; h++) {
        float vbuf[256];
        size_t kvh = h / hpk;
        const float* qh = q + h * hd;
        float* oh = attn_out + h * hd;
        memset(oh, 0, hd * 4);
        float rmax = -INFINITY, rsum = 0.0f;
        for (size_t t = 0; t < seq; t++) {
            size_t off = t * rb;
            if (prec == OR_KV_Q8_0) {
                size_t bph = (hd + 31) / 32, kb0 = kvh * bph;
                float score = 0.0f;
                for (size_t b = 0; b < bph; b++)
                    score += or_dot_q8_0_f32(qh + b * 32, kc + off + (kb0 + b) * 34);
                score *= scale;
                for (size_t b = 0; b < bph; b++) {
                    float blk[32];
                    or_dequantize_q8_0(vc + off + (kb0 + b) * 34, blk);
                    size_t s = b * 32, e = s + 32 < hd ? s + 32 : hd;
                    memcpy(vbuf + s, blk, (e - s) * 4);
                }
                online_step(score, vbuf, oh, hd, &rmax, &rsum);
            } else {
                const float* kr = (const float*)(kc + off) + kvh * hd;
                const float* vr = (const float*)(vc + off) + kvh * hd;
                float score = or_dot_product(qh, kr, hd) * scale;
                online_step(score, vr, oh, hd, &rmax, &rsum);
            }
        }
        if (rsum > 0.0f) {
            float inv = 1.0f / rsum;
            for (size_t i = 0; i < hd; i++) oh[i] *= inv;
        }
    }
}

static void gqa_attention(or_model* m, size_t layer, size_t pos) {
    const or_model_info* c = &m->cfg;
    size_t cl = m->layer_map[layer];
    size_t base = cl * c->max_seq_len * m->kv_row_bytes;
    gqa_attention_rows(m->q, (const uint8_t*)m->kc + base, (const uint8_t*)m->vc + base, m->kv_row_bytes,
                       m->kv_prec, c->n_heads, c->n_kv_heads, c->head_dim, pos + 1, m->attn_out);
}

void or_attention(const float* q, const void* kc, const void* vc, int prec, size_t n_heads, size_t n_kv_heads,
                  size_t head_dim, size_t seq, float* out) {
    size_t kv_dim = n_kv_heads * head_dim;
    size_t rb = prec == OR_KV_Q8_0 ? ((kv_dim + 31) / 32) * 34 : kv_dim * 4;
    gqa_attention_rows(q, (const uint8_t*)kc, (const uint8_t*)vc, rb, prec, n_heads, n_kv_heads, head_dim, seq, out);
}

/* transformer.rs:304-350 with compute_qkv :55-110 */
static int attention(or_model* m, size_t layer, size_t pos) {
    const or_model_info* c = &m->cfg;
    const layer_w* w = &m->layers[layer];
    size_t D = c->dim, KV = c->kv_dim, hd = c->head_dim;
    or_rms_norm(m->xb, m->x, w->norm, D, c->rms_norm_eps);
    if (linear(m, m->q, D, &w->wq, m->xb, D, D, D)) return 1;
    if (linear(m, m->k, KV, &w->wk, m->xb, D, KV, D)) return 1;
    if (linear(m, m->v, KV, &w->wv, m->xb, D, KV, D)) return 1;
    if (w->q_norm)
        for (size_t h = 0; h < c->n_heads; h++) or_rms_norm_in_place(m->q + h * hd, w->q_norm, hd, c->rms_norm_eps);
    if (w->k_norm)
        for (size_t h = 0; h < c->n_kv_heads; h++) or_rms_norm_in_place(m->k + h * hd, w->k_norm, hd, c->rms_norm_eps);
    if (pos >= c->max_seq_len) return 1;
    size_t half = hd / 2;
    or_rope_rotate(m->q, c->n_heads, hd, m->rcos + pos * half, m->rsin + pos * half);
    or_rope_rotate(m->k, c->n_kv_heads, hd, m->rcos + pos * half, m->rsin + pos * half);
    if (kv_store(m, layer, pos)) return 1;
    gqa_attention(m, layer, pos);
    if (linear(m, m->xb, D, &w->wo, m->attn_out, D, D, D)) return 1;
    or_vec_add(m->x, m->xb, D);
    return ffn(m, &w->ffn);
}

/* model.rs:336-485 */
int or_model_forward_step(or_model* m, uint32_t token, size_t pos, int compute_logits) {
    const or_model_info* c = &m->cfg;
    if ((size_t)token >= c->vocab_size) return 10;     /* InvalidToken */
    if (pos >= c->max_seq_len) return 11;               /* ContextOverflow */
    size_t ts = 4, bs = 1;
    or_type_size(m->embd.type, &ts);
    or_block_size(m->embd.type, &bs);
    size_t rb = (c->dim * ts) / bs;
    size_t ro = m->embd.offset + (size_t)token * rb;
    if (ro + rb > m->img_len) return 10;
    if (or_dequantize_slice(m->embd.type, m->img + ro, rb, m->x, c->dim, NULL)) return 12;
    for (size_t l = 0; l < c->n_layers; l++) {
        int rc = m->layers[l].is_attn ? attention(m, l, pos) : ssm(m, l);
        if (rc) return 13;
    }
    if (!compute_logits) return 0;
    if (m->out_norm) or_rms_norm(m->xb, m->x, m->out_norm, c->dim, c->rms_norm_eps);
    else memcpy(m->xb, m->x, c->dim * 4);
    if (linear(m, m->logits, c->vocab_size, &m->head, m->xb, c->dim, c->vocab_size, c->dim)) return 14;
    return 0;
}
