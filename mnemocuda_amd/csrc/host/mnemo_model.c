/*
 * mnemo_model.c -- the split model directory (include/mnemo_model.h): a small JSON reader,
 * config / manifest parsing with the reference's keys and defaults, validation, and the
 * upload of resident tensors and expert layers into device memory.
 *
 * The reference finds keys with strstr over the raw text (src/engine.c:331-347, 540-620,
 * 697-708), which also matches keys nested elsewhere; this reader walks the JSON structure
 * and matches whole keys at the level the format defines.
 */
#define _POSIX_C_SOURCE 200809L
#include "../../../include/mnemo_model.h"

#include <errno.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>

#include "../../../include/mnemo_host.h"
#include "mnemo_host_private.h"

static int fail(int code, const char *fmt, ...) {
    char msg[256];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(msg, sizeof msg, fmt, ap);
    va_end(ap);
    return mnemo_record_error(code, msg);
}

/* ------------------------------------------------------------------ JSON reader */
typedef struct {
    const char *p, *end;
    int err;
} Json;

static void ws(Json *j) {
    while (j->p < j->end && (*j->p == ' ' || *j->p == '\t' || *j->p == '\n' || *j->p == '\r')) j->p++;
}
static int peek(Json *j) {
    ws(j);
    return j->p < j->end ? (unsigned char)*j->p : -1;
}
static int expect(Json *j, char c) {
    if (peek(j) != (unsigned char)c) {
        j->err = 1;
        return 0;
    }
    j->p++;
    return 1;
}
static void put_utf8(char *out, size_t cap, size_t *n, unsigned cp) {
    char b[4];
    int k;
    if (cp < 0x80) { b[0] = (char)cp; k = 1; }
    else if (cp < 0x800) { b[0] = (char)(0xC0 | (cp >> 6)); b[1] = (char)(0x80 | (cp & 0x3F)); k = 2; }
    else { b[0] = (char)(0xE0 | (cp >> 12)); b[1] = (char)(0x80 | ((cp >> 6) & 0x3F)); b[2] = (char)(0x80 | (cp & 0x3F)); k = 3; }
    for (int i = 0; i < k; i++)
        if (*n + 1 < cap) out[(*n)++] = b[i];
}
/* A string into out (truncated to cap-1 bytes, always terminated). */
static int str(Json *j, char *out, size_t cap) {
    size_t n = 0;
    if (!expect(j, '"')) return 0;
    while (j->p < j->end && *j->p != '"') {
        char c = *j->p++;
        if (c == '\\') {
            if (j->p >= j->end) break;
            char e = *j->p++;
            unsigned cp = 0;
            switch (e) {
            case 'n': cp = '\n'; break;
            case 't': cp = '\t'; break;
            case 'r': cp = '\r'; break;
            case 'b': cp = '\b'; break;
            case 'f': cp = '\f'; break;
            case 'u':
                for (int i = 0; i < 4; i++) {
                    if (j->p >= j->end) { j->err = 1; return 0; }
                    char h = *j->p++;
                    cp = cp * 16 + (unsigned)(h >= 'a' ? h - 'a' + 10 : h >= 'A' ? h - 'A' + 10 : h - '0');
                }
                break;
            default: cp = (unsigned char)e;  /* \" \\ \/ */
            }
            put_utf8(out, cap, &n, cp);
        } else if (n + 1 < cap) {
            out[n++] = c;
        }
    }
    if (cap) out[n < cap ? n : cap - 1] = 0;
    return expect(j, '"');
}
/* A number: its text is parsed as an unsigned integer when it is one (sizes and offsets
 * beyond 2^53 stay exact), else as a double. */
static int num(Json *j, double *d, unsigned long long *u, int *is_uint) {
    ws(j);
    const char *s = j->p;
    char *e1 = NULL, *e2 = NULL;
    char buf[64];
    size_t len = 0;
    while (j->p < j->end && len + 1 < sizeof buf && strchr("+-0123456789.eE", *j->p)) buf[len++] = *j->p++;
    buf[len] = 0;
    if (len == 0) { j->err = 1; return 0; }
    *d = strtod(buf, &e1);
    *is_uint = 0;
    if (buf[0] != '-' && !strpbrk(buf, ".eE")) {
        errno = 0;
        *u = strtoull(buf, &e2, 10);
        *is_uint = errno == 0 && e2 && *e2 == 0;
    }
    (void)s;
    if (!e1 || *e1) { j->err = 1; return 0; }
    return 1;
}
static int skip(Json *j, int depth) {
    int c = peek(j);
    if (depth > 64) { j->err = 1; return 0; }
    if (c == '"') { char tmp[8]; return str(j, tmp, sizeof tmp); }
    if (c == '{' || c == '[') {
        const char close = c == '{' ? '}' : ']';
        j->p++;
        if (peek(j) == (unsigned char)close) { j->p++; return 1; }
        for (;;) {
            if (c == '{') {
                char tmp[8];
                if (!str(j, tmp, sizeof tmp) || !expect(j, ':')) return 0;
            }
            if (!skip(j, depth + 1)) return 0;
            if (peek(j) == ',') { j->p++; continue; }
            return expect(j, close);
        }
    }
    if (c == 't' || c == 'f' || c == 'n') {
        while (j->p < j->end && *j->p >= 'a' && *j->p <= 'z') j->p++;
        return 1;
    }
    double d; unsigned long long u; int iu;
    return num(j, &d, &u, &iu);
}
/* Object iteration: begin with obj_begin, then obj_key until it returns 0. */
static int obj_begin(Json *j) { return expect(j, '{'); }
static int obj_key(Json *j, char *key, size_t cap, int *first) {
    int c = peek(j);
    if (c == '}') { j->p++; return 0; }
    if (!*first) {
        if (!expect(j, ',')) return 0;
    }
    *first = 0;
    if (!str(j, key, cap) || !expect(j, ':')) return 0;
    return 1;
}

/* ------------------------------------------------------------------ config.json */
typedef struct {
    char key[160];
    double v;
    int has;
} Kv;

static int collect_numbers(const char *text, Kv **out, int *n) {
    Json j = {text, text + strlen(text), 0};
    int cap = 64, cnt = 0, first = 1;
    Kv *kv = (Kv *)malloc(sizeof(Kv) * cap);
    if (!kv) return MNEMO_ERR_ALLOC;
    char key[160];
    if (!obj_begin(&j)) { free(kv); return MNEMO_ERR_BAD_ARG; }
    while (obj_key(&j, key, sizeof key, &first)) {
        int c = peek(&j);
        if (c == '-' || (c >= '0' && c <= '9')) {
            double d; unsigned long long u; int iu;
            if (!num(&j, &d, &u, &iu)) break;
            if (cnt == cap) {
                cap *= 2;
                Kv *t = (Kv *)realloc(kv, sizeof(Kv) * cap);
                if (!t) { free(kv); return MNEMO_ERR_ALLOC; }
                kv = t;
            }
            snprintf(kv[cnt].key, sizeof kv[cnt].key, "%s", key);
            kv[cnt].v = d;
            kv[cnt].has = 1;
            cnt++;
        } else if (!skip(&j, 0)) {
            break;
        }
    }
    if (j.err) { free(kv); return MNEMO_ERR_BAD_ARG; }
    *out = kv;
    *n = cnt;
    return 0;
}

static int find(const Kv *kv, int n, const char *prefix, const char *suffix, double *v) {
    char key[200];
    if (prefix) snprintf(key, sizeof key, "%s.%s", prefix, suffix);
    else snprintf(key, sizeof key, "%s", suffix);
    for (int i = 0; i < n; i++)
        if (strcmp(kv[i].key, key) == 0) { *v = kv[i].v; return 1; }
    return 0;
}

int mnemo_parse_config(const char *json_text, mnemo_model_config *cfg) {
    if (!json_text || !cfg) return fail(MNEMO_ERR_BAD_ARG, "parse_config: NULL argument");
    memset(cfg, 0, sizeof *cfg);
    /* prefix detection in the reference's order (src/engine.c:383-389) */
    const char *prefixes[] = {"qwen35moe", "glm4moe", "qwen3next", "llama", "qwen2"};
    const char *prefix = "qwen3moe";
    for (size_t i = 0; i < sizeof prefixes / sizeof prefixes[0]; i++) {
        char pat[40];
        snprintf(pat, sizeof pat, "\"%s.", prefixes[i]);
        if (strstr(json_text, pat)) { prefix = prefixes[i]; break; }
    }
    snprintf(cfg->prefix, sizeof cfg->prefix, "%s", prefix);
    Kv *kv = NULL;
    int n = 0, rc = collect_numbers(json_text, &kv, &n);
    if (rc) return fail(rc, "parse_config: config.json is not a JSON object of metadata");
    double v;
    int missing = 0;
    const char *req[4] = {"embedding_length", "block_count", "attention.head_count", "attention.head_count_kv"};
    int *dst[4] = {&cfg->hidden_size, &cfg->n_layers, &cfg->n_heads, &cfg->n_kv_heads};
    for (int i = 0; i < 4; i++) {
        if (find(kv, n, prefix, req[i], &v)) *dst[i] = (int)v;
        else { fail(MNEMO_ERR_BAD_ARG, "config.json: missing required key %s.%s", prefix, req[i]); missing++; }
    }
#define OPT_I(field, suffix, def) cfg->field = find(kv, n, prefix, suffix, &v) ? (int)v : (def)
#define OPT_F(field, suffix, def) cfg->field = find(kv, n, prefix, suffix, &v) ? (float)v : (def)
    OPT_I(eff, "expert_feed_forward_length", 1536);
    OPT_I(head_dim, "attention.key_length", 128);
    OPT_I(n_experts, "expert_count", 128);
    OPT_I(experts_per_tok, "expert_used_count", 8);
    OPT_F(rope_theta, "rope.freq_base", 1000000.0f);
    OPT_F(rms_eps, "attention.layer_norm_rms_epsilon", 1e-6f);
    OPT_I(context_length, "context_length", 40960);
    OPT_I(full_attention_interval, "full_attention_interval", 0);
#undef OPT_I
#undef OPT_F
    if (find(kv, n, NULL, "tokenizer.ggml.tokens_count", &v) && v > 0) cfg->vocab_size = (int)v;
    else if (find(kv, n, NULL, "vocab_size", &v) && v > 0) cfg->vocab_size = (int)v;
    else cfg->vocab_size = 151936;
    free(kv);
    if (missing) return MNEMO_ERR_BAD_ARG;
    if (cfg->hidden_size <= 0 || cfg->hidden_size > 65536)
        return fail(MNEMO_ERR_BAD_ARG, "config.json: invalid hidden size %d", cfg->hidden_size);
    if (cfg->n_layers <= 0 || cfg->n_layers > 1024)
        return fail(MNEMO_ERR_BAD_ARG, "config.json: invalid block count %d", cfg->n_layers);
    if (cfg->n_heads <= 0 || cfg->n_kv_heads <= 0 || cfg->n_heads % cfg->n_kv_heads)
        return fail(MNEMO_ERR_BAD_ARG, "config.json: head counts %d / %d", cfg->n_heads, cfg->n_kv_heads);
    /* the expert table is split by n_experts and the kernels size their tables by these */
    if (cfg->n_experts <= 0 || cfg->n_experts > 512)
        return fail(MNEMO_ERR_BAD_ARG, "config.json: invalid expert count %d (1..512)", cfg->n_experts);
    if (cfg->experts_per_tok <= 0 || cfg->experts_per_tok > cfg->n_experts || cfg->experts_per_tok > 16)
        return fail(MNEMO_ERR_BAD_ARG, "config.json: invalid expert_used_count %d (1..min(16, %d))",
                    cfg->experts_per_tok, cfg->n_experts);
    if (cfg->eff <= 0 || cfg->eff > 65536)
        return fail(MNEMO_ERR_BAD_ARG, "config.json: invalid expert_feed_forward_length %d", cfg->eff);
    if (cfg->head_dim <= 0 || cfg->head_dim > 512 || cfg->head_dim % 2)
        return fail(MNEMO_ERR_BAD_ARG, "config.json: invalid key_length %d (even, 2..512)", cfg->head_dim);
    if (cfg->context_length <= 0)
        return fail(MNEMO_ERR_BAD_ARG, "config.json: invalid context_length %d", cfg->context_length);
    return 0;
}

/* ------------------------------------------------------------------ resident_manifest.json */
static int tensor_entry(Json *j, mnemo_tensor_info *e) {
    char key[64];
    int first = 1;
    memset(e, 0, sizeof *e);
    e->type_id = -1;
    if (!obj_begin(j)) return 0;
    while (obj_key(j, key, sizeof key, &first)) {
        double d; unsigned long long u; int iu;
        if (strcmp(key, "name") == 0) {
            if (!str(j, e->name, sizeof e->name)) return 0;
        } else if (strcmp(key, "offset") == 0 || strcmp(key, "size") == 0 || strcmp(key, "type_id") == 0) {
            if (!num(j, &d, &u, &iu) || !iu) { j->err = 1; return 0; }
            if (key[0] == 'o') e->offset = (size_t)u;
            else if (key[0] == 's') e->size = (size_t)u;
            else e->type_id = (int)u;
        } else if (strcmp(key, "dims") == 0) {
            if (!expect(j, '[')) return 0;
            if (peek(j) == ']') { j->p++; continue; }
            for (;;) {
                if (!num(j, &d, &u, &iu)) return 0;
                if (e->n_dims < 4) e->dims[e->n_dims++] = (long long)d;
                if (peek(j) == ',') { j->p++; continue; }
                if (!expect(j, ']')) return 0;
                break;
            }
        } else if (!skip(j, 0)) {
            return 0;
        }
    }
    return !j->err;
}

int mnemo_parse_resident_manifest(const char *json_text, mnemo_tensor_info *out, int max, int *n) {
    if (!json_text || !n || max < 0 || (max > 0 && !out)) return fail(MNEMO_ERR_BAD_ARG, "parse_resident_manifest: bad arguments");
    Json j = {json_text, json_text + strlen(json_text), 0};
    char key[64];
    int first = 1, found = 0, cnt = 0;
    *n = 0;
    if (!obj_begin(&j)) return fail(MNEMO_ERR_BAD_ARG, "resident_manifest.json: not a JSON object");
    while (obj_key(&j, key, sizeof key, &first)) {
        if (strcmp(key, "tensors") != 0) {
            if (!skip(&j, 0)) break;
            continue;
        }
        found = 1;
        if (!expect(&j, '[')) break;
        if (peek(&j) == ']') { j.p++; continue; }
        for (;;) {
            mnemo_tensor_info e;
            if (!tensor_entry(&j, &e)) break;
            if (!e.name[0] || e.type_id < 0) return fail(MNEMO_ERR_BAD_ARG, "resident_manifest.json: entry %d lacks name or type_id", cnt);
            if (cnt < max) out[cnt] = e;
            cnt++;
            if (peek(&j) == ',') { j.p++; continue; }
            expect(&j, ']');
            break;
        }
    }
    if (j.err) return fail(MNEMO_ERR_BAD_ARG, "resident_manifest.json: malformed JSON near byte %ld", (long)(j.p - json_text));
    if (!found) return fail(MNEMO_ERR_BAD_ARG, "resident_manifest.json: no \"tensors\" array");
    *n = cnt;
    return 0;
}

/* ------------------------------------------------------------------ expert_manifest.json */
static int layer_sizes(Json *j, mnemo_expert_layer_info *info) {
    char key[64];
    int first = 1;
    if (!obj_begin(j)) return 0;
    while (obj_key(j, key, sizeof key, &first)) {
        double d; unsigned long long u; int iu;
        size_t *dst = strcmp(key, "expert_size") == 0 ? &info->expert_size
                    : strcmp(key, "gate_size") == 0   ? &info->gate_size
                    : strcmp(key, "up_size") == 0     ? &info->up_size
                    : strcmp(key, "down_size") == 0   ? &info->down_size : NULL;
        if (dst) {
            if (!num(j, &d, &u, &iu) || !iu) { j->err = 1; return 0; }
            *dst = (size_t)u;
        } else if (!skip(j, 0)) {
            return 0;
        }
    }
    return !j->err;
}

/* Looks for the layer's object at the top level or under a top-level "layers" object. */
static int find_layer(Json *j, const char *want, mnemo_expert_layer_info *info, int depth) {
    char key[64];
    int first = 1;
    if (!obj_begin(j)) return -1;
    while (obj_key(j, key, sizeof key, &first)) {
        if (strcmp(key, want) == 0 && peek(j) == '{') return layer_sizes(j, info) ? 1 : -1;
        if (depth == 0 && strcmp(key, "layers") == 0 && peek(j) == '{') {
            int r = find_layer(j, want, info, 1);
            if (r != 0) return r;
            continue;
        }
        if (!skip(j, 0)) return -1;
    }
    return j->err ? -1 : 0;
}

int mnemo_parse_expert_manifest(const char *json_text, int layer, mnemo_expert_layer_info *info) {
    if (!json_text || !info || layer < 0) return fail(MNEMO_ERR_BAD_ARG, "parse_expert_manifest: bad arguments");
    memset(info, 0, sizeof *info);
    char want[16];
    snprintf(want, sizeof want, "%d", layer);
    Json j = {json_text, json_text + strlen(json_text), 0};
    if (find_layer(&j, want, info, 0) < 0)
        return fail(MNEMO_ERR_BAD_ARG, "expert_manifest.json: malformed JSON near byte %ld", (long)(j.p - json_text));
    return 0;
}

size_t mnemo_row_bytes(int type_id, int n) {
    if (n <= 0) return 0;
    switch (type_id) {
    case MNEMO_TYPE_F32: return (size_t)n * 4;
    case MNEMO_TYPE_Q4_K: return (size_t)((n + 255) / 256) * 144;
    case MNEMO_TYPE_Q6_K: return (size_t)((n + 255) / 256) * 210;
    default: return 0;
    }
}

/* ------------------------------------------------------------------ the directory */
struct mnemo_model {
    char dir[1024];
    mnemo_model_config cfg;
    mnemo_tensor_info *tensors;
    size_t *dev_off;  /* per tensor, in d_resident */
    int n_tensors;
    size_t resident_file_size, resident_dev_size;
    mnemo_expert_layer_info *layers;
    int *has_layer;
    void *d_resident;
    void **d_experts;
};

static char *read_text(const char *path, long max_bytes) {
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    if (fseek(f, 0, SEEK_END) != 0) { fclose(f); return NULL; }
    long sz = ftell(f);
    if (sz < 0 || sz > max_bytes || fseek(f, 0, SEEK_SET) != 0) { fclose(f); return NULL; }
    char *buf = (char *)malloc((size_t)sz + 1);
    if (!buf) { fclose(f); return NULL; }
    size_t got = fread(buf, 1, (size_t)sz, f);
    fclose(f);
    buf[got] = 0;
    return buf;
}

static long long file_size(const char *path) {
    struct stat st;
    return stat(path, &st) == 0 ? (long long)st.st_size : -1;
}

void mnemo_model_close(mnemo_model *m) {
    if (!m) return;
    if (m->d_resident) hipFree(m->d_resident);
    if (m->d_experts) {
        for (int i = 0; i < m->cfg.n_layers; i++)
            if (m->d_experts[i]) hipFree(m->d_experts[i]);
        free(m->d_experts);
    }
    free(m->tensors);
    free(m->dev_off);
    free(m->layers);
    free(m->has_layer);
    free(m);
}

int mnemo_model_open(const char *dir, mnemo_model **out) {
    if (!dir || !out) return fail(MNEMO_ERR_BAD_ARG, "model_open: NULL argument");
    *out = NULL;
    mnemo_model *m = (mnemo_model *)calloc(1, sizeof *m);
    if (!m) return fail(MNEMO_ERR_ALLOC, "model_open: out of host memory");
    snprintf(m->dir, sizeof m->dir, "%s", dir);
    char path[1200];
    int rc;
    snprintf(path, sizeof path, "%s/config.json", dir);
    char *text = read_text(path, 64L << 20);
    if (!text) { mnemo_model_close(m); return fail(MNEMO_ERR_IO, "model_open: cannot read %s", path); }
    rc = mnemo_parse_config(text, &m->cfg);
    free(text);
    if (rc) { mnemo_model_close(m); return rc; }

    snprintf(path, sizeof path, "%s/resident_manifest.json", dir);
    text = read_text(path, 256L << 20);
    if (!text) { mnemo_model_close(m); return fail(MNEMO_ERR_IO, "model_open: cannot read %s", path); }
    int n = 0;
    rc = mnemo_parse_resident_manifest(text, NULL, 0, &n);
    if (!rc && n > 0) {
        m->tensors = (mnemo_tensor_info *)calloc((size_t)n, sizeof *m->tensors);
        m->dev_off = (size_t *)calloc((size_t)n, sizeof *m->dev_off);
        if (!m->tensors || !m->dev_off) rc = fail(MNEMO_ERR_ALLOC, "model_open: out of host memory");
        else rc = mnemo_parse_resident_manifest(text, m->tensors, n, &n);
    }
    free(text);
    if (rc) { mnemo_model_close(m); return rc; }
    m->n_tensors = n;
    snprintf(path, sizeof path, "%s/resident_weights.bin", dir);
    long long rsz = file_size(path);
    if (rsz < 0) { mnemo_model_close(m); return fail(MNEMO_ERR_IO, "model_open: cannot stat %s", path); }
    m->resident_file_size = (size_t)rsz;
    size_t off = 0;
    for (int i = 0; i < n; i++) {
        const mnemo_tensor_info *t = &m->tensors[i];
        if (t->offset > m->resident_file_size || t->size > m->resident_file_size - t->offset) {
            mnemo_model_close(m);
            return fail(MNEMO_ERR_BAD_ARG, "resident tensor %s [%zu, +%zu) outside resident_weights.bin (%zu B)",
                        t->name, t->offset, t->size, (size_t)rsz);
        }
        off = (off + 255) & ~(size_t)255;
        m->dev_off[i] = off;
        off += t->size;
    }
    m->resident_dev_size = off ? off : 256;

    /* experts */
    const int L = m->cfg.n_layers;
    m->layers = (mnemo_expert_layer_info *)calloc((size_t)L, sizeof *m->layers);
    m->has_layer = (int *)calloc((size_t)L, sizeof *m->has_layer);
    m->d_experts = (void **)calloc((size_t)L, sizeof *m->d_experts);
    if (!m->layers || !m->has_layer || !m->d_experts) { mnemo_model_close(m); return fail(MNEMO_ERR_ALLOC, "model_open: out of host memory"); }
    snprintf(path, sizeof path, "%s/expert_manifest.json", dir);
    char *em = read_text(path, 64L << 20);  /* optional */
    for (int l = 0; l < L; l++) {
        snprintf(path, sizeof path, "%s/experts/layer_%02d.bin", dir, l);
        long long esz = file_size(path);
        if (esz < 0) continue;  /* a layer without an expert file has no MoE (src/engine.c:690-692) */
        mnemo_expert_layer_info *li = &m->layers[l];
        if (em && (rc = mnemo_parse_expert_manifest(em, l, li))) { free(em); mnemo_model_close(m); return rc; }
        const size_t per = (size_t)esz / (size_t)m->cfg.n_experts;
        if (!li->expert_size) li->expert_size = per;
        if (li->expert_size * (size_t)m->cfg.n_experts != (size_t)esz) {
            free(em);
            mnemo_model_close(m);
            return fail(MNEMO_ERR_BAD_ARG, "experts/layer_%02d.bin: %lld B is not %d experts x %zu B", l, esz,
                        m->cfg.n_experts, li->expert_size);
        }
        if (!li->gate_size && !li->up_size && !li->down_size) {
            /* no per-tensor sizes: thirds (src/forward.c:866-870) */
            li->gate_size = li->up_size = li->expert_size / 3;
            li->down_size = li->expert_size - 2 * (li->expert_size / 3);
        }
        if (li->gate_size + li->up_size + li->down_size > li->expert_size) {
            free(em);
            mnemo_model_close(m);
            return fail(MNEMO_ERR_BAD_ARG, "expert layer %d: gate + up + down = %zu > expert_size %zu", l,
                        li->gate_size + li->up_size + li->down_size, li->expert_size);
        }
        li->down_type_id = mnemo_down_type_id(li->down_size, m->cfg.hidden_size, m->cfg.eff);
        li->n_experts = m->cfg.n_experts;
        m->has_layer[l] = 1;
    }
    free(em);
    *out = m;
    return 0;
}

const mnemo_model_config *mnemo_model_config_of(const mnemo_model *m) { return m ? &m->cfg : NULL; }
int mnemo_model_n_tensors(const mnemo_model *m) { return m ? m->n_tensors : 0; }

int mnemo_model_tensor_at(const mnemo_model *m, int i, mnemo_tensor_info *info) {
    if (!m || !info || i < 0 || i >= m->n_tensors) return fail(MNEMO_ERR_BAD_ARG, "model_tensor_at: index %d", i);
    *info = m->tensors[i];
    return 0;
}

int mnemo_model_expert_layer(const mnemo_model *m, int layer, mnemo_expert_layer_info *info) {
    if (!m || !info || layer < 0 || layer >= m->cfg.n_layers || !m->has_layer[layer])
        return fail(MNEMO_ERR_BAD_ARG, "model_expert_layer: layer %d has no expert file", layer);
    *info = m->layers[layer];
    return 0;
}

/* Copies [off, off + size) of a file to dst on the device through a pinned staging buffer. */
static int upload_file(const char *path, size_t off, size_t size, void *dst, void *stage, size_t stage_size) {
    FILE *f = fopen(path, "rb");
    if (!f) return fail(MNEMO_ERR_IO, "upload: cannot open %s", path);
    if (fseeko(f, (off_t)off, SEEK_SET) != 0) { fclose(f); return fail(MNEMO_ERR_IO, "upload: seek in %s", path); }
    size_t done = 0;
    while (done < size) {
        const size_t want = size - done < stage_size ? size - done : stage_size;
        const size_t got = fread(stage, 1, want, f);
        if (got != want) { fclose(f); return fail(MNEMO_ERR_IO, "upload: short read in %s", path); }
        if (hipMemcpy((char *)dst + done, stage, got, hipMemcpyHostToDevice) != hipSuccess) {
            fclose(f);
            return fail(MNEMO_ERR_LAUNCH, "upload: hipMemcpy failed");
        }
        done += got;
    }
    fclose(f);
    return 0;
}

int mnemo_model_upload(mnemo_model *m, int with_experts) {
    if (!m) return fail(MNEMO_ERR_BAD_ARG, "model_upload: NULL model");
    const size_t stage_size = 64u << 20;
    void *stage = NULL;
    if (hipHostMalloc(&stage, stage_size, 0) != hipSuccess) return fail(MNEMO_ERR_ALLOC, "model_upload: pinned staging buffer");
    int rc = 0;
    char path[1200];
    if (!m->d_resident) {
        if (hipMalloc(&m->d_resident, m->resident_dev_size) != hipSuccess) {
            m->d_resident = NULL;
            rc = fail(MNEMO_ERR_ALLOC, "model_upload: %zu B of device memory", m->resident_dev_size);
        }
        snprintf(path, sizeof path, "%s/resident_weights.bin", m->dir);
        for (int i = 0; !rc && i < m->n_tensors; i++)
            rc = upload_file(path, m->tensors[i].offset, m->tensors[i].size, (char *)m->d_resident + m->dev_off[i], stage,
                             stage_size);
        if (rc && m->d_resident) {  // a partial copy is not kept: a later call starts over
            (void)hipFree(m->d_resident);
            m->d_resident = NULL;
        }
    }
    for (int l = 0; !rc && with_experts && l < m->cfg.n_layers; l++) {
        if (!m->has_layer[l] || m->d_experts[l]) continue;
        const size_t bytes = m->layers[l].expert_size * (size_t)m->layers[l].n_experts;
        if (hipMalloc(&m->d_experts[l], bytes) != hipSuccess) {
            m->d_experts[l] = NULL;
            rc = fail(MNEMO_ERR_ALLOC, "model_upload: %zu B for expert layer %d", bytes, l);
            break;
        }
        snprintf(path, sizeof path, "%s/experts/layer_%02d.bin", m->dir, l);
        rc = upload_file(path, 0, bytes, m->d_experts[l], stage, stage_size);
        if (rc) {
            (void)hipFree(m->d_experts[l]);
            m->d_experts[l] = NULL;
        }
    }
    hipHostFree(stage);
    return rc;
}

int mnemo_model_tensor(const mnemo_model *m, const char *name, mnemo_tensor_info *info, void **dev_ptr) {
    if (!m || !name) return fail(MNEMO_ERR_BAD_ARG, "model_tensor: NULL argument");
    for (int i = 0; i < m->n_tensors; i++) {
        if (strcmp(m->tensors[i].name, name) != 0) continue;
        if (info) *info = m->tensors[i];
        if (dev_ptr) *dev_ptr = m->d_resident ? (char *)m->d_resident + m->dev_off[i] : NULL;
        return 0;
    }
    return fail(MNEMO_ERR_BAD_ARG, "model_tensor: no tensor %s", name);
}

int mnemo_model_experts(const mnemo_model *m, int layer, void **dev_ptr) {
    if (!m || !dev_ptr || layer < 0 || layer >= m->cfg.n_layers || !m->d_experts[layer])
        return fail(MNEMO_ERR_BAD_ARG, "model_experts: layer %d not uploaded", layer);
    *dev_ptr = m->d_experts[layer];
    return 0;
}
