/*
 * pico_amd/host/checkpoint.c -- checkpoints of params and AdamW state.
 *
 * The reference saves nothing: params are plain float arrays
 * (src/tensor.h:14-15) that live as long as the process.  Here a checkpoint
 * is a safetensors file, so any safetensors reader can open it:
 *
 *   u64 little-endian N | N bytes of JSON header (space-padded to a multiple
 *   of 8) | raw little-endian tensor bytes
 *
 * The header maps each name to {"dtype", "shape", "data_offsets": [begin,
 * end)} (offsets into the data section); "__metadata__" holds strings.
 * Params are F32 with their shape.  With an AdamW optimizer, each of its
 * params also gets "<name>.adam_m" and "<name>.adam_v", and "adamw.step" is
 * the step count as an I32 scalar; the hyper-parameters go to the metadata.
 * Loading checks every name, dtype and shape before anything is written to
 * the device, then restores the tensors, the moments and the step count, so
 * a resumed run continues exactly as the saved one would have.
 */
#include <ctype.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "pk_host.h"

#define CK_MAX_DIMS 8

struct CkEntry {
    char* name;
    char dtype[8];
    int ndim;
    int64_t shape[CK_MAX_DIMS];
    uint64_t begin, end;
};

/* -------------------------------------------------------------- writing */
struct CkBuf {
    char* s;
    size_t n, cap;
    int oom;
};

static void cb_put(struct CkBuf* b, const char* fmt, ...) {
    if(b->oom) return;
    for(;;) {
        va_list ap;
        va_start(ap, fmt);
        int k = vsnprintf(b->s + b->n, b->cap - b->n, fmt, ap);
        va_end(ap);
        if(k < 0) {
            b->oom = 1;
            return;
        }
        if(b->n + (size_t)k < b->cap) {
            b->n += (size_t)k;
            return;
        }
        size_t cap = b->cap ? 2 * b->cap : 4096;
        while(cap <= b->n + (size_t)k) cap *= 2;
        char* ns = (char*)realloc(b->s, cap);
        if(!ns) {
            b->oom = 1;
            return;
        }
        b->s = ns;
        b->cap = cap;
    }
}

static int name_ok(const char* s) {
    if(!s || !*s) return 0;
    for(; *s; s++)
        if(*s == '"' || *s == '\\' || (unsigned char)*s < 0x20) return 0;
    return 1;
}

/* one item to write: device source and element count, or a host int */
struct CkItem {
    char name[256];
    const struct PicoTensor* shape_of; /* NULL: a scalar I32 */
    const float* dev;
    int64_t numel;
    int32_t i32;
};

static int ck_fail(const char* fmt, const char* a) {
    pkh_set_error(fmt, a);
    PKH_ERR("%s\n", pico_gpu_last_error());
    return PK_EINVAL;
}

static int contiguous(const struct PicoTensor* t) {
    int64_t s = 1;
    for(int d = t->ndim - 1; d >= 0; d--) {
        if(t->shape[d] != 1 && t->strides[d] != s) return 0;
        s *= t->shape[d];
    }
    return 1;
}

static int check_tensors(int n, struct PicoTensor* const* tensors, const char* const* names) {
    if(n < 0 || (n > 0 && !tensors)) return ck_fail("checkpoint: %s", "bad tensor list");
    for(int i = 0; i < n; i++) {
        const struct PicoTensor* t = tensors[i];
        if(!t || !pkh_node((struct PicoTensor*)t) || !pkh_is_gpu(t))
            return ck_fail("checkpoint: %s", "tensors must be GPU tensors of this library");
        if(!contiguous(t)) return ck_fail("checkpoint: %s", "tensors must be contiguous");
        if(t->ndim > CK_MAX_DIMS) return ck_fail("checkpoint: %s", "more than 8 dims");
        if(names && !name_ok(names[i]))
            return ck_fail("checkpoint: bad name '%s'", names[i] ? names[i] : "(null)");
    }
    return 0;
}

static void item_name(char* dst, const char* const* names, int i, const char* suffix) {
    if(names)
        snprintf(dst, 256, "%s%s", names[i], suffix);
    else
        snprintf(dst, 256, "param.%d%s", i, suffix);
}

/* the items of a checkpoint, in file order; returns the count or -1 */
static int ck_items(int n, struct PicoTensor* const* tensors, const char* const* names,
                    const struct PicoOptimAdamW* o, struct CkItem** out) {
    struct CkItem* it = (struct CkItem*)calloc((size_t)(3 * n + 1), sizeof(*it));
    if(!it) return -1;
    int k = 0;
    for(int i = 0; i < n; i++) {
        item_name(it[k].name, names, i, "");
        it[k].shape_of = tensors[i];
        it[k].dev = tensors[i]->data;
        it[k].numel = tensors[i]->numel;
        k++;
    }
    if(o) {
        for(int i = 0; i < n; i++) {
            float *m, *v;
            if(!pkh_adamw_moments(o, tensors[i], &m, &v)) continue;
            item_name(it[k].name, names, i, ".adam_m");
            it[k].shape_of = tensors[i];
            it[k].dev = m;
            it[k].numel = tensors[i]->numel;
            k++;
            item_name(it[k].name, names, i, ".adam_v");
            it[k].shape_of = tensors[i];
            it[k].dev = v;
            it[k].numel = tensors[i]->numel;
            k++;
        }
        snprintf(it[k].name, 256, "adamw.step");
        it[k].i32 = pkh_adamw_step(o);
        k++;
    }
    *out = it;
    return k;
}

int pico_checkpoint_save(const char* path, int n, struct PicoTensor* const* tensors,
                         const char* const* names, const struct PicoOptimAdamW* adamw) {
    if(pkh_init()) return PK_EINVAL;
    if(!path) return ck_fail("pico_checkpoint_save: %s", "NULL path");
    int rc = check_tensors(n, tensors, names);
    if(rc) return rc;
    if(adamw && pkh_adamw_sync_step((struct PicoOptimAdamW*)adamw)) return PK_EINVAL;
    struct CkItem* it = NULL;
    const int count = ck_items(n, tensors, names, adamw, &it);
    if(count < 0) return ck_fail("pico_checkpoint_save: %s", "out of host memory");

    struct CkBuf h = {0};
    cb_put(&h, "{\"__metadata__\":{\"format\":\"pt\",\"writer\":\"pico_amd\"");
    if(adamw) {
        float lr, b1, b2, eps, wd;
        pkh_adamw_hparams(adamw, &lr, &b1, &b2, &eps, &wd);
        cb_put(&h, ",\"adamw.lr\":\"%.9g\",\"adamw.beta1\":\"%.9g\",\"adamw.beta2\":\"%.9g\","
                   "\"adamw.eps\":\"%.9g\",\"adamw.weight_decay\":\"%.9g\"",
               lr, b1, b2, eps, wd);
    }
    cb_put(&h, "}");
    uint64_t off = 0;
    for(int k = 0; k < count; k++) {
        if(it[k].shape_of) {
            const uint64_t bytes = (uint64_t)it[k].numel * 4;
            cb_put(&h, ",\"%s\":{\"dtype\":\"F32\",\"shape\":[", it[k].name);
            for(int d = 0; d < it[k].shape_of->ndim; d++)
                cb_put(&h, "%s%lld", d ? "," : "", (long long)it[k].shape_of->shape[d]);
            cb_put(&h, "],\"data_offsets\":[%llu,%llu]}", (unsigned long long)off,
                   (unsigned long long)(off + bytes));
            off += bytes;
        } else {
            cb_put(&h, ",\"%s\":{\"dtype\":\"I32\",\"shape\":[],\"data_offsets\":[%llu,%llu]}",
                   it[k].name, (unsigned long long)off, (unsigned long long)(off + 4));
            off += 4;
        }
    }
    cb_put(&h, "}");
    while(!h.oom && h.n % 8) cb_put(&h, " ");
    if(h.oom) {
        free(it);
        free(h.s);
        return ck_fail("pico_checkpoint_save: %s", "out of host memory");
    }

    FILE* f = fopen(path, "wb");
    if(!f) {
        free(it);
        free(h.s);
        return ck_fail("pico_checkpoint_save: cannot open '%s' for writing", path);
    }
    unsigned char len[8];
    for(int b = 0; b < 8; b++) len[b] = (unsigned char)(((uint64_t)h.n >> (8 * b)) & 0xff);
    int ok = fwrite(len, 1, 8, f) == 8 && fwrite(h.s, 1, h.n, f) == h.n;
    float* host = NULL;
    size_t host_cap = 0;
    for(int k = 0; ok && k < count; k++) {
        if(!it[k].shape_of) {
            unsigned char v[4];
            for(int b = 0; b < 4; b++) v[b] = (unsigned char)(((uint32_t)it[k].i32 >> (8 * b)) & 0xff);
            ok = fwrite(v, 1, 4, f) == 4;
            continue;
        }
        const size_t bytes = (size_t)it[k].numel * 4;
        if(bytes > host_cap) {
            float* nh = (float*)realloc(host, bytes);
            if(!nh) {
                ok = 0;
                break;
            }
            host = nh;
            host_cap = bytes;
        }
        ok = pkh_copy_d2h(host, it[k].dev, bytes) == 0 && fwrite(host, 1, bytes, f) == bytes;
    }
    ok = (fclose(f) == 0) && ok;
    free(host);
    free(it);
    free(h.s);
    if(!ok) return ck_fail("pico_checkpoint_save: writing '%s' failed", path);
    return 0;
}

/* -------------------------------------------------------------- reading */
/* A small JSON reader for safetensors headers: objects, arrays, strings,
 * numbers and literals; only the fields a tensor entry needs are kept. */
struct Js {
    const char* p;
    const char* end;
    int err;
};

static void js_ws(struct Js* j) {
    while(j->p < j->end && isspace((unsigned char)*j->p)) j->p++;
}

static int js_eat(struct Js* j, char c) {
    js_ws(j);
    if(j->p < j->end && *j->p == c) {
        j->p++;
        return 1;
    }
    return 0;
}

/* a string into dst (cap bytes, truncated); escapes other than \" and \\ are
 * kept as written */
static int js_str(struct Js* j, char* dst, size_t cap) {
    js_ws(j);
    if(j->p >= j->end || *j->p != '"') return j->err = 1, 0;
    j->p++;
    size_t n = 0;
    while(j->p < j->end && *j->p != '"') {
        char c = *j->p++;
        if(c == '\\' && j->p < j->end) c = *j->p++;
        if(dst && n + 1 < cap) dst[n++] = c;
    }
    if(j->p >= j->end) return j->err = 1, 0;
    j->p++;
    if(dst && cap) dst[n] = 0;
    return 1;
}

static int js_u64(struct Js* j, uint64_t* v) {
    js_ws(j);
    if(j->p >= j->end || !isdigit((unsigned char)*j->p)) return j->err = 1, 0;
    uint64_t x = 0;
    while(j->p < j->end && isdigit((unsigned char)*j->p)) x = 10 * x + (uint64_t)(*j->p++ - '0');
    *v = x;
    return 1;
}

static void js_skip(struct Js* j) {
    js_ws(j);
    if(j->p >= j->end) {
        j->err = 1;
        return;
    }
    char c = *j->p;
    if(c == '"') {
        js_str(j, NULL, 0);
    } else if(c == '{' || c == '[') {
        const char close = c == '{' ? '}' : ']';
        j->p++;
        if(js_eat(j, close)) return;
        do {
            if(c == '{') {
                js_str(j, NULL, 0);
                if(!js_eat(j, ':')) j->err = 1;
            }
            js_skip(j);
        } while(!j->err && js_eat(j, ','));
        if(!js_eat(j, close)) j->err = 1;
    } else {
        while(j->p < j->end && *j->p != ',' && *j->p != '}' && *j->p != ']') j->p++;
    }
}

static int js_entry(struct Js* j, struct CkEntry* e) {
    if(!js_eat(j, '{')) return j->err = 1, 0;
    int have_dtype = 0, have_shape = 0, have_off = 0;
    if(!js_eat(j, '}')) {
        do {
            char key[32];
            if(!js_str(j, key, sizeof(key)) || !js_eat(j, ':')) return j->err = 1, 0;
            if(!strcmp(key, "dtype")) {
                have_dtype = js_str(j, e->dtype, sizeof(e->dtype));
            } else if(!strcmp(key, "shape")) {
                if(!js_eat(j, '[')) return j->err = 1, 0;
                e->ndim = 0;
                if(!js_eat(j, ']')) {
                    do {
                        uint64_t v;
                        if(e->ndim >= CK_MAX_DIMS || !js_u64(j, &v)) return j->err = 1, 0;
                        e->shape[e->ndim++] = (int64_t)v;
                    } while(js_eat(j, ','));
                    if(!js_eat(j, ']')) return j->err = 1, 0;
                }
                have_shape = 1;
            } else if(!strcmp(key, "data_offsets")) {
                if(!js_eat(j, '[') || !js_u64(j, &e->begin) || !js_eat(j, ',') ||
                   !js_u64(j, &e->end) || !js_eat(j, ']'))
                    return j->err = 1, 0;
                have_off = 1;
            } else {
                js_skip(j);
            }
        } while(!j->err && js_eat(j, ','));
        if(!js_eat(j, '}')) return j->err = 1, 0;
    }
    return !j->err && have_dtype && have_shape && have_off;
}

static char* ck_strdup(const char* s) {
    const size_t n = strlen(s) + 1;
    char* d = (char*)malloc(n);
    if(d) memcpy(d, s, n);
    return d;
}

static void free_entries(struct CkEntry* e, int n) {
    for(int i = 0; i < n; i++) free(e[i].name);
    free(e);
}

/* the header's tensor entries; returns their count or -1 */
static int ck_parse(const char* text, size_t len, struct CkEntry** out) {
    struct Js j = {text, text + len, 0};
    int n = 0, cap = 64;
    struct CkEntry* e = (struct CkEntry*)calloc((size_t)cap, sizeof(*e));
    if(!e || !js_eat(&j, '{')) {
        free(e);
        return -1;
    }
    if(!js_eat(&j, '}')) {
        do {
            char name[256];
            if(!js_str(&j, name, sizeof(name)) || !js_eat(&j, ':')) break;
            if(!strcmp(name, "__metadata__")) {
                js_skip(&j);
                continue;
            }
            if(n == cap) {
                struct CkEntry* ne = (struct CkEntry*)realloc(e, sizeof(*e) * (size_t)(2 * cap));
                if(!ne) {
                    j.err = 1;
                    break;
                }
                memset(ne + cap, 0, sizeof(*e) * (size_t)cap);
                e = ne;
                cap *= 2;
            }
            e[n].name = ck_strdup(name);
            if(!e[n].name || !js_entry(&j, &e[n])) {
                n += e[n].name != NULL;
                j.err = 1;
                break;
            }
            n++;
        } while(!j.err && js_eat(&j, ','));
        if(!j.err && !js_eat(&j, '}')) j.err = 1;
    }
    if(j.err) {
        free_entries(e, n);
        return -1;
    }
    *out = e;
    return n;
}

static const struct CkEntry* find_entry(const struct CkEntry* e, int n, const char* name) {
    for(int i = 0; i < n; i++)
        if(!strcmp(e[i].name, name)) return &e[i];
    return NULL;
}

int pico_checkpoint_load(const char* path, int n, struct PicoTensor* const* tensors,
                         const char* const* names, struct PicoOptimAdamW* adamw) {
    if(pkh_init()) return PK_EINVAL;
    if(!path) return ck_fail("pico_checkpoint_load: %s", "NULL path");
    int rc = check_tensors(n, tensors, names);
    if(rc) return rc;
    FILE* f = fopen(path, "rb");
    if(!f) return ck_fail("pico_checkpoint_load: cannot open '%s'", path);
    unsigned char len[8];
    uint64_t hl = 0;
    if(fread(len, 1, 8, f) != 8) {
        fclose(f);
        return ck_fail("pico_checkpoint_load: '%s' is not a safetensors file", path);
    }
    for(int b = 7; b >= 0; b--) hl = (hl << 8) | len[b];
    if(hl == 0 || hl > ((uint64_t)1 << 30)) {
        fclose(f);
        return ck_fail("pico_checkpoint_load: '%s' has an implausible header", path);
    }
    char* text = (char*)malloc((size_t)hl);
    if(!text || fread(text, 1, (size_t)hl, f) != (size_t)hl) {
        free(text);
        fclose(f);
        return ck_fail("pico_checkpoint_load: cannot read the header of '%s'", path);
    }
    struct CkEntry* e = NULL;
    const int ne = ck_parse(text, (size_t)hl, &e);
    free(text);
    if(ne < 0) {
        fclose(f);
        return ck_fail("pico_checkpoint_load: '%s' has a malformed header", path);
    }
    struct CkItem* it = NULL;
    const int count = ck_items(n, tensors, names, adamw, &it);
    if(count < 0) {
        free_entries(e, ne);
        fclose(f);
        return ck_fail("pico_checkpoint_load: %s", "out of host memory");
    }
    /* every item must be present with its dtype and shape before anything is written */
    const struct CkEntry** src = (const struct CkEntry**)calloc((size_t)(count ? count : 1),
                                                                 sizeof(*src));
    rc = src ? 0 : ck_fail("pico_checkpoint_load: %s", "out of host memory");
    for(int k = 0; !rc && k < count; k++) {
        const struct CkEntry* x = find_entry(e, ne, it[k].name);
        if(!x) {
            rc = ck_fail("pico_checkpoint_load: '%s' is missing from the file", it[k].name);
            break;
        }
        int match;
        if(it[k].shape_of) {
            match = !strcmp(x->dtype, "F32") && x->ndim == it[k].shape_of->ndim &&
                    x->end - x->begin == (uint64_t)it[k].numel * 4;
            for(int d = 0; match && d < x->ndim; d++)
                match = x->shape[d] == it[k].shape_of->shape[d];
        } else {
            match = !strcmp(x->dtype, "I32") && x->ndim == 0 && x->end - x->begin == 4;
        }
        if(!match) rc = ck_fail("pico_checkpoint_load: '%s' has another dtype or shape", it[k].name);
        src[k] = x;
    }
    const long data0 = (long)(8 + hl);
    float* host = NULL;
    size_t host_cap = 0;
    int32_t step = 0;
    for(int k = 0; !rc && k < count; k++) {
        const size_t bytes = (size_t)(src[k]->end - src[k]->begin);
        if(bytes > host_cap) {
            float* nh = (float*)realloc(host, bytes);
            if(!nh) {
                rc = ck_fail("pico_checkpoint_load: %s", "out of host memory");
                break;
            }
            host = nh;
            host_cap = bytes;
        }
        if(fseek(f, data0 + (long)src[k]->begin, SEEK_SET) || fread(host, 1, bytes, f) != bytes) {
            rc = ck_fail("pico_checkpoint_load: '%s' is truncated", path);
            break;
        }
        if(it[k].shape_of) {
            if(pkh_copy_h2d((void*)it[k].dev, host, bytes)) rc = PK_EINVAL;
        } else {
            const unsigned char* b = (const unsigned char*)host;
            step = (int32_t)((uint32_t)b[0] | (uint32_t)b[1] << 8 | (uint32_t)b[2] << 16 |
                             (uint32_t)b[3] << 24);
        }
    }
    if(!rc && adamw) rc = pkh_adamw_set_step(adamw, step);
    free(host);
    free((void*)src);
    free(it);
    free_entries(e, ne);
    fclose(f);
    return rc;
}
