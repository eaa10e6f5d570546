/*
 * tbq_gguf.c -- GGUF file to HBM (include/tbq_gguf.h), C11 over tbq.h.
 *
 * The reference reads the header with fread and maps the file
 * (tb_gguf_load, layer4/tb_gguf.c:563-828) and uploads a fixed list of
 * qtypes (tb_gguf_cuda_upload_all, :469-520).  Here the whole file is
 * mapped first and parsed from memory with a cursor that checks every read
 * against the file size, and every tensor of a qtype libtbq knows is
 * uploaded.  The data section starts at the next multiple of
 * general.alignment (the GGUF rule; the reference always uses 32, the
 * default, so both agree on files without that key).
 */
#define _POSIX_C_SOURCE 200809L

#include "tbq_gguf.h"

#include <fcntl.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

int tbq_host_fail(const char *msg); /* tbq_api.hip: sets tbq_last_error() */

static int failf(const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return tbq_host_fail(buf);
}

/* GGUF metadata value types */
enum { GT_U8 = 0, GT_I8, GT_U16, GT_I16, GT_U32, GT_I32, GT_F32, GT_BOOL, GT_STR, GT_ARR, GT_U64, GT_I64, GT_F64 };

typedef struct {
    char *key;
    int type;
    long long i;         /* integer and bool types */
    double f;            /* float types */
    const char *s;       /* GT_STR: bytes in the map */
    size_t slen;
} kv_t;

typedef struct {
    char *name;
    int qtype, n_dims;
    long long dims[4];
    uint64_t offset;     /* from the data section */
    size_t bytes;        /* 0: unknown qtype */
    void *dev;
} tensor_t;

struct tbq_gguf {
    int fd;
    const uint8_t *map;
    size_t size;
    uint32_t version;
    size_t data_off;
    int n_kv, n_tensors;
    kv_t *kv;
    tensor_t *t;
    void **owned;        /* fused matrices and KV caches */
    int n_owned, cap_owned;
    int layout;          /* 0: the reference's block layouts; TBQ_GGML: ggml's */
};

/* ---- bounds-checked cursor over the map ---------------------------------- */
typedef struct {
    const uint8_t *p;
    size_t left;
    int ok;
} cur_t;

static int rd(cur_t *c, void *dst, size_t n) {
    if (!c->ok || c->left < n) return c->ok = 0;
    memcpy(dst, c->p, n);
    c->p += n;
    c->left -= n;
    return 1;
}
static uint32_t rd_u32(cur_t *c) {
    uint32_t v = 0;
    rd(c, &v, 4);
    return v;
}
static uint64_t rd_u64(cur_t *c) {
    uint64_t v = 0;
    rd(c, &v, 8);
    return v;
}
static const char *rd_str(cur_t *c, size_t *len) {
    const uint64_t n = rd_u64(c);
    if (!c->ok || n > c->left) {
        c->ok = 0;
        return NULL;
    }
    const char *s = (const char *)c->p;
    c->p += n;
    c->left -= n;
    *len = (size_t)n;
    return s;
}
static char *dup_str(const char *s, size_t n) {
    char *r = (char *)malloc(n + 1);
    if (r) {
        memcpy(r, s, n);
        r[n] = 0;
    }
    return r;
}
static size_t scalar_size(int type) {
    switch (type) {
    case GT_U8: case GT_I8: case GT_BOOL: return 1;
    case GT_U16: case GT_I16: return 2;
    case GT_U32: case GT_I32: case GT_F32: return 4;
    case GT_U64: case GT_I64: case GT_F64: return 8;
    default: return 0;
    }
}
/* A scalar of `type` into kv's i / f fields. */
static void rd_scalar(cur_t *c, int type, kv_t *kv) {
    uint8_t b[8] = {0};
    const size_t n = scalar_size(type);
    if (!n || !rd(c, b, n)) {
        c->ok = 0;
        return;
    }
    switch (type) {
    case GT_U8: kv->i = b[0]; break;
    case GT_BOOL: kv->i = b[0] != 0; break;
    case GT_I8: kv->i = (int8_t)b[0]; break;
    case GT_U16: { uint16_t v; memcpy(&v, b, 2); kv->i = v; break; }
    case GT_I16: { int16_t v; memcpy(&v, b, 2); kv->i = v; break; }
    case GT_U32: { uint32_t v; memcpy(&v, b, 4); kv->i = v; break; }
    case GT_I32: { int32_t v; memcpy(&v, b, 4); kv->i = v; break; }
    case GT_U64: { uint64_t v; memcpy(&v, b, 8); kv->i = (long long)v; break; }
    case GT_I64: { int64_t v; memcpy(&v, b, 8); kv->i = v; break; }
    case GT_F32: { float v; memcpy(&v, b, 4); kv->f = v; break; }
    case GT_F64: { double v; memcpy(&v, b, 8); kv->f = v; break; }
    }
}
/* Skip one array value (elements of any type, strings included). */
static void skip_array(cur_t *c) {
    const uint32_t et = rd_u32(c);
    const uint64_t n = rd_u64(c);
    if (!c->ok) return;
    if (et == GT_STR) {
        for (uint64_t i = 0; i < n && c->ok; i++) {
            size_t l;
            rd_str(c, &l);
        }
        return;
    }
    const size_t es = scalar_size((int)et);
    if (!es || n > c->left / es) {
        c->ok = 0;
        return;
    }
    c->p += n * es;
    c->left -= n * es;
}

/* ---- open / close -------------------------------------------------------- */
void tbq_gguf_close(tbq_gguf *g) {
    if (!g) return;
    for (int i = 0; i < g->n_tensors; i++) {
        if (g->t[i].dev) tbq_free(g->t[i].dev);
        free(g->t[i].name);
    }
    for (int i = 0; i < g->n_owned; i++) tbq_free(g->owned[i]);
    for (int i = 0; i < g->n_kv; i++) free(g->kv[i].key);
    free(g->t);
    free(g->kv);
    free(g->owned);
    if (g->map) munmap((void *)g->map, g->size);
    if (g->fd >= 0) close(g->fd);
    free(g);
}

static tbq_gguf *open_fail(tbq_gguf *g) {
    tbq_gguf_close(g);
    return NULL;
}

tbq_gguf *tbq_gguf_open(const char *path) {
    tbq_gguf *g = (tbq_gguf *)calloc(1, sizeof *g);
    if (!g) return failf("tbq_gguf_open: out of memory"), NULL;
    g->fd = open(path, O_RDONLY);
    if (g->fd < 0) return failf("tbq_gguf_open: cannot open %s", path), open_fail(g);
    struct stat st;
    if (fstat(g->fd, &st) != 0 || st.st_size < 24)
        return failf("tbq_gguf_open: %s is not a GGUF file (too short)", path), open_fail(g);
    g->size = (size_t)st.st_size;
    void *m = mmap(NULL, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) return failf("tbq_gguf_open: mmap of %s failed", path), open_fail(g);
    g->map = (const uint8_t *)m;

    cur_t c = {g->map, g->size, 1};
    if (rd_u32(&c) != 0x46554747u) return failf("tbq_gguf_open: %s: bad magic", path), open_fail(g);
    g->version = rd_u32(&c);
    if (g->version < 2 || g->version > 3)
        return failf("tbq_gguf_open: %s: GGUF version %u not supported", path, g->version), open_fail(g);
    const uint64_t nt = rd_u64(&c), nkv = rd_u64(&c);
    /* every KV takes >= 12 bytes, every tensor info >= 24: counts the file cannot hold are corrupt */
    if (!c.ok || nkv > g->size / 12 || nt > g->size / 24)
        return failf("tbq_gguf_open: %s: implausible counts", path), open_fail(g);
    g->kv = (kv_t *)calloc(nkv ? nkv : 1, sizeof(kv_t));
    g->t = (tensor_t *)calloc(nt ? nt : 1, sizeof(tensor_t));
    if (!g->kv || !g->t) return failf("tbq_gguf_open: out of memory"), open_fail(g);

    uint64_t align = 32;
    for (uint64_t i = 0; i < nkv; i++) {
        kv_t *kv = &g->kv[i];
        size_t kl;
        const char *k = rd_str(&c, &kl);
        kv->type = (int)rd_u32(&c);
        if (!c.ok) break;
        kv->key = dup_str(k, kl);
        g->n_kv = (int)i + 1;
        if (kv->type == GT_STR) {
            kv->s = rd_str(&c, &kv->slen);
        } else if (kv->type == GT_ARR) {
            skip_array(&c);
        } else {
            rd_scalar(&c, kv->type, kv);
        }
        if (c.ok && kv->key && strcmp(kv->key, "general.alignment") == 0 && kv->type != GT_STR &&
            kv->type != GT_ARR && kv->type != GT_F32 && kv->type != GT_F64) {
            if (kv->i <= 0 || (kv->i & (kv->i - 1))) {
                failf("tbq_gguf_open: %s: general.alignment %lld is not a power of two", path, kv->i);
                return open_fail(g);
            }
            align = (uint64_t)kv->i;
        }
    }
    if (!c.ok) return failf("tbq_gguf_open: %s: truncated metadata", path), open_fail(g);

    for (uint64_t i = 0; i < nt; i++) {
        tensor_t *t = &g->t[i];
        size_t nl;
        const char *nm = rd_str(&c, &nl);
        const uint32_t nd = rd_u32(&c);
        if (!c.ok || nd < 1 || nd > 4) {
            failf("tbq_gguf_open: %s: tensor %llu: bad header", path, (unsigned long long)i);
            return open_fail(g);
        }
        t->name = dup_str(nm, nl);
        g->n_tensors = (int)i + 1;
        t->n_dims = (int)nd;
        for (int d = 0; d < 4; d++) t->dims[d] = 1;
        for (uint32_t d = 0; d < nd; d++) t->dims[d] = (long long)rd_u64(&c);
        t->qtype = (int)rd_u32(&c);
        t->offset = rd_u64(&c);
        if (!c.ok) break;
        long long rows = 1;
        int bad = t->dims[0] <= 0 || t->dims[0] > (1ll << 31);
        for (int d = 1; d < 4; d++) {
            bad |= t->dims[d] <= 0 || t->dims[d] > (1ll << 40) / rows;
            if (!bad) rows *= t->dims[d];
        }
        if (bad) {
            failf("tbq_gguf_open: %s: tensor %s: bad dims", path, t->name ? t->name : "?");
            return open_fail(g);
        }
        const size_t rb = tbq_row_bytes(t->qtype, (int)t->dims[0]);
        t->bytes = rb && (unsigned long long)rows <= SIZE_MAX / rb ? rb * (size_t)rows : 0;
    }
    if (!c.ok) return failf("tbq_gguf_open: %s: truncated tensor table", path), open_fail(g);
    const size_t hdr_end = g->size - c.left;
    g->data_off = (size_t)((hdr_end + align - 1) & ~(align - 1));
    for (int i = 0; i < g->n_tensors; i++) {
        const tensor_t *t = &g->t[i];
        if (t->bytes && (g->data_off > g->size || t->offset > g->size - g->data_off ||
                         t->bytes > g->size - g->data_off - t->offset)) {
            failf("tbq_gguf_open: %s: tensor %s extends past the end of the file", path, t->name);
            return open_fail(g);
        }
    }
    return g;
}

/* ---- lookups -------------------------------------------------------------- */
int tbq_gguf_n_tensors(const tbq_gguf *g) { return g ? g->n_tensors : 0; }

int tbq_gguf_find(const tbq_gguf *g, const char *name) {
    if (!g || !name) return -1;
    for (int i = 0; i < g->n_tensors; i++)
        if (g->t[i].name && strcmp(g->t[i].name, name) == 0) return i;
    return -1;
}

const char *tbq_gguf_tensor_name(const tbq_gguf *g, int i) {
    return g && i >= 0 && i < g->n_tensors ? g->t[i].name : NULL;
}

int tbq_gguf_tensor_info(const tbq_gguf *g, int i, int *qtype, int *n_dims, long long dims[4], size_t *bytes) {
    if (!g || i < 0 || i >= g->n_tensors) return failf("tbq_gguf_tensor_info: no tensor %d", i);
    const tensor_t *t = &g->t[i];
    if (qtype) *qtype = t->qtype;
    if (n_dims) *n_dims = t->n_dims;
    if (dims)
        for (int d = 0; d < 4; d++) dims[d] = t->dims[d];
    if (bytes) *bytes = t->bytes;
    return 1;
}

const void *tbq_gguf_tensor_host(const tbq_gguf *g, int i) {
    if (!g || i < 0 || i >= g->n_tensors || !g->t[i].bytes) return NULL;
    return g->map + g->data_off + g->t[i].offset;
}

static const kv_t *find_kv(const tbq_gguf *g, const char *key) {
    if (!g || !key) return NULL;
    for (int i = 0; i < g->n_kv; i++)
        if (g->kv[i].key && strcmp(g->kv[i].key, key) == 0) return &g->kv[i];
    return NULL;
}

int tbq_gguf_get_int(const tbq_gguf *g, const char *key, long long *out) {
    const kv_t *kv = find_kv(g, key);
    if (!kv || kv->type == GT_STR || kv->type == GT_ARR || kv->type == GT_F32 || kv->type == GT_F64)
        return failf("tbq_gguf: no integer key %s", key ? key : "(null)");
    *out = kv->i;
    return 1;
}

int tbq_gguf_get_float(const tbq_gguf *g, const char *key, double *out) {
    const kv_t *kv = find_kv(g, key);
    if (!kv || kv->type == GT_STR || kv->type == GT_ARR) return failf("tbq_gguf: no number key %s", key ? key : "(null)");
    *out = kv->type == GT_F32 || kv->type == GT_F64 ? kv->f : (double)kv->i;
    return 1;
}

int tbq_gguf_get_str(const tbq_gguf *g, const char *key, char *buf, size_t n) {
    const kv_t *kv = find_kv(g, key);
    if (!kv || kv->type != GT_STR || !buf || !n) return failf("tbq_gguf: no string key %s", key ? key : "(null)");
    const size_t l = kv->slen < n - 1 ? kv->slen : n - 1;
    memcpy(buf, kv->s, l);
    buf[l] = 0;
    return 1;
}

/* ---- device residency ------------------------------------------------------ */
static int upload(tbq_gguf *g, int i) {
    tensor_t *t = &g->t[i];
    if (t->dev) return 1;
    if (!t->bytes) return failf("tbq_gguf: tensor %s has qtype %d, unknown to libtbq", t->name, t->qtype);
    t->dev = tbq_malloc(t->bytes);
    if (!t->dev) return 0;
    if (!tbq_memcpy_h2d(t->dev, g->map + g->data_off + t->offset, t->bytes, NULL) || !tbq_stream_sync(NULL)) {
        tbq_free(t->dev);
        t->dev = NULL;
        return 0;
    }
    return 1;
}

int tbq_gguf_upload_all(tbq_gguf *g) {
    if (!g) return failf("tbq_gguf_upload_all: null handle"), -1;
    if (!tbq_init()) return -1;
    int n = 0;
    for (int i = 0; i < g->n_tensors; i++) {
        if (!g->t[i].bytes) continue;
        if (!upload(g, i)) return -1;
        n++;
    }
    return n;
}

const void *tbq_gguf_tensor_device(const tbq_gguf *g, int i) {
    return g && i >= 0 && i < g->n_tensors ? g->t[i].dev : NULL;
}

static void *own(tbq_gguf *g, size_t bytes) {
    if (g->n_owned == g->cap_owned) {
        const int cap = g->cap_owned ? 2 * g->cap_owned : 16;
        void **p = (void **)realloc(g->owned, (size_t)cap * sizeof(void *));
        if (!p) return failf("tbq_gguf: out of memory"), NULL;
        g->owned = p;
        g->cap_owned = cap;
    }
    void *d = tbq_malloc(bytes);
    if (d) g->owned[g->n_owned++] = d;
    return d;
}

/* Index of tensor `fmt` (printf-style name), with qtype and shape checked
 * (want_qt < 0 accepts any qtype; dims < 0 are not checked) and uploaded
 * unless dev is 0 (tensors that only go into a fused matrix). */
static int need(tbq_gguf *g, int dev, int want_qt, long long d0, long long d1, const char *fmt, ...) {
    char name[160];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(name, sizeof name, fmt, ap);
    va_end(ap);
    const int i = tbq_gguf_find(g, name);
    if (i < 0) return failf("tbq_gguf: tensor %s not in the file", name), -1;
    const tensor_t *t = &g->t[i];
    if (want_qt >= 0 && t->qtype != want_qt)
        return failf("tbq_gguf: tensor %s has qtype %d, expected %d", name, t->qtype, want_qt), -1;
    if ((d0 >= 0 && t->dims[0] != d0) || (d1 >= 0 && t->dims[1] != d1))
        return failf("tbq_gguf: tensor %s has shape %lld x %lld, expected %lld x %lld", name, t->dims[0], t->dims[1],
                     d0, d1), -1;
    if (!t->bytes) return failf("tbq_gguf: tensor %s has qtype %d, unknown to libtbq", name, t->qtype), -1;
    if (dev && !upload(g, i)) return -1;
    return i;
}

/* One device matrix holding the rows of tensors a, b (and c) in order. */
static void *fuse(tbq_gguf *g, int a, int b, int c) {
    const size_t n = g->t[a].bytes + g->t[b].bytes + (c >= 0 ? g->t[c].bytes : 0);
    unsigned char *d = (unsigned char *)own(g, n);
    if (!d) return NULL;
    size_t off = 0;
    const int ids[3] = {a, b, c};
    for (int k = 0; k < 3; k++) {
        if (ids[k] < 0) continue;
        if (!tbq_memcpy_h2d(d + off, g->map + g->data_off + g->t[ids[k]].offset, g->t[ids[k]].bytes, NULL)) return NULL;
        off += g->t[ids[k]].bytes;
    }
    return tbq_stream_sync(NULL) ? d : NULL;
}

static int arch_of(const tbq_gguf *g, char *arch, size_t n) {
    return tbq_gguf_get_str(g, "general.architecture", arch, n);
}

static int arch_int(const tbq_gguf *g, const char *arch, const char *suffix, long long *out, long long dflt, int required) {
    char key[128];
    snprintf(key, sizeof key, "%s.%s", arch, suffix);
    if (tbq_gguf_get_int(g, key, out)) return 1;
    if (required) return failf("tbq_gguf: metadata %s missing", key);
    *out = dflt;
    return 1;
}

static double arch_float(const tbq_gguf *g, const char *arch, const char *suffix, double dflt) {
    char key[128];
    double v;
    snprintf(key, sizeof key, "%s.%s", arch, suffix);
    return tbq_gguf_get_float(g, key, &v) ? v : dflt;
}

int tbq_gguf_set_layout(tbq_gguf *g, int layout) {
    if (!g || (layout != 0 && layout != TBQ_GGML)) return failf("tbq_gguf_set_layout: layout must be 0 or TBQ_GGML");
    g->layout = layout;
    return 1;
}

/* The qtype id an assembled model or layer carries for file qtype qt: the
 * file's ggml id, with TBQ_GGML added when the handle reads ggml's layouts
 * (F32 stays 0, which the dense model's qt_* fields reserve for "the
 * model's qtype_layers"; it reads the same in both layouts). */
static int lq(const tbq_gguf *g, int qt) { return qt == 0 ? 0 : (qt | g->layout); }

int tbq_gguf_dense_model(tbq_gguf *g, int max_ctx, tbq_dense_model *m, tbq_dense_layer *layers, int n_layers) {
    if (!g || !m || !layers || max_ctx <= 0) return failf("tbq_gguf_dense_model: bad arguments");
    if (!tbq_init()) return 0;
    char arch[64];
    if (!arch_of(g, arch, sizeof arch)) return 0;
    long long L, H, NQ, NKV, D, F;
    if (!arch_int(g, arch, "block_count", &L, 0, 1) || !arch_int(g, arch, "embedding_length", &H, 0, 1) ||
        !arch_int(g, arch, "attention.head_count", &NQ, 0, 1) ||
        !arch_int(g, arch, "attention.head_count_kv", &NKV, NQ, 0) ||
        !arch_int(g, arch, "attention.key_length", &D, NQ > 0 ? H / NQ : 0, 0) ||
        !arch_int(g, arch, "feed_forward_length", &F, 0, 1))
        return 0;
    if (L != n_layers) return failf("tbq_gguf_dense_model: the file has %lld layers, the array %d", L, n_layers);
    const int te = tbq_gguf_find(g, "token_embd.weight");
    if (te < 0) return failf("tbq_gguf: tensor token_embd.weight not in the file");
    const int out_i = tbq_gguf_find(g, "output.weight");
    const int head = out_i >= 0 ? out_i : te;   /* tied lm_head, as layer4/tb_infer.c:1019-1020 */
    const int qe = g->t[te].qtype;
    const long long V = g->t[te].dims[1];
    if (g->t[te].dims[0] != H || g->t[head].dims[0] != H || g->t[head].dims[1] != V || g->t[head].qtype != qe)
        return failf("tbq_gguf_dense_model: token_embd / output shapes or qtypes disagree");
    int on = need(g, 1, 0, H, -1, "output_norm.weight");
    if (on < 0 || !upload(g, te) || !upload(g, head)) return 0;
    int qt = -1;   /* the model's qtype_layers: layer 0's attn_q */
    for (int l = 0; l < n_layers; l++) {
        const int iq = need(g, 0, -1, H, NQ * D, "blk.%d.attn_q.weight", l);
        const int ik = need(g, 0, -1, H, NKV * D, "blk.%d.attn_k.weight", l);
        const int iv = need(g, 0, -1, H, NKV * D, "blk.%d.attn_v.weight", l);
        const int io = need(g, 1, -1, NQ * D, H, "blk.%d.attn_output.weight", l);
        const int ig = need(g, 0, -1, H, F, "blk.%d.ffn_gate.weight", l);
        const int iu = need(g, 0, -1, H, F, "blk.%d.ffn_up.weight", l);
        const int id = need(g, 1, -1, F, H, "blk.%d.ffn_down.weight", l);
        const int ian = need(g, 1, 0, H, -1, "blk.%d.attn_norm.weight", l);
        const int iqn = need(g, 1, 0, D, -1, "blk.%d.attn_q_norm.weight", l);
        const int ikn = need(g, 1, 0, D, -1, "blk.%d.attn_k_norm.weight", l);
        const int ifn = need(g, 1, 0, H, -1, "blk.%d.ffn_norm.weight", l);
        if (iq < 0 || ik < 0 || iv < 0 || io < 0 || ig < 0 || iu < 0 || id < 0 || ian < 0 || iqn < 0 || ikn < 0 ||
            ifn < 0)
            return 0;
        if (qt < 0) qt = g->t[iq].qtype;
        /* a qt_* field of 0 means qtype_layers, so an F32 matrix needs qtype_layers F32 */
        const int mats[7] = {iq, ik, iv, io, ig, iu, id};
        for (int k = 0; k < 7; k++)
            if (g->t[mats[k]].qtype == 0 && qt != 0)
                return failf("tbq_gguf_dense_model: %s is F32 among quantised layer matrices", g->t[mats[k]].name);
        tbq_dense_layer *ly = &layers[l];
        memset(ly, 0, sizeof *ly);
        ly->attn_norm = (const float *)g->t[ian].dev;
        ly->q_norm = (const float *)g->t[iqn].dev;
        ly->k_norm = (const float *)g->t[ikn].dev;
        ly->ffn_norm = (const float *)g->t[ifn].dev;
        ly->wo = g->t[io].dev;
        ly->qt_o = lq(g, g->t[io].qtype);
        ly->wdown = g->t[id].dev;
        ly->qt_down = lq(g, g->t[id].qtype);
        /* one fused device matrix where the rows share a qtype, else the
         * separate matrices (one launch each) */
        if (g->t[iq].qtype == g->t[ik].qtype && g->t[iq].qtype == g->t[iv].qtype) {
            if (!(ly->wqkv = fuse(g, iq, ik, iv))) return 0;
            ly->qt_qkv = lq(g, g->t[iq].qtype);
        } else {
            if (!upload(g, iq) || !upload(g, ik) || !upload(g, iv)) return 0;
            ly->wq = g->t[iq].dev;
            ly->wk = g->t[ik].dev;
            ly->wv = g->t[iv].dev;
            ly->qt_q = lq(g, g->t[iq].qtype);
            ly->qt_k = lq(g, g->t[ik].qtype);
            ly->qt_v = lq(g, g->t[iv].qtype);
        }
        if (g->t[ig].qtype == g->t[iu].qtype) {
            if (!(ly->wgu = fuse(g, ig, iu, -1))) return 0;
            ly->qt_gu = lq(g, g->t[ig].qtype);
        } else {
            if (!upload(g, ig) || !upload(g, iu)) return 0;
            ly->wgate = g->t[ig].dev;
            ly->wup = g->t[iu].dev;
            ly->qt_gate = lq(g, g->t[ig].qtype);
            ly->qt_up = lq(g, g->t[iu].qtype);
        }
    }
    const size_t kv_bytes = (size_t)L * (size_t)NKV * (size_t)max_ctx * (size_t)D * 4;
    float *kc = (float *)own(g, kv_bytes), *vc = (float *)own(g, kv_bytes);
    if (!kc || !vc) return 0;
    memset(m, 0, sizeof *m);
    m->n_layers = (int)L;
    m->hidden = (int)H;
    m->n_heads = (int)NQ;
    m->n_kv_heads = (int)NKV;
    m->head_dim = (int)D;
    m->ffn = (int)F;
    m->vocab = (int)V;
    m->max_ctx = max_ctx;
    m->norm_eps = (float)arch_float(g, arch, "attention.layer_norm_rms_epsilon", 1e-6);
    m->rope_theta = (float)arch_float(g, arch, "rope.freq_base", 10000.0);
    m->qtype_layers = lq(g, qt);
    m->qtype_embd = lq(g, qe);
    m->tok_embd = g->t[te].dev;
    m->lm_head = g->t[head].dev;
    m->output_norm = (const float *)g->t[on].dev;
    m->layers = layers;
    m->k_cache = kc;
    m->v_cache = vc;
    return tbq_dense_workspace_size(m) > 0;   /* validates the shape */
}

/* One device matrix holding the rows of tensors ids[0..n) in order. */
static void *fuse_n(tbq_gguf *g, const int *ids, int n) {
    size_t total = 0;
    for (int k = 0; k < n; k++) total += g->t[ids[k]].bytes;
    unsigned char *d = (unsigned char *)own(g, total);
    if (!d) return NULL;
    size_t off = 0;
    for (int k = 0; k < n; k++) {
        const tensor_t *t = &g->t[ids[k]];
        if (!tbq_memcpy_h2d(d + off, g->map + g->data_off + t->offset, t->bytes, NULL)) return NULL;
        off += t->bytes;
    }
    return tbq_stream_sync(NULL) ? d : NULL;
}

/* The E per-expert tensors blk.<layer>.ffn_<kind>.<e>.weight (d0 x d1 each,
 * one qtype) as one packed device matrix of E * d1 rows; *qt gets their
 * qtype. */
static const void *split_experts(tbq_gguf *g, int layer, const char *kind, long long E, long long d0, long long d1,
                                 int *qt) {
    int ids[256];
    for (long long e = 0; e < E; e++) {
        ids[e] = need(g, 0, e ? *qt : -1, d0, d1, "blk.%d.ffn_%s.%lld.weight", layer, kind, e);
        if (ids[e] < 0) return NULL;
        if (!e) *qt = g->t[ids[0]].qtype;
    }
    return fuse_n(g, ids, (int)E);
}

int tbq_gguf_moe_layer(tbq_gguf *g, int layer, tbq_moe_layer *Lout) {
    if (!g || !Lout) return failf("tbq_gguf_moe_layer: bad arguments");
    if (!tbq_init()) return 0;
    char arch[64];
    if (!arch_of(g, arch, sizeof arch)) return 0;
    long long H, E, K, F;
    if (!arch_int(g, arch, "embedding_length", &H, 0, 1) || !arch_int(g, arch, "expert_count", &E, 0, 1) ||
        !arch_int(g, arch, "expert_used_count", &K, 0, 1))
        return 0;
    if (E <= 0 || E > 256) return failf("tbq_gguf_moe_layer: expert_count %lld outside 1..256", E);
    const int ir = need(g, 1, 0, H, E, "blk.%d.ffn_gate_inp.weight", layer);
    if (ir < 0) return 0;
    char name[160];
    snprintf(name, sizeof name, "blk.%d.ffn_gate_exps.weight", layer);
    const void *dg, *du, *dd;
    int qg, qu, qd;
    if (tbq_gguf_find(g, name) >= 0) {
        /* packed: blk.N.ffn_{gate,up,down}_exps, each tensor in its own qtype
         * (layer4/tb_infer.c:780-816) */
        const int ig = need(g, 1, -1, H, -1, "blk.%d.ffn_gate_exps.weight", layer);
        if (ig < 0) return 0;
        F = g->t[ig].dims[1];
        const int iu = need(g, 1, -1, H, F, "blk.%d.ffn_up_exps.weight", layer);
        const int id = need(g, 1, -1, F, H, "blk.%d.ffn_down_exps.weight", layer);
        if (iu < 0 || id < 0) return 0;
        if (g->t[ig].dims[2] != E || g->t[iu].dims[2] != E || g->t[id].dims[2] != E)
            return failf("tbq_gguf_moe_layer: expert tensors of layer %d do not hold %lld experts", layer, E);
        dg = g->t[ig].dev;
        du = g->t[iu].dev;
        dd = g->t[id].dev;
        qg = g->t[ig].qtype;
        qu = g->t[iu].qtype;
        qd = g->t[id].qtype;
    } else {
        /* split: blk.N.ffn_{gate,up,down}.<e>.weight, the reference's
         * fallback (layer4/tb_infer.c:783-791), packed here into the same
         * device layout */
        const int i0 = need(g, 0, -1, H, -1, "blk.%d.ffn_gate.0.weight", layer);
        if (i0 < 0) return failf("tbq_gguf_moe_layer: layer %d has neither ffn_gate_exps nor ffn_gate.0", layer);
        F = g->t[i0].dims[1];
        if (!(dg = split_experts(g, layer, "gate", E, H, F, &qg)) || !(du = split_experts(g, layer, "up", E, H, F, &qu)) ||
            !(dd = split_experts(g, layer, "down", E, F, H, &qd)))
            return 0;
    }
    memset(Lout, 0, sizeof *Lout);
    Lout->H = (int)H;
    Lout->F = (int)F;
    Lout->E = (int)E;
    Lout->top_k = (int)K;
    Lout->qtype = lq(g, qg);
    Lout->qt_gate = lq(g, qg);
    Lout->qt_up = lq(g, qu);
    Lout->qt_down = lq(g, qd);
    Lout->router = (const float *)g->t[ir].dev;
    Lout->bias = NULL;
    Lout->gate = dg;
    Lout->up = du;
    Lout->down = dd;
    return 1;
}
