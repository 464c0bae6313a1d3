/* sf37_gguf.c - GGUF weight residency for the _mapped entry points.
 *
 * Reads the GGUF v3 container the engine maps (header, key/value section,
 * tensor table, aligned data section; the reader of sf37.c:506-604) and
 * binds one MoE layer's tensors by the engine's tensor contract
 * (sf37.c:1760-1782): router `moe.gate.weight` (F32, BF16 or Q8_0 as stored,
 * F16 widened exactly to F32), `moe.router_bias` (F32), `moe.gate_proj` /
 * `moe.up_proj` (Q3GU, type 11), `moe.down_proj` (Q2D, type 10),
 * `share_expert.*_proj` (Q8_0; or Q3GU gate/up and Q2D down) and
 * `post_attention_layernorm.weight` (BF16).  The weights become
 * device-resident copies of their map ranges (the same registry the _mapped
 * calls resolve against), so a bound layer runs through sf37_hip_moe_layer /
 * sf37_hip_moe_block with the map as its model map.  Closing a handle that
 * mapped the file itself also drops the device copies of that mapping.
 */
#include <errno.h>
#include <fcntl.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "../../include/sf37_hip.h"

sf37_hip_tensor *sf37i_map_tensor(const void *model_map, uint64_t model_size, uint64_t offset, uint64_t bytes,
                                  const char *label, int *held, uint64_t *range_off, uint64_t *range_bytes);
void sf37i_drop_range(const void *model_map, uint64_t offset, uint64_t bytes);
void sf37i_drop_map(const void *model_map);

enum { GG_F32 = 0, GG_F16 = 1, GG_Q8_0 = 8, GG_Q2D = 10, GG_Q3GU = 11, GG_BF16 = 30 };
enum { GV_U8, GV_I8, GV_U16, GV_I16, GV_U32, GV_I32, GV_F32, GV_BOOL, GV_STR, GV_ARR, GV_U64, GV_I64, GV_F64 };
#define GG_MAX_DIMS 4

typedef struct {
    char *name;
    uint32_t ndim, type;
    uint64_t dim[GG_MAX_DIMS];
    uint64_t offset, bytes;   /* absolute in the map */
} gg_tensor;

struct sf37_hip_gguf {
    const uint8_t *map;
    uint64_t size;
    int fd;            /* >= 0 when the file was opened (and mapped) here */
    uint32_t version, alignment;
    uint64_t n_tensors;
    gg_tensor *t;
    sf37_hip_tensor **owned;   /* handles given out by the binder (8 per bound layer) */
    uint32_t n_owned, cap_owned;
    uint64_t (*made)[2];       /* holds this handle has on binder-made ranges: offset, bytes */
    uint32_t n_made, cap_made;
};

typedef struct {
    const uint8_t *p;
    uint64_t size, pos;
    int ok;
} gg_cur;

static int cur_need(gg_cur *c, uint64_t n) {
    if (!c->ok || n > c->size - c->pos) c->ok = 0;
    return c->ok;
}
static uint64_t cur_u(gg_cur *c, int bytes) {
    uint64_t v = 0;
    if (!cur_need(c, (uint64_t)bytes)) return 0;
    memcpy(&v, c->p + c->pos, (size_t)bytes);   /* little-endian host */
    c->pos += (uint64_t)bytes;
    return v;
}
static void cur_str(gg_cur *c, const uint8_t **s, uint64_t *len) {
    *len = cur_u(c, 8);
    *s = NULL;
    if (cur_need(c, *len)) {
        *s = c->p + c->pos;
        c->pos += *len;
    }
}
static void cur_skip_value(gg_cur *c, uint32_t type, int depth) {
    static const uint8_t fixed[] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
    if (type == GV_STR) {
        const uint8_t *s;
        uint64_t len;
        cur_str(c, &s, &len);
    } else if (type == GV_ARR) {
        const uint32_t et = (uint32_t)cur_u(c, 4);
        const uint64_t n = cur_u(c, 8);
        if (depth > 2 || et > GV_F64) {
            c->ok = 0;
            return;
        }
        if (et != GV_STR && et != GV_ARR) {
            if (fixed[et] && n > (c->size - c->pos) / fixed[et]) c->ok = 0;
            else c->pos += n * fixed[et];
        } else {
            for (uint64_t i = 0; i < n && c->ok; i++) cur_skip_value(c, et, depth + 1);
        }
    } else if (type <= GV_F64) {
        if (cur_need(c, fixed[type])) c->pos += fixed[type];
    } else {
        c->ok = 0;
    }
}

/* Bytes of a tensor of this type and shape, 0 if unsupported (sf37.c:463-471). */
static uint64_t gg_nbytes(uint32_t type, const uint64_t *dim, uint32_t ndim) {
    uint64_t block, bsize, n = 1;
    switch (type) {
        case GG_F32: block = 1; bsize = 4; break;
        case GG_F16: case GG_BF16: block = 1; bsize = 2; break;
        case GG_Q8_0: block = 32; bsize = 34; break;
        case GG_Q2D: block = 256; bsize = 84; break;
        case GG_Q3GU: block = 256; bsize = 110; break;
        default: return 0;
    }
    for (uint32_t i = 0; i < ndim; i++) {
        if (dim[i] == 0 || n > UINT64_MAX / dim[i]) return 0;
        n *= dim[i];
    }
    if (dim[0] % block) return 0;
    return n / block * bsize;
}

static void gg_free(sf37_hip_gguf *g) {
    if (!g) return;
    for (uint32_t i = 0; i < g->n_owned; i++) sf37_hip_tensor_free(g->owned[i]);
    free(g->owned);
    /* a caller's map outlives the handle: give back this handle's holds (a
     * range another open handle still holds stays) */
    if (g->fd < 0)
        for (uint32_t i = 0; i < g->n_made; i++) sf37i_drop_range(g->map, g->made[i][0], g->made[i][1]);
    free(g->made);
    for (uint64_t i = 0; g->t && i < g->n_tensors; i++) free(g->t[i].name);
    free(g->t);
    if (g->fd >= 0) {
        /* the device copies are keyed by the map address, which a later
         * mapping may reuse: drop them with the mapping */
        sf37i_drop_map(g->map);
        munmap((void *)g->map, (size_t)g->size);
        close(g->fd);
    }
    free(g);
}

static sf37_hip_gguf *gg_fail(sf37_hip_gguf *g, const char *what) {
    fprintf(stderr, "sf37_hip gguf: %s\n", what);
    gg_free(g);
    return NULL;
}

sf37_hip_gguf *sf37_hip_gguf_from_map(const void *map, uint64_t size) {
    if (!map || size < 24) return gg_fail(NULL, "no map or shorter than a GGUF header");
    sf37_hip_gguf *g = (sf37_hip_gguf *)calloc(1, sizeof(*g));
    if (!g) return NULL;
    g->map = (const uint8_t *)map;
    g->size = size;
    g->fd = -1;
    g->alignment = 32;
    gg_cur c = {g->map, size, 0, 1};
    if (memcmp(g->map, "GGUF", 4) != 0) return gg_fail(g, "not a GGUF file (magic)");
    c.pos = 4;
    g->version = (uint32_t)cur_u(&c, 4);
    g->n_tensors = cur_u(&c, 8);
    const uint64_t n_kv = cur_u(&c, 8);
    if (!c.ok) return gg_fail(g, "truncated header");
    if (g->version != 3) return gg_fail(g, "unsupported GGUF version (3 is read)");
    for (uint64_t i = 0; i < n_kv && c.ok; i++) {
        const uint8_t *key;
        uint64_t klen;
        cur_str(&c, &key, &klen);
        const uint32_t type = (uint32_t)cur_u(&c, 4);
        if (c.ok && type == GV_U32 && klen == 17 && !memcmp(key, "general.alignment", 17)) {
            gg_cur tmp = c;
            const uint32_t a = (uint32_t)cur_u(&tmp, 4);
            if (tmp.ok && a) g->alignment = a;
        }
        cur_skip_value(&c, type, 0);
    }
    if (!c.ok) return gg_fail(g, "truncated or malformed key/value section");
    if (g->n_tensors > (size - c.pos) / 24) return gg_fail(g, "tensor count exceeds the file");
    g->t = (gg_tensor *)calloc(g->n_tensors ? g->n_tensors : 1, sizeof(gg_tensor));
    if (!g->t) return gg_fail(g, "out of memory");
    for (uint64_t i = 0; i < g->n_tensors; i++) {
        gg_tensor *t = &g->t[i];
        const uint8_t *name;
        uint64_t nlen;
        cur_str(&c, &name, &nlen);
        t->ndim = (uint32_t)cur_u(&c, 4);
        if (!c.ok || t->ndim == 0 || t->ndim > GG_MAX_DIMS) return gg_fail(g, "malformed tensor entry");
        for (uint32_t d = 0; d < t->ndim; d++) t->dim[d] = cur_u(&c, 8);
        t->type = (uint32_t)cur_u(&c, 4);
        t->offset = cur_u(&c, 8);
        if (!c.ok) return gg_fail(g, "truncated tensor table");
        t->name = (char *)malloc(nlen + 1);
        if (!t->name) return gg_fail(g, "out of memory");
        memcpy(t->name, name, nlen);
        t->name[nlen] = 0;
        t->bytes = gg_nbytes(t->type, t->dim, t->ndim);   /* 0: a type the MoE path does not read */
    }
    const uint64_t a = g->alignment;
    const uint64_t data = (c.pos + a - 1) / a * a;
    for (uint64_t i = 0; i < g->n_tensors; i++) {
        gg_tensor *t = &g->t[i];
        if (t->offset > UINT64_MAX - data) return gg_fail(g, "tensor offset overflows");
        t->offset += data;
        if (t->offset > size || t->bytes > size - t->offset) return gg_fail(g, "tensor points outside the file");
    }
    return g;
}

sf37_hip_gguf *sf37_hip_gguf_open(const char *path) {
    if (!path) return NULL;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) {
        fprintf(stderr, "sf37_hip gguf: open %s: %s\n", path, strerror(errno));
        return NULL;
    }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        close(fd);
        return gg_fail(NULL, "cannot stat the file or it is too small");
    }
    void *m = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (m == MAP_FAILED) {
        close(fd);
        return gg_fail(NULL, "mmap failed");
    }
    sf37_hip_gguf *g = sf37_hip_gguf_from_map(m, (uint64_t)st.st_size);
    if (!g) {
        munmap(m, (size_t)st.st_size);
        close(fd);
        return NULL;
    }
    g->fd = fd;
    return g;
}

void sf37_hip_gguf_close(sf37_hip_gguf *g) { gg_free(g); }

const void *sf37_hip_gguf_map(const sf37_hip_gguf *g, uint64_t *size) {
    if (!g) return NULL;
    if (size) *size = g->size;
    return g->map;
}

static const gg_tensor *gg_find(const sf37_hip_gguf *g, const char *name) {
    for (uint64_t i = 0; i < g->n_tensors; i++)
        if (!strcmp(g->t[i].name, name)) return &g->t[i];
    return NULL;
}

int sf37_hip_gguf_tensor(const sf37_hip_gguf *g, const char *name, uint64_t *offset, uint64_t *bytes,
                         uint32_t *type, uint32_t *ndim, uint64_t *dims) {
    if (!g || !name) return 0;
    const gg_tensor *t = gg_find(g, name);
    if (!t) return 0;
    if (offset) *offset = t->offset;
    if (bytes) *bytes = t->bytes;
    if (type) *type = t->type;
    if (ndim) *ndim = t->ndim;
    if (dims)
        for (uint32_t d = 0; d < GG_MAX_DIMS; d++) dims[d] = d < t->ndim ? t->dim[d] : 1;
    return 1;
}

/* Tensor il.<suffix> with the given type (type < 0: any) and rank. */
static const gg_tensor *gg_req(const sf37_hip_gguf *g, uint32_t il, const char *suffix, int type, uint32_t ndim) {
    char name[192];
    snprintf(name, sizeof(name), "model.layers.%u.%s", il, suffix);
    const gg_tensor *t = gg_find(g, name);
    if (!t) fprintf(stderr, "sf37_hip gguf: missing tensor %s\n", name);
    else if ((type >= 0 && t->type != (uint32_t)type) || t->ndim != ndim || !t->bytes) {
        fprintf(stderr, "sf37_hip gguf: tensor %s has type %u / rank %u\n", name, t->type, t->ndim);
        t = NULL;
    }
    return t;
}

static sf37_hip_tensor *gg_keep(sf37_hip_gguf *g, sf37_hip_tensor *t) {
    if (!t) return NULL;
    if (g->n_owned == g->cap_owned) {
        const uint32_t cap = g->cap_owned ? 2u * g->cap_owned : 64u;
        sf37_hip_tensor **n = (sf37_hip_tensor **)realloc(g->owned, cap * sizeof(*n));
        if (!n) {
            sf37_hip_tensor_free(t);
            fprintf(stderr, "sf37_hip gguf: out of memory for bound tensors\n");
            return NULL;
        }
        g->owned = n;
        g->cap_owned = cap;
    }
    g->owned[g->n_owned++] = t;
    return t;
}

/* Device-resident tensor over a registered range: sf37_hip_evict_model_cache
 * leaves it alone; the range lives while some handle holds it. */
static sf37_hip_tensor *gg_resident(sf37_hip_gguf *g, const gg_tensor *t) {
    int held = 0;
    uint64_t roff = 0, rbytes = 0;
    sf37_hip_tensor *d = sf37i_map_tensor(g->map, g->size, t->offset, t->bytes, t->name, &held, &roff, &rbytes);
    if (d && held) {
        if (g->n_made == g->cap_made) {
            const uint32_t cap = g->cap_made ? 2u * g->cap_made : 64u;
            uint64_t(*n)[2] = (uint64_t(*)[2])realloc(g->made, cap * sizeof(*n));
            if (!n) {
                sf37_hip_tensor_free(d);
                sf37i_drop_range(g->map, roff, rbytes);
                return NULL;
            }
            g->made = n;
            g->cap_made = cap;
        }
        g->made[g->n_made][0] = roff;
        g->made[g->n_made][1] = rbytes;
        g->n_made++;
    }
    return gg_keep(g, d);
}

/* Router rows: F32, BF16 and Q8_0 stay resident as stored (the layer reads
 * each type, *type set to it); F16 is widened to F32 on the host (exact). */
static sf37_hip_tensor *gg_router(sf37_hip_gguf *g, const gg_tensor *t, uint32_t *type) {
    *type = t->type == GG_F16 ? (uint32_t)GG_F32 : t->type;
    if (t->type == GG_F32 || t->type == GG_BF16 || t->type == GG_Q8_0) return gg_resident(g, t);
    if (t->type != GG_F16) {
        fprintf(stderr, "sf37_hip gguf: router type %u (F32, BF16, F16 or Q8_0 are read)\n", t->type);
        return NULL;
    }
    const uint64_t n = t->bytes / 2;
    float *f = (float *)malloc(n * 4);
    if (!f) return NULL;
    const uint16_t *h = (const uint16_t *)(g->map + t->offset);
    for (uint64_t i = 0; i < n; i++) {   /* IEEE half -> single */
        uint32_t bits;
        const uint32_t s = (uint32_t)(h[i] & 0x8000u) << 16, e = (h[i] >> 10) & 0x1fu, m = h[i] & 0x3ffu;
        if (e == 0x1fu) bits = s | 0x7f800000u | (m << 13);
        else if (e) bits = s | ((e + 112u) << 23) | (m << 13);
        else if (!m) bits = s;
        else {
            uint32_t ee = 113u, mm = m;
            while (!(mm & 0x400u)) { mm <<= 1; ee--; }
            bits = s | (ee << 23) | ((mm & 0x3ffu) << 13);
        }
        memcpy(&f[i], &bits, 4);
    }
    sf37_hip_tensor *d = sf37_hip_tensor_alloc(n * 4);
    const int ok = d && sf37_hip_tensor_write(d, 0, f, n * 4);
    free(f);
    if (!ok) {
        sf37_hip_tensor_free(d);
        return NULL;
    }
    return gg_keep(g, d);
}

int sf37_hip_gguf_bind_moe_layer(sf37_hip_gguf *g, uint32_t il, sf37_hip_moe_layer_weights *w,
                                 uint64_t *post_norm_offset) {
    if (!g || !w) return 0;
    const gg_tensor *rt = gg_req(g, il, "moe.gate.weight", -1, 2);
    const gg_tensor *rb = gg_req(g, il, "moe.router_bias", GG_F32, 1);
    const gg_tensor *ga = gg_req(g, il, "moe.gate_proj.weight", GG_Q3GU, 3);
    const gg_tensor *up = gg_req(g, il, "moe.up_proj.weight", GG_Q3GU, 3);
    const gg_tensor *dn = gg_req(g, il, "moe.down_proj.weight", GG_Q2D, 3);
    /* the shared expert: Q8_0 (the engine's contract), or Q3GU gate/up with a
     * Q2D down (the benchmark configurations' "same formats" option) */
    const gg_tensor *sg = gg_req(g, il, "share_expert.gate_proj.weight", -1, 2);
    const gg_tensor *su = gg_req(g, il, "share_expert.up_proj.weight", -1, 2);
    const gg_tensor *sd = gg_req(g, il, "share_expert.down_proj.weight", -1, 2);
    const gg_tensor *pn = gg_req(g, il, "post_attention_layernorm.weight", GG_BF16, 1);
    if (!rt || !rb || !ga || !up || !dn || !sg || !su || !sd || !pn) return 0;
    const int sh_q8 = sg->type == GG_Q8_0 && su->type == GG_Q8_0 && sd->type == GG_Q8_0;
    const int sh_q3 = sg->type == GG_Q3GU && su->type == GG_Q3GU && sd->type == GG_Q2D;
    if (!sh_q8 && !sh_q3) {
        fprintf(stderr, "sf37_hip gguf: layer %u shared expert types %u/%u/%u (Q8_0, or Q3GU with a Q2D down)\n", il,
                sg->type, su->type, sd->type);
        return 0;
    }
    /* GGUF dims are (columns, rows[, experts]): gate/up (D, F, E), down (F, D, E) */
    const uint64_t D = ga->dim[0], F = ga->dim[1], E = ga->dim[2];
    if (up->dim[0] != D || up->dim[1] != F || up->dim[2] != E || dn->dim[0] != F || dn->dim[1] != D ||
        dn->dim[2] != E || rt->dim[0] != D || rt->dim[1] != E || rb->dim[0] != E || sg->dim[0] != D ||
        sg->dim[1] != F || su->dim[0] != D || su->dim[1] != F || sd->dim[0] != F || sd->dim[1] != D ||
        pn->dim[0] != D || D > 0xffffffffu || F > 0xffffffffu || E > 0xffffffffu) {
        fprintf(stderr, "sf37_hip gguf: layer %u MoE tensor shapes disagree\n", il);
        return 0;
    }
    memset(w, 0, sizeof(*w));
    w->router = gg_router(g, rt, &w->router_type);
    w->shared_type = sh_q3 ? (uint32_t)GG_Q3GU : 0u;
    w->router_bias = gg_resident(g, rb);
    w->gate = gg_resident(g, ga);
    w->up = gg_resident(g, up);
    w->down = gg_resident(g, dn);
    w->sh_gate = gg_resident(g, sg);
    w->sh_up = gg_resident(g, su);
    w->sh_down = gg_resident(g, sd);
    if (!w->router || !w->router_bias || !w->gate || !w->up || !w->down || !w->sh_gate || !w->sh_up || !w->sh_down)
        return 0;
    w->n_expert = (uint32_t)E;
    w->topk = 8;                                   /* SF37_EXPERT_USED, sf37.c:45 */
    w->in_dim = (uint32_t)D;
    w->mid_dim = (uint32_t)F;
    w->scale = 3.0f;                               /* routed weight scale, sf37.c:2157 */
    w->clamp_routed = (il == 43u || il == 44u) ? 7.0f : 0.0f;    /* sf37.c:2103-2106 */
    w->clamp_shared = (il == 43u || il == 44u) ? 16.0f : 0.0f;
    if (post_norm_offset) *post_norm_offset = pn->offset;
    return 1;
}
