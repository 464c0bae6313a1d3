/*
 * sf37_hip.c - host side of the MI355X MoE backend: the C ABI declared in
 * include/sf37_hip.h.  Argument checks follow the reference backend
 * (sf37_cuda.cu, cited per function) and run before any launch; kernels
 * live in the .hip files and are reached through sf37_launch.h.
 *
 * Device buffers: every allocation made here carries SF37_PAD bytes of
 * slack past its end, because the weight-block kernels read whole dwords
 * around blocks that end on a 2-byte boundary.
 */
#define __HIP_PLATFORM_AMD__ 1
#include <hip/hip_runtime_api.h>

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/sf37_hip.h"
#include "sf37_launch.h"

#define SF37_PAD 256u
#define QK SF37_HIP_QK_K
#define Q3B SF37_HIP_Q3_BLOCK_SIZE
#define Q2B SF37_HIP_Q2_BLOCK_SIZE
#define Q8B SF37_HIP_Q8_0_BLOCK_SIZE
#define Q8KB SF37_HIP_Q8K_BLOCK_SIZE

struct sf37_hip_tensor {
    void *ptr;
    uint64_t bytes;
    int owned;
};

/* ------------------------------------------------------------------------ */
/* state                                                                     */
/* ------------------------------------------------------------------------ */

static int g_init;
static hipStream_t g_stream;
static void *g_scratch;
static uint64_t g_scratch_bytes;
static int g_model_fd = -1;

#define N_LAYER_BUFS 12
static sf37_hip_tensor *g_layer_bufs[N_LAYER_BUFS];
static uint64_t g_layer_buf_bytes[N_LAYER_BUFS];

static int64_t g_opt_q8k = 1;
static int64_t g_opt_q8k_min_rows = 512;
static int64_t g_opt_write_gate_up = 0;
static int64_t g_opt_decode = 1;
static int64_t g_opt_router_always = 0;
static int64_t g_opt_up_dyn_pct = -1, g_opt_up_wgs = 0, g_opt_dn_wgs = 0, g_opt_upsel_max_tok = 1;
static int64_t g_opt_down_combine = 1;
static int64_t g_opt_prefill = 1;
static int64_t g_opt_prefill_min_pairs = 256;
static int64_t g_opt_shared_min_tok = 64;
static int64_t g_opt_shared_stream = 1;
static int64_t g_opt_shared_slot = 1;
/* the shared expert's side stream (default priority) and its fork / join
 * events, made on first use */
static hipStream_t g_side;
static hipEvent_t g_ev_fork, g_ev_join;

/* arrival counters of the fused decode kernels: zeroed once, left zero by
 * every completed launch */
static uint32_t *g_dec_cnt;
static uint64_t g_dec_cnt_words;

typedef struct {
    const uint8_t *map;
    uint64_t off, bytes;
    void *dev;
    int owned;   /* allocated here (freed on evict/cleanup) */
    int cache;   /* on-demand cache entry (dropped by evict) */
    uint32_t holds;   /* GGUF binder handles holding it (0: registered by the caller) */
} map_range;

static map_range *g_ranges;
static size_t g_nranges, g_cap_ranges;

/* f32 copies of resident bf16 weights (dense matvec / router), made once per
 * weight range and dropped with the range they were read from. */
typedef struct {
    const void *src;
    uint64_t n;
    float *f32;
} widened;

static widened *g_wide;
static size_t g_nwide, g_cap_wide;

static void widen_forget(const void *dev, uint64_t bytes) {
    size_t w = 0;
    for (size_t i = 0; i < g_nwide; i++) {
        const uintptr_t a = (uintptr_t)g_wide[i].src, lo = (uintptr_t)dev;
        if (a >= lo && a - lo < bytes) (void)hipFree(g_wide[i].f32);
        else g_wide[w++] = g_wide[i];
    }
    g_nwide = w;
}

static int hip_ok(hipError_t err, const char *what) {
    if (err == hipSuccess) return 1;
    fprintf(stderr, "sf37: HIP %s failed: %s\n", what, hipGetErrorString(err));
    (void)hipGetLastError();
    return 0;
}

/* ---- stage profiling (events around launches) ---------------------------- */
typedef struct {
    hipEvent_t a, b;
    uint32_t stage;
} prof_pair;

static int g_prof_on;
static prof_pair *g_prof;
static size_t g_nprof, g_cap_prof;
static hipEvent_t g_prof_open;

static const char *const k_stage_names[SF37_HIP_N_STAGES] = {
    "router", "select", "q8_0_act", "q8_0_gemm", "swiglu", "q8k_x", "dispatch",
    "gate_up", "q8k_mid", "down", "combine", "add", "other", "dec_route", "dec_up", "dec_down", "dec_select", "dec_combine", "dec_mid",
    "pf_act_x", "pf_tiles", "pf_gate_up", "pf_act_mid", "pf_down",
    "sh_repack", "sh_act", "sh_gate_up", "sh_down"};

static void prof_begin(hipStream_t st) {
    if (!g_prof_on) return;
    if (hipEventCreate(&g_prof_open) != hipSuccess || hipEventRecord(g_prof_open, st) != hipSuccess) {
        g_prof_open = NULL;
        (void)hipGetLastError();
    }
}

static void prof_end(uint32_t stage, hipStream_t st) {
    if (!g_prof_on || !g_prof_open) return;
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess || hipEventRecord(e, st) != hipSuccess) {
        (void)hipGetLastError();
        return;
    }
    if (g_nprof == g_cap_prof) {
        const size_t cap = g_cap_prof ? 2 * g_cap_prof : 256;
        prof_pair *n = (prof_pair *)realloc(g_prof, cap * sizeof(prof_pair));
        if (!n) return;
        g_prof = n;
        g_cap_prof = cap;
    }
    prof_pair pp = {g_prof_open, e, stage};
    g_prof[g_nprof++] = pp;
    g_prof_open = NULL;
}

static int launch_ok(int err, const char *what) { return hip_ok((hipError_t)err, what); }

/* Launch wrappers: events around the launch on its stream when profiling. */
#define LAUNCH_ON(st, stage, call, what) \
    (prof_begin(st), launch_ok((call), (what)) ? (prof_end((stage), (st)), 1) : 0)
#define LAUNCH(stage, call, what) LAUNCH_ON(g_stream, stage, call, what)

int sf37_hip_profile_enable(int on) {
    g_prof_on = on ? 1 : 0;
    return 1;
}

const char *sf37_hip_profile_stage_name(uint32_t stage) {
    return stage < SF37_HIP_N_STAGES ? k_stage_names[stage] : NULL;
}

int sf37_hip_profile_read(double *ms, uint64_t *count, uint32_t n_stages) {
    if (!g_init) return 0;
    for (uint32_t i = 0; i < n_stages; i++) {
        if (ms) ms[i] = 0.0;
        if (count) count[i] = 0;
    }
    if (!hip_ok(hipStreamSynchronize(g_stream), "profile sync")) return 0;
    for (size_t i = 0; i < g_nprof; i++) {
        float t = 0.0f;
        if (hipEventElapsedTime(&t, g_prof[i].a, g_prof[i].b) == hipSuccess && g_prof[i].stage < n_stages) {
            if (ms) ms[g_prof[i].stage] += t;
            if (count) count[g_prof[i].stage]++;
        }
        (void)hipEventDestroy(g_prof[i].a);
        (void)hipEventDestroy(g_prof[i].b);
    }
    (void)hipGetLastError();
    g_nprof = 0;
    return 1;
}

static int ensure_init(void) {
    if (g_init) return 1;
    return sf37_hip_init();
}

static uint64_t align256(uint64_t v) { return (v + 255u) & ~(uint64_t)255u; }

/* Requests for device memory the library serves (scratch, counters, layer
 * buffers, range copies, widened weights, tensors), whether or not a buffer
 * had to grow: the no-alloc entry point makes none. */
static uint64_t g_mem_requests;

uint64_t sf37_hip_device_memory_requests(void) { return g_mem_requests; }

/* One reusable scratch area (the reference's cuda_tmp_alloc,
 * sf37_cuda.cu:1579-1592).  Growing it waits for queued work first. */
static char *scratch_get(uint64_t bytes, const char *what) {
    g_mem_requests++;
    if (bytes <= g_scratch_bytes && g_scratch) return (char *)g_scratch;
    if (g_scratch) {
        if (!hip_ok(hipStreamSynchronize(g_stream), "scratch sync")) return NULL;
        (void)hipFree(g_scratch);
        g_scratch = NULL;
        g_scratch_bytes = 0;
    }
    void *p = NULL;
    if (!hip_ok(hipMalloc(&p, bytes + SF37_PAD), what)) return NULL;
    g_scratch = p;
    g_scratch_bytes = bytes;
    return (char *)p;
}

static void *layer_buf(int i, uint64_t bytes);

/* Router logits with binary64 sums.  Above 16 tokens the product is split
 * over K into slices whose partial sums go to layer buffer 11 and are added
 * in slice order; if that buffer cannot be had it runs unsplit (same sums,
 * fewer workgroups). */
static int router_matmul_part(float *out, const float *w, const float *x, uint64_t in_dim, uint64_t out_dim,
                              uint64_t n_tok, uint32_t *slices_left, double **part_out, sf37_stream_t s) {
    const uint64_t pb = sf37k_f32_matmul_part_bytes(in_dim, out_dim, n_tok);
    double *part = pb ? (double *)layer_buf(11, pb) : NULL;
    if (part_out) *part_out = part;
    return sf37k_f32_matmul(out, w, x, in_dim, out_dim, n_tok, part, part ? pb : 0, slices_left, s);
}

static int router_matmul(float *out, const float *w, const float *x, uint64_t in_dim, uint64_t out_dim,
                         uint64_t n_tok, sf37_stream_t s) {
    return router_matmul_part(out, w, x, in_dim, out_dim, n_tok, NULL, NULL, s);
}

/* Weight rows and activations are read with dword loads. */
static int aligned4(const void *p) {
    if (((uintptr_t)p & 3u) == 0) return 1;
    fprintf(stderr, "sf37: HIP buffer %p is not 4-byte aligned\n", p);
    return 0;
}

static int q8k_use_for(uint64_t rows) {
    return g_opt_q8k && rows >= (uint64_t)g_opt_q8k_min_rows;
}

static int mapped_range_ok(uint64_t model_size, uint64_t offset, uint64_t bytes) {
    return offset <= model_size && bytes <= model_size - offset;   /* sf37_cuda.cu:5843-5845 */
}

/* ------------------------------------------------------------------------ */
/* runtime (sf37_cuda.cu:1594-1680)                                          */
/* ------------------------------------------------------------------------ */

int sf37_hip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return -1;
    }
    return n;
}

void sf37_hip_print_devices(void) {
    const int n = sf37_hip_device_count();
    if (n < 0) {
        fprintf(stderr, "sf37: HIP device query failed\n");
        return;
    }
    for (int i = 0; i < n; i++) {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, i) != hipSuccess) continue;
        fprintf(stderr, "sf37: HIP device %d: %s (%s), %d CUs, %.1f GiB\n", i, p.name,
                p.gcnArchName, p.multiProcessorCount, (double)p.totalGlobalMem / (1u << 30));
    }
}

int sf37_hip_init(void) {
    if (g_init) return 1;
    if (!hip_ok(hipSetDevice(0), "set device")) return 0;
    g_stream = NULL;
    /* the no-alloc entry point's static scratch on this device */
    if (!hip_ok((hipError_t)sf37k_noalloc_scratch_init(), "no-alloc scratch address")) (void)0;
    g_init = 1;
    return 1;
}

static void free_ranges(int cache_only) {
    size_t w = 0;
    for (size_t i = 0; i < g_nranges; i++) {
        if (!cache_only || g_ranges[i].cache) {
            widen_forget(g_ranges[i].dev, g_ranges[i].bytes);
            if (g_ranges[i].owned && g_ranges[i].dev) (void)hipFree(g_ranges[i].dev);
        } else {
            g_ranges[w++] = g_ranges[i];
        }
    }
    g_nranges = w;
}

void sf37_hip_cleanup(void) {
    if (!g_init) return;
    (void)hipDeviceSynchronize();
    free_ranges(0);
    free(g_ranges);
    g_ranges = NULL;
    g_cap_ranges = 0;
    widen_forget(NULL, UINT64_MAX);
    free(g_wide);
    g_wide = NULL;
    g_cap_wide = 0;
    if (g_scratch) (void)hipFree(g_scratch);
    g_scratch = NULL;
    g_scratch_bytes = 0;
    if (g_dec_cnt) (void)hipFree(g_dec_cnt);
    g_dec_cnt = NULL;
    g_dec_cnt_words = 0;
    if (g_side) (void)hipStreamDestroy(g_side);
    if (g_ev_fork) (void)hipEventDestroy(g_ev_fork);
    if (g_ev_join) (void)hipEventDestroy(g_ev_join);
    g_side = NULL;
    g_ev_fork = g_ev_join = NULL;
    for (int i = 0; i < N_LAYER_BUFS; i++) {
        if (g_layer_bufs[i]) {
            (void)hipFree(g_layer_bufs[i]->ptr);
            free(g_layer_bufs[i]);
        }
        g_layer_bufs[i] = NULL;
        g_layer_buf_bytes[i] = 0;
    }
    g_init = 0;
}

int sf37_hip_synchronize(void) {
    if (!ensure_init()) return 0;
    return hip_ok(hipStreamSynchronize(g_stream), "synchronize");
}

int sf37_hip_memory_info(uint64_t *free_bytes, uint64_t *total_bytes) {
    if (!ensure_init()) return 0;
    size_t f = 0, t = 0;
    if (!hip_ok(hipMemGetInfo(&f, &t), "memory info")) return 0;
    if (free_bytes) *free_bytes = f;
    if (total_bytes) *total_bytes = t;
    return 1;
}

/* Layer markers only bracket per-layer work in the reference (weight
 * streaming); with every weight resident there is nothing to do. */
int sf37_hip_begin_layer(uint32_t layer) {
    (void)layer;
    return ensure_init();
}

void sf37_hip_end_layer(void) {}

int sf37_hip_set_stream(void *stream) {
    if (!ensure_init()) return 0;
    g_stream = (hipStream_t)stream;
    return 1;
}

void *sf37_hip_get_stream(void) { return (void *)g_stream; }

int sf37_hip_set_option(const char *name, int64_t value) {
    if (!name) return 0;
    if (!strcmp(name, "q8k")) g_opt_q8k = value ? 1 : 0;
    else if (!strcmp(name, "q8k_min_rows")) g_opt_q8k_min_rows = value < 0 ? 0 : value;
    else if (!strcmp(name, "moe_write_gate_up")) g_opt_write_gate_up = value ? 1 : 0;
    else if (!strcmp(name, "decode_fused")) g_opt_decode = value ? 1 : 0;
    else if (!strcmp(name, "router_with_logits")) g_opt_router_always = value ? 1 : 0;
    else if (!strcmp(name, "decode_up_dyn_pct")) g_opt_up_dyn_pct = value < 0 ? -1 : (value > 100 ? 100 : value);
    else if (!strcmp(name, "decode_up_wgs")) g_opt_up_wgs = value < 0 ? 0 : value;
    else if (!strcmp(name, "decode_down_wgs")) g_opt_dn_wgs = value < 0 ? 0 : value;
    else if (!strcmp(name, "decode_select_in_up_max_tokens")) g_opt_upsel_max_tok = value < 0 ? 0 : value;
    else if (!strcmp(name, "decode_down_combine")) g_opt_down_combine = value ? 1 : 0;
    else if (!strcmp(name, "prefill_mfma")) g_opt_prefill = value ? 1 : 0;
    else if (!strcmp(name, "prefill_min_pairs")) g_opt_prefill_min_pairs = value < 0 ? 0 : value;
    else if (!strcmp(name, "shared_min_tokens")) g_opt_shared_min_tok = value < 0 ? 0 : value;
    else if (!strcmp(name, "shared_stream")) g_opt_shared_stream = value ? 1 : 0;
    else if (!strcmp(name, "decode_shared_slot")) g_opt_shared_slot = value ? 1 : 0;
    else return 0;
    return 1;
}

int64_t sf37_hip_get_option(const char *name) {
    if (!name) return -1;
    if (!strcmp(name, "q8k")) return g_opt_q8k;
    if (!strcmp(name, "q8k_min_rows")) return g_opt_q8k_min_rows;
    if (!strcmp(name, "moe_write_gate_up")) return g_opt_write_gate_up;
    if (!strcmp(name, "decode_fused")) return g_opt_decode;
    if (!strcmp(name, "router_with_logits")) return g_opt_router_always;
    if (!strcmp(name, "decode_up_dyn_pct")) return g_opt_up_dyn_pct;
    if (!strcmp(name, "decode_up_wgs")) return g_opt_up_wgs;
    if (!strcmp(name, "decode_down_wgs")) return g_opt_dn_wgs;
    if (!strcmp(name, "decode_select_in_up_max_tokens")) return g_opt_upsel_max_tok;
    if (!strcmp(name, "decode_down_combine")) return g_opt_down_combine;
    if (!strcmp(name, "prefill_mfma")) return g_opt_prefill;
    if (!strcmp(name, "prefill_min_pairs")) return g_opt_prefill_min_pairs;
    if (!strcmp(name, "shared_min_tokens")) return g_opt_shared_min_tok;
    if (!strcmp(name, "shared_stream")) return g_opt_shared_stream;
    if (!strcmp(name, "decode_shared_slot")) return g_opt_shared_slot;
    return -1;
}

/* ------------------------------------------------------------------------ */
/* tensors (sf37_cuda.cu:1680-1850)                                          */
/* ------------------------------------------------------------------------ */

static sf37_hip_tensor *tensor_new(void *ptr, uint64_t bytes, int owned) {
    sf37_hip_tensor *t = (sf37_hip_tensor *)calloc(1, sizeof(*t));
    if (!t) return NULL;
    t->ptr = ptr;
    t->bytes = bytes;
    t->owned = owned;
    return t;
}

sf37_hip_tensor *sf37_hip_tensor_alloc(uint64_t bytes) {
    g_mem_requests++;
    if (!ensure_init()) return NULL;
    void *p = NULL;
    if (!hip_ok(hipMalloc(&p, bytes + SF37_PAD), "tensor alloc")) return NULL;
    sf37_hip_tensor *t = tensor_new(p, bytes, 1);
    if (!t) (void)hipFree(p);
    return t;
}

sf37_hip_tensor *sf37_hip_tensor_alloc_managed(uint64_t bytes) {
    g_mem_requests++;
    if (!ensure_init()) return NULL;
    void *p = NULL;
    if (!hip_ok(hipMallocManaged(&p, bytes + SF37_PAD, hipMemAttachGlobal), "managed tensor alloc"))
        return NULL;
    sf37_hip_tensor *t = tensor_new(p, bytes, 1);
    if (!t) (void)hipFree(p);
    return t;
}

void sf37_hip_tensor_free(sf37_hip_tensor *tensor) {
    if (!tensor) return;
    if (tensor->owned && tensor->ptr) {
        (void)hipStreamSynchronize(g_stream);
        (void)hipFree(tensor->ptr);
    }
    free(tensor);
}

uint64_t sf37_hip_tensor_bytes(const sf37_hip_tensor *tensor) { return tensor ? tensor->bytes : 0; }

void *sf37_hip_tensor_device_ptr(const sf37_hip_tensor *tensor) { return tensor ? tensor->ptr : NULL; }

sf37_hip_tensor *sf37_hip_tensor_view(const sf37_hip_tensor *base, uint64_t offset, uint64_t bytes) {
    if (!base || offset > base->bytes || bytes > base->bytes - offset) return NULL;
    return tensor_new((char *)base->ptr + offset, bytes, 0);
}

int sf37_hip_tensor_write(sf37_hip_tensor *tensor, uint64_t offset, const void *data, uint64_t bytes) {
    if (!tensor || (!data && bytes) || offset > tensor->bytes || bytes > tensor->bytes - offset) return 0;
    if (!bytes) return 1;
    if (!hip_ok(hipMemcpyAsync((char *)tensor->ptr + offset, data, bytes, hipMemcpyHostToDevice, g_stream),
                "tensor write"))
        return 0;
    return hip_ok(hipStreamSynchronize(g_stream), "tensor write sync");
}

int sf37_hip_tensor_read(const sf37_hip_tensor *tensor, uint64_t offset, void *data, uint64_t bytes) {
    if (!tensor || (!data && bytes) || offset > tensor->bytes || bytes > tensor->bytes - offset) return 0;
    if (!bytes) return 1;
    if (!hip_ok(hipMemcpyAsync(data, (const char *)tensor->ptr + offset, bytes, hipMemcpyDeviceToHost,
                               g_stream),
                "tensor read"))
        return 0;
    return hip_ok(hipStreamSynchronize(g_stream), "tensor read sync");
}

int sf37_hip_tensor_copy(sf37_hip_tensor *dst, uint64_t dst_offset, const sf37_hip_tensor *src,
                         uint64_t src_offset, uint64_t bytes) {
    if (!dst || !src || dst_offset > dst->bytes || bytes > dst->bytes - dst_offset ||
        src_offset > src->bytes || bytes > src->bytes - src_offset)
        return 0;
    if (!bytes) return 1;
    return hip_ok(hipMemcpyAsync((char *)dst->ptr + dst_offset, (const char *)src->ptr + src_offset, bytes,
                                 hipMemcpyDeviceToDevice, g_stream),
                  "tensor copy");
}

int sf37_hip_tensor_fill_f32(sf37_hip_tensor *tensor, float value, uint64_t count) {
    if (!tensor || count > tensor->bytes / sizeof(float)) return 0;
    if (!count) return 1;
    uint32_t bits;
    memcpy(&bits, &value, 4);
    return hip_ok(hipMemsetD32Async((hipDeviceptr_t)tensor->ptr, (int)bits, count, g_stream), "tensor fill");
}

/* ------------------------------------------------------------------------ */
/* model map (sf37_cuda.cu:1131-1188, 1418-1478)                             */
/* ------------------------------------------------------------------------ */

static int range_push(const uint8_t *map, uint64_t off, uint64_t bytes, void *dev, int owned, int cache) {
    if (g_nranges == g_cap_ranges) {
        const size_t cap = g_cap_ranges ? g_cap_ranges * 2 : 16;
        map_range *n = (map_range *)realloc(g_ranges, cap * sizeof(map_range));
        if (!n) return 0;
        g_ranges = n;
        g_cap_ranges = cap;
    }
    map_range r = {map, off, bytes, dev, owned, cache, 0};
    g_ranges[g_nranges++] = r;
    return 1;
}

static int upload_range(const uint8_t *map, uint64_t off, uint64_t bytes, int cache, const char *label) {
    g_mem_requests++;
    void *dev = NULL;
    char what[160];
    snprintf(what, sizeof(what), "model range upload (%s)", label ? label : "range");
    if (!hip_ok(hipMalloc(&dev, bytes + SF37_PAD), what)) return 0;
    if (!hip_ok(hipMemcpy(dev, map + off, bytes, hipMemcpyHostToDevice), what) ||
        !range_push(map, off, bytes, dev, 1, cache)) {
        (void)hipFree(dev);
        return 0;
    }
    return 1;
}

/* Device address of map[offset, offset+bytes): a registered range, else an
 * on-demand cached copy (kept until sf37_hip_evict_model_cache). */
static const void *model_ptr(const void *model_map, uint64_t offset, uint64_t bytes, const char *label) {
    const uint8_t *map = (const uint8_t *)model_map;
    for (size_t i = g_nranges; i-- > 0;) {   /* newest registration wins */
        const map_range *r = &g_ranges[i];
        if (r->map == map && offset >= r->off && bytes <= r->bytes && offset - r->off <= r->bytes - bytes)
            return (const char *)r->dev + (offset - r->off);
    }
    if (!ensure_init() || !upload_range(map, offset, bytes, 1, label)) return NULL;
    return g_ranges[g_nranges - 1].dev;
}

/* Forget every range of one host map (registered or cached), freeing the
 * device copies the library made: a map about to be unmapped, whose address
 * a later mapping may reuse. */
void sf37i_drop_map(const void *model_map) {
    if (!g_init || !model_map) return;
    (void)hipStreamSynchronize(g_stream);
    size_t w = 0;
    for (size_t i = 0; i < g_nranges; i++) {
        if (g_ranges[i].map == (const uint8_t *)model_map) {
            widen_forget(g_ranges[i].dev, g_ranges[i].bytes);
            if (g_ranges[i].owned && g_ranges[i].dev) (void)hipFree(g_ranges[i].dev);
        } else {
            g_ranges[w++] = g_ranges[i];
        }
    }
    g_nranges = w;
}

void sf37i_drop_range(const void *model_map, uint64_t offset, uint64_t bytes);

/* A non-owning tensor over a device copy of map[offset, offset+bytes) that
 * sf37_hip_evict_model_cache does not free, for the GGUF layer binder
 * (sf37_gguf.c): a registered (non-cache) range that covers it, else a new
 * registered range made here.  Ranges made here are held by the binder
 * handles that use them: *held = 1 and *range_off / *range_bytes name the
 * range when the caller took a hold (a new range, or one another handle made
 * and still holds), which it gives back with sf37i_drop_range when its handle
 * closes; the range is freed when the last hold goes.  Ranges the caller
 * registered (set_model_map_range/_spans, register_device_range) are used
 * without a hold (*held = 0) and stay until evicted or cleaned up. */
sf37_hip_tensor *sf37i_map_tensor(const void *model_map, uint64_t model_size, uint64_t offset, uint64_t bytes,
                                  const char *label, int *held, uint64_t *range_off, uint64_t *range_bytes) {
    *held = 0;
    if (!model_map || !bytes || !mapped_range_ok(model_size, offset, bytes) || !ensure_init()) return NULL;
    const uint8_t *map = (const uint8_t *)model_map;
    for (size_t i = g_nranges; i-- > 0;) {
        map_range *r = &g_ranges[i];
        if (!r->cache && r->map == map && offset >= r->off && bytes <= r->bytes && offset - r->off <= r->bytes - bytes) {
            sf37_hip_tensor *t = tensor_new((char *)r->dev + (offset - r->off), bytes, 0);
            if (t && r->holds) {
                r->holds++;
                *held = 1;
                *range_off = r->off;
                *range_bytes = r->bytes;
            }
            return t;
        }
    }
    if (!upload_range(map, offset, bytes, 0, label)) return NULL;
    g_ranges[g_nranges - 1].holds = 1;
    sf37_hip_tensor *t = tensor_new(g_ranges[g_nranges - 1].dev, bytes, 0);
    if (!t) {
        sf37i_drop_range(map, offset, bytes);
        return NULL;
    }
    *held = 1;
    *range_off = offset;
    *range_bytes = bytes;
    return t;
}

/* Give back one hold on the binder-made range map[offset, offset+bytes)
 * (the newest held range of exactly that extent); the device copy is freed
 * with the last hold. */
void sf37i_drop_range(const void *model_map, uint64_t offset, uint64_t bytes) {
    if (!g_init || !model_map) return;
    for (size_t i = g_nranges; i-- > 0;) {
        map_range *r = &g_ranges[i];
        if (!r->cache && r->holds && r->map == (const uint8_t *)model_map && r->off == offset && r->bytes == bytes) {
            if (--r->holds) return;
            (void)hipStreamSynchronize(g_stream);
            widen_forget(r->dev, r->bytes);
            if (r->owned && r->dev) (void)hipFree(r->dev);
            memmove(r, r + 1, (g_nranges - i - 1) * sizeof(map_range));
            g_nranges--;
            return;
        }
    }
}

/* Holds on the registered range that covers map[offset, offset+bytes):
 * -1 when no registered range covers it, 0 for a caller-registered range,
 * else the number of binder handles holding it. */
int sf37_hip_model_range_holds(const void *model_map, uint64_t offset, uint64_t bytes) {
    if (!g_init || !model_map) return -1;
    for (size_t i = g_nranges; i-- > 0;) {
        const map_range *r = &g_ranges[i];
        if (!r->cache && r->map == (const uint8_t *)model_map && offset >= r->off && bytes <= r->bytes &&
            offset - r->off <= r->bytes - bytes)
            return (int)r->holds;
    }
    return -1;
}

int sf37_hip_set_model_fd(int fd) {
    g_model_fd = fd;   /* weights are uploaded from the map; the fd is not needed */
    return 1;
}

int sf37_hip_set_model_map_range(const void *model_map, uint64_t model_size, uint64_t map_offset,
                                 uint64_t map_size, uint64_t max_tensor_bytes) {
    (void)max_tensor_bytes;
    if (!model_map || !mapped_range_ok(model_size, map_offset, map_size) || !ensure_init()) return 0;
    if (!map_size) return 1;
    return upload_range((const uint8_t *)model_map, map_offset, map_size, 0, "model map");
}

int sf37_hip_set_model_map_spans(const void *model_map, uint64_t model_size, const uint64_t *offsets,
                                 const uint64_t *sizes, uint32_t count, uint64_t max_tensor_bytes) {
    if (!model_map || (count && (!offsets || !sizes))) return 0;
    for (uint32_t i = 0; i < count; i++)
        if (!sf37_hip_set_model_map_range(model_map, model_size, offsets[i], sizes[i], max_tensor_bytes))
            return 0;
    return 1;
}

int sf37_hip_cache_model_range(const void *model_map, uint64_t model_size, uint64_t offset, uint64_t bytes,
                               const char *label) {
    if (!model_map || !mapped_range_ok(model_size, offset, bytes)) return 0;
    return model_ptr(model_map, offset, bytes, label) != NULL;
}

void sf37_hip_evict_model_cache(const char *reason) {
    (void)reason;
    if (!g_init) return;
    (void)hipStreamSynchronize(g_stream);
    free_ranges(1);
}

int sf37_hip_register_device_range(const void *model_map, uint64_t model_size, uint64_t map_offset,
                                   uint64_t bytes, const sf37_hip_tensor *device) {
    if (!model_map || !device || bytes > device->bytes || !mapped_range_ok(model_size, map_offset, bytes) ||
        !ensure_init())
        return 0;
    return range_push((const uint8_t *)model_map, map_offset, bytes, device->ptr, 0, 0);
}

/* ------------------------------------------------------------------------ */
/* elementwise / norm (sf37_cuda.cu:2037-2180, 6117-6164)                    */
/* ------------------------------------------------------------------------ */

int sf37_hip_rms_norm_weight1_f32(sf37_hip_tensor *out, const sf37_hip_tensor *x,
                                  const sf37_hip_tensor *weight, uint32_t n, float eps) {
    if (!out || !x || !weight || !ensure_init()) return 0;
    if (out->bytes < (uint64_t)n * 4u || x->bytes < (uint64_t)n * 4u || weight->bytes < (uint64_t)n * 4u) return 0;
    return LAUNCH(SF37_HIP_STAGE_OTHER, sf37k_rms_norm((float *)out->ptr, (const float *)x->ptr, weight->ptr, 0, n, 1, eps,
                                    (sf37_stream_t)g_stream),
                     "rms_norm_weight1 launch");
}

int sf37_hip_rms_norm_weight1_bf16(sf37_hip_tensor *out, const sf37_hip_tensor *x,
                                   const sf37_hip_tensor *weight, uint32_t n, float eps) {
    if (!out || !x || !weight || !ensure_init()) return 0;
    if (out->bytes < (uint64_t)n * 4u || x->bytes < (uint64_t)n * 4u || weight->bytes < (uint64_t)n * 2u) return 0;
    return LAUNCH(SF37_HIP_STAGE_OTHER, sf37k_rms_norm((float *)out->ptr, (const float *)x->ptr, weight->ptr, 1, n, 1, eps,
                                    (sf37_stream_t)g_stream),
                     "rms_norm_weight1_bf16 launch");
}

int sf37_hip_rms_norm_weight1_bf16_mapped(sf37_hip_tensor *out, const sf37_hip_tensor *x,
                                          const void *model_map, uint64_t model_size,
                                          uint64_t weight_offset, uint32_t n, float eps) {
    return sf37_hip_rms_norm_weight1_bf16_batch_mapped(out, x, model_map, model_size, weight_offset, n, 1, eps);
}

int sf37_hip_rms_norm_weight1_bf16_batch_mapped(sf37_hip_tensor *out, const sf37_hip_tensor *x,
                                                const void *model_map, uint64_t model_size,
                                                uint64_t weight_offset, uint32_t n, uint32_t n_tok,
                                                float eps) {
    if (!out || !x || !model_map || n_tok == 0 || !ensure_init()) return 0;
    const uint64_t bytes = (uint64_t)n * n_tok * 4u;
    if (!mapped_range_ok(model_size, weight_offset, (uint64_t)n * 2u) || out->bytes < bytes || x->bytes < bytes)
        return 0;
    const void *w = model_ptr(model_map, weight_offset, (uint64_t)n * 2u, "rms norm weight");
    if (!w) return 0;
    return LAUNCH(SF37_HIP_STAGE_OTHER, sf37k_rms_norm((float *)out->ptr, (const float *)x->ptr, w, 1, n, n_tok, eps,
                                    (sf37_stream_t)g_stream),
                     "rms_norm_weight1_bf16 batch launch");
}

int sf37_hip_add_inplace_f32(sf37_hip_tensor *dst, const sf37_hip_tensor *src, uint64_t n) {
    if (!dst || !src || !ensure_init()) return 0;
    if (dst->bytes < n * 4u || src->bytes < n * 4u) return 0;
    return LAUNCH(SF37_HIP_STAGE_ADD, sf37k_add_inplace((float *)dst->ptr, (const float *)src->ptr, n, (sf37_stream_t)g_stream),
                     "add inplace f32 launch");
}

int sf37_hip_swiglu_f32(sf37_hip_tensor *out, const sf37_hip_tensor *gate, const sf37_hip_tensor *up,
                        uint64_t n, float clamp) {
    if (!out || !gate || !up || !ensure_init()) return 0;
    if (out->bytes < n * 4u || gate->bytes < n * 4u || up->bytes < n * 4u) return 0;
    return LAUNCH(SF37_HIP_STAGE_SWIGLU, sf37k_swiglu((float *)out->ptr, (const float *)gate->ptr, (const float *)up->ptr, n, clamp,
                                  (sf37_stream_t)g_stream),
                     "swiglu launch");
}

/* ------------------------------------------------------------------------ */
/* Q8_0 (sf37_cuda.cu:3319-3781, 6405-6440, 6649-6916)                       */
/* ------------------------------------------------------------------------ */

static int q8_0_run(float *out0, float *out1, const uint8_t *w0, const uint8_t *w1, uint64_t in_dim,
                    uint64_t out_dim, const float *x, uint64_t n_tok) {
    const uint64_t nb = (in_dim + 31u) / 32u;
    if (!aligned4(x) || !aligned4(out0) || (out1 && !aligned4(out1))) return 0;
    const uint64_t xq_bytes = align256(n_tok * nb * 32u);
    char *s = scratch_get(xq_bytes + n_tok * nb * 4u, "q8_0 activations");
    if (!s) return 0;
    int8_t *xq = (int8_t *)s;
    float *xs = (float *)(s + xq_bytes);
    if (!LAUNCH(SF37_HIP_STAGE_Q8_0_ACT, sf37k_q8_0_quantize(xq, xs, x, in_dim, n_tok, (sf37_stream_t)g_stream), "q8_0 quantize launch"))
        return 0;
    return LAUNCH(SF37_HIP_STAGE_Q8_0_GEMM, sf37k_q8_0_matmul(out0, out1, w0, w1, xq, xs, in_dim, out_dim, n_tok, (sf37_stream_t)g_stream),
                     "q8_0 matmul launch");
}

static uint64_t q8_0_bytes(uint64_t in_dim, uint64_t out_dim) { return out_dim * ((in_dim + 31u) / 32u) * Q8B; }

int sf37_hip_matvec_q8_0(sf37_hip_tensor *out, const sf37_hip_tensor *weights, uint64_t in_dim,
                         uint64_t out_dim, const sf37_hip_tensor *x) {
    if (!out || !weights || !x || !ensure_init()) return 0;
    if (out->bytes < out_dim * 4u || x->bytes < in_dim * 4u || weights->bytes < q8_0_bytes(in_dim, out_dim)) return 0;
    return q8_0_run((float *)out->ptr, NULL, (const uint8_t *)weights->ptr, NULL, in_dim, out_dim,
                    (const float *)x->ptr, 1);
}

int sf37_hip_matvec_q8_0_pair(sf37_hip_tensor *out0, sf37_hip_tensor *out1, const sf37_hip_tensor *weights0,
                              const sf37_hip_tensor *weights1, uint64_t in_dim, uint64_t out_dim,
                              const sf37_hip_tensor *x) {
    if (!out0 || !out1 || !weights0 || !weights1 || !x || !ensure_init()) return 0;
    const uint64_t wb = q8_0_bytes(in_dim, out_dim);
    if (out0->bytes < out_dim * 4u || out1->bytes < out_dim * 4u || x->bytes < in_dim * 4u ||
        weights0->bytes < wb || weights1->bytes < wb)
        return 0;
    return q8_0_run((float *)out0->ptr, (float *)out1->ptr, (const uint8_t *)weights0->ptr,
                    (const uint8_t *)weights1->ptr, in_dim, out_dim, (const float *)x->ptr, 1);
}

int sf37_hip_matvec_q8_0_mapped(sf37_hip_tensor *out, const void *model_map, uint64_t model_size,
                                uint64_t weight_offset, uint64_t in_dim, uint64_t out_dim,
                                const sf37_hip_tensor *x) {
    return sf37_hip_matmul_q8_0_mapped(out, model_map, model_size, weight_offset, in_dim, out_dim, x, 1);
}

int sf37_hip_matmul_q8_0_mapped(sf37_hip_tensor *out, const void *model_map, uint64_t model_size,
                                uint64_t weight_offset, uint64_t in_dim, uint64_t out_dim,
                                const sf37_hip_tensor *x, uint64_t n_tok) {
    if (!out || !model_map || !x || n_tok == 0 || !ensure_init()) return 0;
    const uint64_t wb = q8_0_bytes(in_dim, out_dim);
    if (!mapped_range_ok(model_size, weight_offset, wb) || out->bytes < n_tok * out_dim * 4u ||
        x->bytes < n_tok * in_dim * 4u)
        return 0;
    const uint8_t *w = (const uint8_t *)model_ptr(model_map, weight_offset, wb, "q8_0 weights");
    if (!w) return 0;
    return q8_0_run((float *)out->ptr, NULL, w, NULL, in_dim, out_dim, (const float *)x->ptr, n_tok);
}

int sf37_hip_matmul_q8_0_pair_mapped(sf37_hip_tensor *out0, sf37_hip_tensor *out1, const void *model_map,
                                     uint64_t model_size, uint64_t weight0_offset, uint64_t weight1_offset,
                                     uint64_t in_dim, uint64_t out_dim, const sf37_hip_tensor *x,
                                     uint64_t n_tok) {
    if (!out0 || !out1 || !model_map || !x || n_tok == 0 || !ensure_init()) return 0;
    const uint64_t wb = q8_0_bytes(in_dim, out_dim);
    if (!mapped_range_ok(model_size, weight0_offset, wb) || !mapped_range_ok(model_size, weight1_offset, wb) ||
        out0->bytes < n_tok * out_dim * 4u || out1->bytes < n_tok * out_dim * 4u || x->bytes < n_tok * in_dim * 4u)
        return 0;
    const uint8_t *w0 = (const uint8_t *)model_ptr(model_map, weight0_offset, wb, "q8_0 pair weights 0");
    const uint8_t *w1 = (const uint8_t *)model_ptr(model_map, weight1_offset, wb, "q8_0 pair weights 1");
    if (!w0 || !w1) return 0;
    return q8_0_run((float *)out0->ptr, (float *)out1->ptr, w0, w1, in_dim, out_dim, (const float *)x->ptr, n_tok);
}

int sf37_hip_matvec_q8_0_pair_mapped(sf37_hip_tensor *out0, sf37_hip_tensor *out1, const void *model_map,
                                     uint64_t model_size, uint64_t weight0_offset, uint64_t weight1_offset,
                                     uint64_t in_dim, uint64_t out_dim, const sf37_hip_tensor *x) {
    return sf37_hip_matmul_q8_0_pair_mapped(out0, out1, model_map, model_size, weight0_offset, weight1_offset,
                                            in_dim, out_dim, x, 1);
}

/* ------------------------------------------------------------------------ */
/* f32 router GEMV/GEMM (sf37_cuda.cu:4100-4147, 7034-7113)                  */
/* ------------------------------------------------------------------------ */

int sf37_hip_matvec_f32(sf37_hip_tensor *out, const sf37_hip_tensor *weights, uint64_t in_dim,
                        uint64_t out_dim, const sf37_hip_tensor *x) {
    if (!out || !weights || !x || !ensure_init()) return 0;
    if (out->bytes < out_dim * 4u || x->bytes < in_dim * 4u || weights->bytes < out_dim * in_dim * 4u) return 0;
    return LAUNCH(SF37_HIP_STAGE_ROUTER, router_matmul((float *)out->ptr, (const float *)weights->ptr, (const float *)x->ptr, in_dim,
                                      out_dim, 1, (sf37_stream_t)g_stream),
                     "f32 matvec launch");
}

int sf37_hip_matvec_f32_mapped(sf37_hip_tensor *out, const void *model_map, uint64_t model_size,
                               uint64_t weight_offset, uint64_t in_dim, uint64_t out_dim,
                               const sf37_hip_tensor *x) {
    return sf37_hip_matmul_f32_mapped(out, model_map, model_size, weight_offset, in_dim, out_dim, x, 1);
}

int sf37_hip_matmul_f32_mapped(sf37_hip_tensor *out, const void *model_map, uint64_t model_size,
                               uint64_t weight_offset, uint64_t in_dim, uint64_t out_dim,
                               const sf37_hip_tensor *x, uint64_t n_tok) {
    if (!out || !model_map || !x || n_tok == 0 || !ensure_init()) return 0;
    const uint64_t wb = out_dim * in_dim * 4u;
    if (!mapped_range_ok(model_size, weight_offset, wb) || out->bytes < n_tok * out_dim * 4u ||
        x->bytes < n_tok * in_dim * 4u)
        return 0;
    const float *w = (const float *)model_ptr(model_map, weight_offset, wb, "f32 weights");
    if (!w) return 0;
    return LAUNCH(SF37_HIP_STAGE_ROUTER, router_matmul((float *)out->ptr, w, (const float *)x->ptr, in_dim, out_dim, n_tok,
                                      (sf37_stream_t)g_stream),
                     "f32 matmul launch");
}

/* ---- bf16 dense weights (sf37_cuda.h:144-147, 324-345) -------------------- */
/* The CPU engine widens every bf16 weight exactly and accumulates in binary64
 * (sf37_bf16_matvec, sf37_ops.c:143-151), the arithmetic of the f32 kernels
 * above: resident bf16 weights are widened once per range into an f32 copy
 * those kernels read; a tensor's weights (which may change between calls)
 * are widened into scratch on every call. */
static const float *bf16_resident_f32(const void *w, uint64_t n) {
    g_mem_requests++;
    for (size_t i = 0; i < g_nwide; i++)
        if (g_wide[i].src == w && g_wide[i].n == n) return g_wide[i].f32;
    if (g_nwide == g_cap_wide) {
        const size_t cap = g_cap_wide ? 2 * g_cap_wide : 16;
        widened *nw = (widened *)realloc(g_wide, cap * sizeof(widened));
        if (!nw) return NULL;
        g_wide = nw;
        g_cap_wide = cap;
    }
    void *f = NULL;
    if (!hip_ok(hipMalloc(&f, n * 4u + SF37_PAD), "bf16 weight widening alloc")) return NULL;
    if (!LAUNCH(SF37_HIP_STAGE_OTHER, sf37k_bf16_widen((float *)f, (const uint16_t *)w, n, (sf37_stream_t)g_stream),
                "bf16 widen launch")) {
        (void)hipFree(f);
        return NULL;
    }
    widened e = {w, n, (float *)f};
    g_wide[g_nwide++] = e;
    return (const float *)f;
}

int sf37_hip_matvec_bf16(sf37_hip_tensor *out, const sf37_hip_tensor *weights, uint64_t in_dim, uint64_t out_dim,
                         const sf37_hip_tensor *x) {
    if (!out || !weights || !x || !ensure_init()) return 0;
    const uint64_t n = in_dim * out_dim;
    if (out->bytes < out_dim * 4u || x->bytes < in_dim * 4u || weights->bytes < n * 2u) return 0;
    float *f = (float *)scratch_get(n * 4u, "bf16 weights");
    if (!f) return 0;
    return LAUNCH(SF37_HIP_STAGE_OTHER, sf37k_bf16_widen(f, (const uint16_t *)weights->ptr, n, (sf37_stream_t)g_stream),
                  "bf16 widen launch") &&
           LAUNCH(SF37_HIP_STAGE_ROUTER, router_matmul((float *)out->ptr, f, (const float *)x->ptr, in_dim, out_dim,
                                                          1, (sf37_stream_t)g_stream),
                  "bf16 matvec launch");
}

int sf37_hip_matvec_bf16_mapped(sf37_hip_tensor *out, const void *model_map, uint64_t model_size,
                                uint64_t weight_offset, uint64_t in_dim, uint64_t out_dim,
                                const sf37_hip_tensor *x) {
    return sf37_hip_matmul_bf16_mapped(out, model_map, model_size, weight_offset, in_dim, out_dim, x, 1);
}

int sf37_hip_matmul_bf16_mapped(sf37_hip_tensor *out, const void *model_map, uint64_t model_size,
                                uint64_t weight_offset, uint64_t in_dim, uint64_t out_dim,
                                const sf37_hip_tensor *x, uint64_t n_tok) {
    if (!out || !model_map || !x || n_tok == 0 || !ensure_init()) return 0;
    const uint64_t wb = out_dim * in_dim * 2u;
    if (!mapped_range_ok(model_size, weight_offset, wb) || out->bytes < n_tok * out_dim * 4u ||
        x->bytes < n_tok * in_dim * 4u)
        return 0;
    const void *w = model_ptr(model_map, weight_offset, wb, "bf16 weights");
    const float *f = w ? bf16_resident_f32(w, out_dim * in_dim) : NULL;
    if (!f) return 0;
    return LAUNCH(SF37_HIP_STAGE_ROUTER, router_matmul((float *)out->ptr, f, (const float *)x->ptr, in_dim, out_dim,
                                                          n_tok, (sf37_stream_t)g_stream),
                  "bf16 matmul launch");
}

/* ------------------------------------------------------------------------ */
/* Q3 / Q2 GEMV (sf37_cuda.cu:5783-5841, 7677-7755)                          */
/* ------------------------------------------------------------------------ */

static int qlow_matvec(int q3, float *out, const uint8_t *w, uint64_t in_dim, uint64_t out_dim, const float *x) {
    const uint64_t nb = in_dim / QK;
    if (!aligned4(w) || !aligned4(x) || !aligned4(out)) return 0;
    if (q8k_use_for(out_dim) && nb <= 128u) {
        void *xq = scratch_get(nb * Q8KB, "q3/q2 q8k activation");
        if (!xq) return 0;
        if (!LAUNCH(SF37_HIP_STAGE_Q8K_X, sf37k_q8k_quantize(xq, x, (uint32_t)in_dim, 1, (sf37_stream_t)g_stream), "q8k quantize launch"))
            return 0;
        return launch_ok(q3 ? sf37k_q3_q8k_matvec(out, w, xq, (uint32_t)nb, out_dim, (sf37_stream_t)g_stream)
                            : sf37k_q2_q8k_matvec(out, w, xq, (uint32_t)nb, out_dim, (sf37_stream_t)g_stream),
                         q3 ? "q3 asym q8k matvec launch" : "q2 asym q8k matvec launch");
    }
    return launch_ok(q3 ? sf37k_q3_f32_matvec(out, w, x, in_dim, out_dim, (sf37_stream_t)g_stream)
                        : sf37k_q2_f32_matvec(out, w, x, in_dim, out_dim, (sf37_stream_t)g_stream),
                     q3 ? "q3 asym matvec launch" : "q2 asym matvec launch");
}

static int qlow_checked(int q3, sf37_hip_tensor *out, const sf37_hip_tensor *weights, uint64_t in_dim,
                        uint64_t out_dim, const sf37_hip_tensor *x) {
    if (!out || !weights || !x || in_dim % QK != 0 || !ensure_init()) return 0;
    const uint64_t wb = out_dim * (in_dim / QK) * (q3 ? Q3B : Q2B);
    if (out->bytes < out_dim * 4u || x->bytes < in_dim * 4u || weights->bytes < wb) return 0;
    return qlow_matvec(q3, (float *)out->ptr, (const uint8_t *)weights->ptr, in_dim, out_dim, (const float *)x->ptr);
}

int sf37_hip_matvec_q3_asym(sf37_hip_tensor *out, const sf37_hip_tensor *weights, uint64_t in_dim,
                            uint64_t out_dim, const sf37_hip_tensor *x) {
    return qlow_checked(1, out, weights, in_dim, out_dim, x);
}

int sf37_hip_matvec_q2_asym(sf37_hip_tensor *out, const sf37_hip_tensor *weights, uint64_t in_dim,
                            uint64_t out_dim, const sf37_hip_tensor *x) {
    return qlow_checked(0, out, weights, in_dim, out_dim, x);
}

static int qlow_mapped(int q3, sf37_hip_tensor *out, const void *model_map, uint64_t model_size,
                       uint64_t weight_offset, uint64_t in_dim, uint64_t out_dim, const sf37_hip_tensor *x) {
    if (!out || !model_map || !x || in_dim % QK != 0 || !ensure_init()) return 0;
    const uint64_t wb = out_dim * (in_dim / QK) * (q3 ? Q3B : Q2B);
    if (!mapped_range_ok(model_size, weight_offset, wb) || out->bytes < out_dim * 4u || x->bytes < in_dim * 4u)
        return 0;
    const uint8_t *w = (const uint8_t *)model_ptr(model_map, weight_offset, wb, q3 ? "q3 weights" : "q2 weights");
    if (!w) return 0;
    return qlow_matvec(q3, (float *)out->ptr, w, in_dim, out_dim, (const float *)x->ptr);
}

int sf37_hip_matvec_q3_asym_mapped(sf37_hip_tensor *out, const void *model_map, uint64_t model_size,
                                   uint64_t weight_offset, uint64_t in_dim, uint64_t out_dim,
                                   const sf37_hip_tensor *x) {
    return qlow_mapped(1, out, model_map, model_size, weight_offset, in_dim, out_dim, x);
}

int sf37_hip_matvec_q2_asym_mapped(sf37_hip_tensor *out, const void *model_map, uint64_t model_size,
                                   uint64_t weight_offset, uint64_t in_dim, uint64_t out_dim,
                                   const sf37_hip_tensor *x) {
    return qlow_mapped(0, out, model_map, model_size, weight_offset, in_dim, out_dim, x);
}

/* ------------------------------------------------------------------------ */
/* router (sf37_cuda.cu:4999-5033, 7757-7966)                                */
/* ------------------------------------------------------------------------ */

#define ROUTER_MAX_EXPERTS 1024u

static int router_run(sf37_hip_tensor *selected, sf37_hip_tensor *weights, sf37_hip_tensor *probs,
                      const sf37_hip_tensor *logits, const float *bias, uint32_t n_experts, uint32_t topk,
                      float scale, uint32_t n_tok) {
    if (n_experts > ROUTER_MAX_EXPERTS) {
        fprintf(stderr, "sf37: HIP router_select supports at most %u experts\n", ROUTER_MAX_EXPERTS);
        return 0;
    }
    return LAUNCH(SF37_HIP_STAGE_SELECT, sf37k_router_select((int32_t *)selected->ptr, (float *)weights->ptr,
                                         probs ? (float *)probs->ptr : NULL, (const float *)logits->ptr, bias,
                                         n_experts, topk, scale, n_tok, (sf37_stream_t)g_stream),
                     "router_select launch");
}

int sf37_hip_router_select(sf37_hip_tensor *selected, sf37_hip_tensor *weights, sf37_hip_tensor *probs,
                           const sf37_hip_tensor *logits, const sf37_hip_tensor *bias, uint32_t n_experts,
                           uint32_t topk, float scale) {
    if (!selected || !weights || !logits || !bias || n_experts == 0 || topk == 0 || topk > 16u ||
        !ensure_init())
        return 0;
    if (selected->bytes < (uint64_t)topk * 4u || weights->bytes < (uint64_t)topk * 4u ||
        logits->bytes < (uint64_t)n_experts * 4u || bias->bytes < (uint64_t)n_experts * 4u ||
        (probs && probs->bytes < (uint64_t)n_experts * 4u))
        return 0;
    return router_run(selected, weights, probs, logits, (const float *)bias->ptr, n_experts, topk, scale, 1);
}

int sf37_hip_router_select_mapped(sf37_hip_tensor *selected, sf37_hip_tensor *weights, sf37_hip_tensor *probs,
                                  const sf37_hip_tensor *logits, const void *model_map, uint64_t model_size,
                                  uint64_t bias_offset, uint32_t n_experts, uint32_t topk, float scale) {
    return sf37_hip_router_select_batch_mapped(selected, weights, probs, logits, model_map, model_size,
                                               bias_offset, n_experts, topk, scale, 1);
}

int sf37_hip_router_select_batch_mapped(sf37_hip_tensor *selected, sf37_hip_tensor *weights,
                                        sf37_hip_tensor *probs, const sf37_hip_tensor *logits,
                                        const void *model_map, uint64_t model_size, uint64_t bias_offset,
                                        uint32_t n_experts, uint32_t topk, float scale, uint32_t n_tok) {
    if (!selected || !weights || !logits || !model_map || n_experts == 0 || topk == 0 || topk > 16u ||
        n_tok == 0 || !ensure_init())
        return 0;
    const uint64_t bias_bytes = (uint64_t)n_experts * 4u;
    if (!mapped_range_ok(model_size, bias_offset, bias_bytes) ||
        logits->bytes < (uint64_t)n_tok * n_experts * 4u || selected->bytes < (uint64_t)n_tok * topk * 4u ||
        weights->bytes < (uint64_t)n_tok * topk * 4u || (probs && probs->bytes < (uint64_t)n_tok * n_experts * 4u))
        return 0;
    const float *bias = (const float *)model_ptr(model_map, bias_offset, bias_bytes, "router_bias");
    if (!bias) return 0;
    return router_run(selected, weights, probs, logits, bias, n_experts, topk, scale, n_tok);
}

/* ------------------------------------------------------------------------ */
/* routed experts (sf37_cuda.cu:5269-5781, 7968-8314)                        */
/* ------------------------------------------------------------------------ */

#define DISPATCH_MAX_EXPERTS 512u

typedef struct {
    const uint8_t *gate_w, *up_w, *down_w;
    const int32_t *selected;
    const float *weights;
    uint32_t n_expert, topk, in_dim, mid_dim, out_dim;
    float clamp;
    const float *x;
    uint32_t n_tok;
    const float *comb_base;   /* combine: out = comb_base + sum (may be out) */
    float *comb_resid;        /* combine: comb_resid += comb_base + sum instead */
    hipEvent_t comb_wait;     /* the combine waits for it (comb_base made on another stream) */
} routed_args;

/* The combine of a routed pipeline, after the work comb_base waits for. */
static int routed_combine(const routed_args *a, float *out, const float *down_pair) {
    if (a->comb_wait && !hip_ok(hipStreamWaitEvent(g_stream, a->comb_wait, 0), "shared expert join")) return 0;
    return LAUNCH(SF37_HIP_STAGE_COMBINE, sf37k_moe_combine(out, down_pair, a->comb_base, a->comb_resid, a->topk,
                                                            a->out_dim, a->n_tok, (sf37_stream_t)g_stream),
                  "routed_moe combine launch");
}

/* Scratch of the Q8_K routed pipeline; mid/down_pair/gate/up may point
 * into caller tensors.  Returns the byte size when base == NULL. */
typedef struct {
    void *xq, *midq;
    uint32_t *ginfo, *sorted, *counts, *offsets, *hist;
    float *mid, *down_pair;
    void *x16, *m16;        /* matrix-core path: fp16 codes in MFMA order */
    float *xtab, *mtab;     /* their per-block tables */
    float *xtabs, *mtabs;   /* the tables in dispatch order */
    uint32_t *tiles;
} routed_scratch;

#define PF_TAB_BYTES 32u

static uint64_t routed_layout(const routed_args *a, int slots, int pf, int need_mid, int need_down,
                              char *base, routed_scratch *s) {
    const uint64_t pairs = (uint64_t)a->n_tok * a->topk;
    const uint64_t groups = slots ? a->topk : a->n_expert;
    uint64_t off = 0;
#define RESERVE(field, type, bytes)                                    \
    do {                                                               \
        if (base) s->field = (type)(base + off);                       \
        off = align256(off + (bytes));                                 \
    } while (0)
    if (pf) {
        RESERVE(x16, void *, (uint64_t)a->n_tok * a->in_dim * 2u);
        RESERVE(xtab, float *, (uint64_t)a->n_tok * (a->in_dim / QK) * PF_TAB_BYTES);
        RESERVE(m16, void *, pairs * a->mid_dim * 2u);
        RESERVE(mtab, float *, pairs * (a->mid_dim / QK) * PF_TAB_BYTES);
        RESERVE(tiles, uint32_t *, ((uint64_t)sf37k_pf_max_tiles((uint32_t)pairs, (uint32_t)groups) + 1u) * 16u);
        RESERVE(xtabs, float *, (uint64_t)(a->in_dim / QK) * 5u * sf37k_pf_tab_stride((uint32_t)pairs) * 4u);
        RESERVE(mtabs, float *, (uint64_t)(a->mid_dim / QK) * 5u * sf37k_pf_tab_stride((uint32_t)pairs) * 4u);
    } else {
        RESERVE(xq, void *, (uint64_t)a->n_tok * (a->in_dim / QK) * Q8KB);
        RESERVE(midq, void *, pairs * (a->mid_dim / QK) * Q8KB);
    }
    RESERVE(ginfo, uint32_t *, (3u + 2u * groups) * 4u);
    RESERVE(sorted, uint32_t *, pairs * 4u);
    RESERVE(counts, uint32_t *, (uint64_t)a->n_expert * 4u);
    RESERVE(offsets, uint32_t *, ((uint64_t)a->n_expert + 1u) * 4u);
    RESERVE(hist, uint32_t *, slots ? 0u : sf37k_moe_dispatch_scratch_bytes((uint32_t)pairs, a->n_expert));
    if (need_mid) RESERVE(mid, float *, pairs * a->mid_dim * 4u);
    if (need_down) RESERVE(down_pair, float *, pairs * a->out_dim * 4u);
#undef RESERVE
    return off;
}

/* The matrix-core path takes grouped (not per-slot) batches with enough
 * pairs, dims it tiles, and operand offsets that fit 32 bits. */
static int prefill_eligible(const routed_args *a, int slots) {
    const uint64_t pairs = (uint64_t)a->n_tok * a->topk;
    return !slots && g_opt_prefill && pairs >= (uint64_t)g_opt_prefill_min_pairs &&
           sf37k_pf_supported(a->in_dim, a->mid_dim, a->out_dim) &&
           (uint64_t)a->n_tok * a->in_dim * 2u < (1ull << 32) && pairs * a->mid_dim * 2u < (1ull << 32);
}

/* Shared expert on the matrix cores for prefill batches (k_prefill.hip):
 * out = down(SwiGLU(gate x, up x)) with the Q8_0 arithmetic of
 * sf37_ops.c:57-141, bit-identical to the q8_0_matmul path. */
static int shared_mfma_eligible(uint32_t n_tok, uint32_t D, uint32_t F) {
    return g_opt_prefill && n_tok >= (uint64_t)g_opt_shared_min_tok && sf37k_sh_supported(D, F, D) &&
           (uint64_t)n_tok * D * 2u < (1ull << 32) && (uint64_t)n_tok * F * 2u < (1ull << 32);
}

/* On stream st with its own activation buffer (layer buffer 8), so it can
 * run beside the routed pipeline, which uses the library scratch. */
static int shared_mfma(float *out, float *mid, const uint8_t *gw, const uint8_t *uw, const uint8_t *dw, uint32_t D,
                       uint32_t F, const float *x, uint32_t n_tok, float clamp, hipStream_t hs) {
    if (!aligned4(x) || !aligned4(out) || !aligned4(mid) || !aligned4(gw) || !aligned4(uw) || !aligned4(dw)) return 0;
    const uint64_t maxd = D > F ? D : F;
    const uint64_t ab = (uint64_t)n_tok * maxd, xb = (uint64_t)n_tok * (maxd / 32u) * 4u;
    char *s = (char *)layer_buf(8, align256(ab) + xb);
    if (!s) return 0;
    const sf37_stream_t st = (sf37_stream_t)hs;
    void *a8 = s;
    float *xs = (float *)(s + align256(ab));
    return LAUNCH_ON(hs, SF37_HIP_STAGE_SH_ACT, sf37k_sh_act(a8, xs, x, D, n_tok, st), "shared activation launch") &&
           LAUNCH_ON(hs, SF37_HIP_STAGE_SH_GATE_UP, sf37k_sh_gate_up(mid, gw, uw, a8, xs, n_tok, D, F, clamp, st),
                     "shared gate/up launch") &&
           LAUNCH_ON(hs, SF37_HIP_STAGE_SH_ACT, sf37k_sh_act(a8, xs, mid, F, n_tok, st), "shared mid activation launch") &&
           LAUNCH_ON(hs, SF37_HIP_STAGE_SH_DOWN, sf37k_sh_down(out, dw, a8, xs, n_tok, F, D, st), "shared down launch");
}

/* The side stream and its events (default priority, no blocking with the
 * null stream; ordering with the library stream only through the events). */
static int side_stream_ready(void) {
    if (g_side) return 1;
    if (!hip_ok(hipEventCreateWithFlags(&g_ev_fork, hipEventDisableTiming), "side stream fork event") ||
        !hip_ok(hipEventCreateWithFlags(&g_ev_join, hipEventDisableTiming), "side stream join event") ||
        !hip_ok(hipStreamCreateWithFlags(&g_side, hipStreamNonBlocking), "side stream"))
        return 0;
    return 1;
}

/* Matrix-core pipeline (k_prefill.hip): x to fp16 MFMA codes, dispatch,
 * tiles, gate/up + SwiGLU*w, mid to fp16 MFMA codes, down, combine. */
static int routed_pf(const routed_args *a, const routed_scratch *s, float *out, float *mid, float *down_pair,
                     float *gate_out, float *up_out) {
    const sf37_stream_t st = (sf37_stream_t)g_stream;
    const uint32_t pairs = a->n_tok * a->topk;
    const uint32_t groups = a->n_expert;
    const uint32_t max_tiles = sf37k_pf_max_tiles(pairs, groups);
    const uint32_t tstride = sf37k_pf_tab_stride(pairs);
    return LAUNCH(SF37_HIP_STAGE_PF_ACT_X, sf37k_pf_act(1, s->x16, s->xtab, a->x, a->in_dim, a->n_tok, st),
                  "routed_moe mfma input codes launch") &&
           LAUNCH(SF37_HIP_STAGE_DISPATCH, sf37k_moe_dispatch(s->ginfo, s->sorted, s->counts, s->offsets, a->selected,
                                                              pairs, a->n_expert, s->hist, st),
                  "routed_moe dispatch launch") &&
           LAUNCH(SF37_HIP_STAGE_PF_TILES, sf37k_pf_tiles(s->tiles, s->ginfo, groups, st), "routed_moe tiles launch") &&
           LAUNCH(SF37_HIP_STAGE_PF_TILES, sf37k_pf_tab_sort(s->xtabs, s->xtab, s->sorted, pairs, a->in_dim, a->topk, st),
                  "routed_moe input tables launch") &&
           LAUNCH(SF37_HIP_STAGE_PF_GATE_UP, sf37k_pf_gate_up(mid, gate_out, up_out, a->gate_w, a->up_w, s->x16, s->xtabs,
                                                             s->tiles, s->sorted, a->weights, max_tiles, tstride,
                                                             a->topk, a->in_dim, a->mid_dim, a->clamp, st),
                  "routed_moe mfma gate/up launch") &&
           LAUNCH(SF37_HIP_STAGE_PF_ACT_MID, sf37k_pf_act(0, s->m16, s->mtab, mid, a->mid_dim, pairs, st),
                  "routed_moe mfma mid codes launch") &&
           LAUNCH(SF37_HIP_STAGE_PF_ACT_MID, sf37k_pf_tab_sort(s->mtabs, s->mtab, s->sorted, pairs, a->mid_dim, 1u, st),
                  "routed_moe mid tables launch") &&
           LAUNCH(SF37_HIP_STAGE_PF_DOWN, sf37k_pf_down(down_pair, a->down_w, s->m16, s->mtabs, s->tiles, s->sorted,
                                                       max_tiles, tstride, a->mid_dim, a->out_dim, st),
                  "routed_moe mfma down launch") &&
           routed_combine(a, out, down_pair);
}

/* Q8_K pipeline: quantize x, group pairs by expert (slots = one group per
 * slot of a single token), gate/up + SwiGLU*w, quantize mid, down, combine. */
static int routed_q8k(const routed_args *a, float *out, float *mid, float *down_pair, float *gate_out,
                      float *up_out, int slots) {
    if (!aligned4(a->gate_w) || !aligned4(a->up_w) || !aligned4(a->down_w) || !aligned4(a->x) ||
        !aligned4(out) || (mid && !aligned4(mid)) || (down_pair && !aligned4(down_pair)))
        return 0;
    routed_scratch s;
    memset(&s, 0, sizeof(s));
    const int pf = prefill_eligible(a, slots);
    const uint64_t bytes = routed_layout(a, slots, pf, mid == NULL, down_pair == NULL, NULL, &s);
    char *base = scratch_get(bytes, "routed moe scratch");
    if (!base) return 0;
    routed_layout(a, slots, pf, mid == NULL, down_pair == NULL, base, &s);
    if (!mid) mid = s.mid;
    if (!down_pair) down_pair = s.down_pair;
    if (pf) return routed_pf(a, &s, out, mid, down_pair, gate_out, up_out);
    const sf37_stream_t st = (sf37_stream_t)g_stream;
    const uint32_t pairs = a->n_tok * a->topk;
    const uint32_t groups = slots ? a->topk : a->n_expert;
    if (!LAUNCH(SF37_HIP_STAGE_Q8K_X, sf37k_q8k_quantize(s.xq, a->x, a->in_dim, a->n_tok, st), "routed_moe q8k input quantize launch"))
        return 0;
    if (slots) {
        if (!LAUNCH(SF37_HIP_STAGE_DISPATCH, sf37k_moe_slots(s.ginfo, s.sorted, a->selected, a->topk, a->n_expert, st),
                       "routed_moe slot groups launch"))
            return 0;
    } else if (!LAUNCH(SF37_HIP_STAGE_DISPATCH, sf37k_moe_dispatch(s.ginfo, s.sorted, s.counts, s.offsets, a->selected, pairs,
                                             a->n_expert, s.hist, st),
                          "routed_moe dispatch launch")) {
        return 0;
    }
    if (!LAUNCH(SF37_HIP_STAGE_GATE_UP, sf37k_moe_gate_up(mid, gate_out, up_out, a->gate_w, a->up_w, s.xq, s.ginfo, s.sorted,
                                     a->weights, groups, pairs, a->topk, a->in_dim, a->mid_dim, a->clamp, st),
                   "routed_moe q8k gate/up launch"))
        return 0;
    if (!LAUNCH(SF37_HIP_STAGE_Q8K_MID, sf37k_q8k_quantize(s.midq, mid, a->mid_dim, pairs, st), "routed_moe q8k mid quantize launch"))
        return 0;
    if (!LAUNCH(SF37_HIP_STAGE_DOWN, sf37k_moe_down(down_pair, a->down_w, s.midq, s.ginfo, s.sorted, groups, pairs, a->mid_dim,
                                  a->out_dim, st),
                   "routed_moe q8k down launch"))
        return 0;
    return routed_combine(a, out, down_pair);
}

/* ---- fused decode path (k_decode.hip) ------------------------------------ */

/* Extra inputs of the fused path beyond the routed arguments. */
typedef struct {
    uint32_t flags;
    const float *router_w, *router_bias, *logits_sel;
    const uint8_t *sh_gate, *sh_up, *sh_down;
    float scale, clamp_shared;
    int32_t *sel;   /* selection output when SELECT (NULL = scratch) */
    float *wts;
    const uint16_t *norm_w;  /* NORM: bf16 norm weights, epsilon, normalised rows (or NULL) */
    float eps;
    float *xn;
    float *sh_out;           /* SHBASE: the shared expert's rows, added by the combine */
    hipEvent_t comb_wait;    /* SHBASE: the combine waits for it (sh_out made on another stream) */
} dec_extra;

static uint32_t *dec_counters(uint64_t words) {
    g_mem_requests++;
    if (g_dec_cnt && words <= g_dec_cnt_words) return g_dec_cnt;
    if (g_dec_cnt) {
        if (!hip_ok(hipStreamSynchronize(g_stream), "decode counter sync")) return NULL;
        (void)hipFree(g_dec_cnt);
        g_dec_cnt = NULL;
        g_dec_cnt_words = 0;
    }
    void *p = NULL;
    if (!hip_ok(hipMalloc(&p, words * 4u + SF37_PAD), "decode counter alloc")) return NULL;
    if (!hip_ok(hipMemset(p, 0, words * 4u + SF37_PAD), "decode counter clear") ||
        !hip_ok(hipDeviceSynchronize(), "decode counter clear sync")) {
        (void)hipFree(p);
        return NULL;
    }
    g_dec_cnt = (uint32_t *)p;
    g_dec_cnt_words = words;
    return g_dec_cnt;
}

/* Shapes the fused kernels take: at most 16 tokens and top-16, square
 * down projection, 256-multiple dims, the Q8_K numerics the staged path
 * would pick, and LDS within 64 KiB. */
static int decode_eligible(const routed_args *a, uint32_t flags) {
    if (!g_opt_decode || a->n_tok == 0 || a->n_tok > SF37_DEC_MAX_TOK || a->topk == 0 || a->topk > 16u ||
        a->topk > a->n_expert || a->out_dim != a->in_dim || a->in_dim % QK != 0 || a->mid_dim % QK != 0 ||
        !q8k_use_for(a->mid_dim) || !q8k_use_for(a->out_dim))
        return 0;
    if ((flags & SF37_DEC_SELECT) && a->n_expert > ROUTER_MAX_EXPERTS) return 0;
    if ((flags & SF37_DEC_SLOTS) && a->n_tok != 1u) return 0;
    return sf37k_decode_supported(a->n_tok, a->topk, a->n_expert, a->in_dim, a->mid_dim,
                                  (flags & SF37_DEC_SHARED) != 0);
}

/* out = [shared +] sum over slots of the routed experts; mid / down_pair /
 * gate_out / up_out receive per-pair results when given (pairs x F, pairs x
 * D), else scratch is used. */
/* fixed_base != NULL: lay the scratch out in [fixed_base, + fixed_bytes) and
 * use fixed_cnt as the item queues instead of the library's allocations. */
/* With size_only, only the scratch bytes this call needs are returned there
 * (nothing is launched). */
static int decode_run_in(const routed_args *a, const dec_extra *ex, float *out, float *mid, float *down_pair,
                         float *gate_out, float *up_out, char *fixed_base, uint64_t fixed_bytes,
                         uint32_t *fixed_cnt, uint64_t *size_only) {
    if (!aligned4(a->gate_w) || !aligned4(a->up_w) || !aligned4(a->down_w) || !aligned4(a->x) ||
        !aligned4(out) || (mid && !aligned4(mid)) || (down_pair && !aligned4(down_pair)) ||
        (gate_out && !aligned4(gate_out)) || (up_out && !aligned4(up_out)))
        return 0;
    const uint32_t T = a->n_tok, E = a->n_expert, K = a->in_dim, F = a->mid_dim, TK = a->topk;
    const uint64_t P = (uint64_t)T * TK;
    /* groups: one per expert id, and with SH9 the shared expert (id E) as
     * up to n_tok groups of its pairs */
    const uint32_t n_grp = E + ((ex->flags & SF37_DEC_SH9) ? T : 0u);
    const uint32_t G = (uint32_t)(P < n_grp ? P : n_grp);
    const int sh = (ex->flags & SF37_DEC_SHARED) != 0;
    sf37_dec_params p;
    memset(&p, 0, sizeof(p));
    p.T = T;
    p.E = E;
    p.K = K;
    p.F = F;
    p.topk = TK;
    p.G = G;
    p.scale = ex->scale;
    p.clamp_routed = a->clamp;
    p.clamp_shared = ex->clamp_shared;
    p.flags = ex->flags | ((uint64_t)T <= (uint64_t)g_opt_upsel_max_tok ? SF37_DEC_UPSEL : 0u);
    /* one token: each slot its own group, in slot order (the slot-order
     * combine makes the grouping order immaterial; the expert-sorted
     * grouping only costs its scan) */
    if (T == 1u && TK <= E) p.flags |= SF37_DEC_SLOTS;
    p.x = a->x;
    p.router_w = ex->router_w;
    p.router_bias = ex->router_bias;
    p.logits_sel = ex->logits_sel;
    p.gate_w = a->gate_w;
    p.up_w = a->up_w;
    p.down_w = a->down_w;
    p.sh_gate = ex->sh_gate;
    p.sh_up = ex->sh_up;
    p.sh_down = ex->sh_down;
    p.out = out;
    /* scratch layout */
    uint64_t off = 0, o_xq, o_xq8, o_xs8, o_gi, o_so, o_mid = 0, o_mq, o_gu = 0, o_smq = 0, o_sms = 0, o_dp = 0,
                      o_sho = 0, o_lg = 0, o_ck = 0, o_cp = 0, o_sel = 0, o_wts = 0, o_go = 0, o_uo = 0;
#define TAKE(var, bytes)            \
    do {                            \
        var = off;                  \
        off = align256(off + (bytes)); \
    } while (0)
    TAKE(o_xq, (uint64_t)T * (K / QK) * SF37_DEC_ACT_BYTES);
    TAKE(o_xq8, (uint64_t)T * K);
    TAKE(o_xs8, (uint64_t)T * (K / 32u) * 4u);
    TAKE(o_gi, (3u + 2u * (uint64_t)G) * 4u);
    TAKE(o_so, P * 4u);
    if (!mid) TAKE(o_mid, P * F * 4u);
    if (!gate_out) TAKE(o_go, P * F * 4u);
    if (!up_out) TAKE(o_uo, P * F * 4u);
    TAKE(o_mq, P * (F / QK) * SF37_DEC_ACT_BYTES);
    if (sh) {
        TAKE(o_gu, 2u * (uint64_t)T * F * 4u);
        TAKE(o_smq, (uint64_t)T * F);
        TAKE(o_sms, (uint64_t)T * (F / 32u) * 4u);
        TAKE(o_sho, (uint64_t)T * K * 4u);
    }
    if (!down_pair) TAKE(o_dp, P * K * 4u);
    if (ex->flags & SF37_DEC_ROUTER) TAKE(o_lg, (uint64_t)T * E * 4u);
    if (ex->flags & SF37_DEC_SELECT) {
        TAKE(o_ck, (uint64_t)T * E * 8u);
        TAKE(o_cp, (uint64_t)T * E * 4u);
    }
    if ((ex->flags & SF37_DEC_SELECT) && !ex->sel) TAKE(o_sel, P * 4u);
    if ((ex->flags & SF37_DEC_SELECT) && !ex->wts) TAKE(o_wts, P * 4u);
#undef TAKE
    if (size_only) {
        *size_only = off;
        return 1;
    }
    char *base;
    uint32_t *cnt;
    if (fixed_base) {
        if (off > fixed_bytes) {
            fprintf(stderr, "sf37: HIP moe_layer_noalloc: this batch needs %llu bytes of scratch, the static "
                            "scratch holds %llu\n", (unsigned long long)off, (unsigned long long)fixed_bytes);
            return 0;
        }
        base = fixed_base;
        cnt = fixed_cnt;
    } else {
        base = scratch_get(off, "decode scratch");
        cnt = dec_counters((uint64_t)sf37k_decode_counters(T, TK, E, K, F));
    }
    if (!base || !cnt) return 0;
    p.xq = base + o_xq;
    p.xq8 = (int8_t *)(base + o_xq8);
    p.xs8 = (float *)(base + o_xs8);
    p.ginfo = (uint32_t *)(base + o_gi);
    p.sorted = (uint32_t *)(base + o_so);
    p.mid = mid ? mid : (float *)(base + o_mid);
    p.gate_out = gate_out ? gate_out : (float *)(base + o_go);
    p.up_out = up_out ? up_out : (float *)(base + o_uo);
    p.midq = base + o_mq;
    if (sh) {
        p.sh_gu = (float *)(base + o_gu);
        p.sh_mq = (int8_t *)(base + o_smq);
        p.sh_ms = (float *)(base + o_sms);
        p.sh_out = (float *)(base + o_sho);
    }
    p.down_pair = down_pair ? down_pair : (float *)(base + o_dp);
    p.logits = (ex->flags & SF37_DEC_ROUTER) ? (float *)(base + o_lg) : NULL;
    if (ex->flags & SF37_DEC_SELECT) {
        p.cand_key = (uint64_t *)(base + o_ck);
        p.cand_p = (float *)(base + o_cp);
        p.sel = ex->sel ? ex->sel : (int32_t *)(base + o_sel);
        p.wts = ex->wts ? ex->wts : (float *)(base + o_wts);
        if (!p.logits_sel) p.logits_sel = p.logits;
        if (!p.logits_sel || !p.router_bias) return 0;
    } else {
        p.sel = (int32_t *)a->selected;
        p.wts = (float *)a->weights;
    }
    if ((ex->flags & SF37_DEC_ROUTER) && !p.router_w) return 0;
    if ((sh || (ex->flags & SF37_DEC_SH9)) && (!p.sh_gate || !p.sh_up || !p.sh_down)) return 0;
    if ((ex->flags & SF37_DEC_SH9) && (sh || (ex->flags & SF37_DEC_SHBASE) || !(ex->flags & SF37_DEC_SELECT) || TK < 2u))
        return 0;
    if (ex->flags & SF37_DEC_SHBASE) {
        if (sh || !ex->sh_out) return 0;
        p.sh_out = ex->sh_out;
    }
    if ((ex->flags & SF37_DEC_NORM) && !ex->norm_w) return 0;
    /* automatic share (-1): half the up items dynamic up to 8 tokens, a
     * quarter above (measured best at 1..16 tokens, 288 experts, top-8) */
    p.up_dyn_pct = g_opt_up_dyn_pct >= 0 ? (uint32_t)g_opt_up_dyn_pct : (T <= 8u ? 50u : 25u);
    p.up_wgs = (uint32_t)g_opt_up_wgs;
    p.dn_wgs = (uint32_t)g_opt_dn_wgs;
    p.norm_w = ex->norm_w;
    p.eps = ex->eps;
    p.xn = ex->xn;
    p.cnt = cnt;
    const sf37_stream_t st = (sf37_stream_t)g_stream;
    const int down_combine = g_opt_down_combine && sf37k_decode_down_combine_supported(&p);
    /* a shared expert made on another stream joins before the launch that adds it */
    const hipEvent_t join = (ex->flags & SF37_DEC_SHBASE) ? ex->comb_wait : NULL;
    return LAUNCH(SF37_HIP_STAGE_DEC_ROUTE, sf37k_decode_route(&p, st), "decode route launch") &&
           ((p.flags & SF37_DEC_UPSEL) ||
            LAUNCH(SF37_HIP_STAGE_DEC_SELECT, sf37k_decode_select(&p, st), "decode select launch")) &&
           LAUNCH(SF37_HIP_STAGE_DEC_UP, sf37k_decode_up(&p, st), "decode up launch") &&
           LAUNCH(SF37_HIP_STAGE_DEC_MID, sf37k_decode_mid(&p, st), "decode mid launch") &&
           (down_combine
                ? (!join || hip_ok(hipStreamWaitEvent(g_stream, join, 0), "shared expert join")) &&
                      LAUNCH(SF37_HIP_STAGE_DEC_DOWN, sf37k_decode_down_combine(&p, st), "decode down+combine launch")
                : LAUNCH(SF37_HIP_STAGE_DEC_DOWN, sf37k_decode_down(&p, st), "decode down launch") &&
                      (!join || hip_ok(hipStreamWaitEvent(g_stream, join, 0), "shared expert join")) &&
                      LAUNCH(SF37_HIP_STAGE_DEC_COMBINE, sf37k_decode_combine(&p, st), "decode combine launch"));
}

static int decode_run(const routed_args *a, const dec_extra *ex, float *out, float *mid, float *down_pair,
                      float *gate_out, float *up_out) {
    return decode_run_in(a, ex, out, mid, down_pair, gate_out, up_out, NULL, 0, NULL, NULL);
}

/* fp32-activation path for one token (sf37_cuda.cu:5382-5446). */
static int routed_f32(const routed_args *a, float *out, float *mid, float *down_slot, float *gate_out,
                      float *up_out) {
    const sf37_stream_t st = (sf37_stream_t)g_stream;
    if (!LAUNCH(SF37_HIP_STAGE_GATE_UP, sf37k_moe_gate_up_f32(mid, gate_out, up_out, a->gate_w, a->up_w, a->x, a->selected,
                                         a->weights, a->topk, a->in_dim, a->mid_dim, a->n_expert, a->clamp, st),
                   "routed_moe gate/up launch"))
        return 0;
    if (!LAUNCH(SF37_HIP_STAGE_DOWN, sf37k_moe_down_f32(down_slot, a->down_w, mid, a->selected, a->topk, a->mid_dim, a->out_dim,
                                      a->n_expert, st),
                   "routed_moe down launch"))
        return 0;
    return LAUNCH(SF37_HIP_STAGE_COMBINE, sf37k_moe_combine(out, down_slot, NULL, NULL, a->topk, a->out_dim, 1, st), "routed_moe sum launch");
}

static int routed_one_impl(sf37_hip_tensor *out, sf37_hip_tensor *gate, sf37_hip_tensor *up,
                           sf37_hip_tensor *mid, sf37_hip_tensor *down, const routed_args *a) {
    float *go = g_opt_write_gate_up ? (float *)gate->ptr : NULL;
    float *uo = g_opt_write_gate_up ? (float *)up->ptr : NULL;
    if (decode_eligible(a, SF37_DEC_SLOTS)) {
        dec_extra ex;
        memset(&ex, 0, sizeof(ex));
        ex.flags = SF37_DEC_SLOTS;
        return decode_run(a, &ex, (float *)out->ptr, (float *)mid->ptr, (float *)down->ptr, go, uo);
    }
    if (q8k_use_for(a->mid_dim) && q8k_use_for(a->out_dim))
        return routed_q8k(a, (float *)out->ptr, (float *)mid->ptr, (float *)down->ptr, go, uo, 1);
    return routed_f32(a, (float *)out->ptr, (float *)mid->ptr, (float *)down->ptr, go, uo);
}

static int routed_common_checks(sf37_hip_tensor *out, sf37_hip_tensor *gate, sf37_hip_tensor *up,
                                sf37_hip_tensor *mid, sf37_hip_tensor *down, const sf37_hip_tensor *selected,
                                const sf37_hip_tensor *weights, uint32_t n_total_expert, uint32_t topk,
                                uint32_t in_dim, uint32_t mid_dim, uint32_t out_dim, const sf37_hip_tensor *x,
                                uint32_t n_tok) {
    if (!out || !gate || !up || !mid || !down || !selected || !weights || !x || n_total_expert == 0 ||
        topk == 0 || in_dim == 0 || mid_dim == 0 || out_dim == 0 || n_tok == 0 || in_dim % QK != 0 ||
        mid_dim % QK != 0)
        return 0;
    const uint64_t pm = (uint64_t)topk * mid_dim * 4u;
    return out->bytes >= (uint64_t)n_tok * out_dim * 4u && gate->bytes >= pm && up->bytes >= pm &&
           mid->bytes >= pm && down->bytes >= (uint64_t)topk * out_dim * 4u &&
           selected->bytes >= (uint64_t)n_tok * topk * 4u && weights->bytes >= (uint64_t)n_tok * topk * 4u &&
           x->bytes >= (uint64_t)n_tok * in_dim * 4u;
}

int sf37_hip_routed_moe_one(sf37_hip_tensor *out, sf37_hip_tensor *gate, sf37_hip_tensor *up,
                            sf37_hip_tensor *mid, sf37_hip_tensor *down, const sf37_hip_tensor *moe_gate,
                            const sf37_hip_tensor *moe_up, const sf37_hip_tensor *moe_down,
                            const sf37_hip_tensor *selected, const sf37_hip_tensor *weights,
                            uint32_t n_total_expert, uint32_t topk, uint32_t in_dim, uint32_t expert_mid_dim,
                            uint32_t out_dim, float clamp, const sf37_hip_tensor *x) {
    if (!ensure_init() || !moe_gate || !moe_up || !moe_down ||
        !routed_common_checks(out, gate, up, mid, down, selected, weights, n_total_expert, topk, in_dim,
                              expert_mid_dim, out_dim, x, 1))
        return 0;
    const uint64_t gb = (uint64_t)n_total_expert * expert_mid_dim * (in_dim / QK) * Q3B;
    const uint64_t db = (uint64_t)n_total_expert * out_dim * (expert_mid_dim / QK) * Q2B;
    if (moe_gate->bytes < gb || moe_up->bytes < gb || moe_down->bytes < db) return 0;
    routed_args a = {(const uint8_t *)moe_gate->ptr, (const uint8_t *)moe_up->ptr, (const uint8_t *)moe_down->ptr,
                     (const int32_t *)selected->ptr, (const float *)weights->ptr, n_total_expert, topk, in_dim,
                     expert_mid_dim, out_dim, clamp, (const float *)x->ptr, 1, NULL, NULL, NULL};
    return routed_one_impl(out, gate, up, mid, down, &a);
}

static int resolve_experts(const void *model_map, uint64_t model_size, uint64_t gate_offset, uint64_t up_offset,
                           uint64_t down_offset, uint32_t n_total_expert, uint32_t in_dim, uint32_t mid_dim,
                           uint32_t out_dim, const uint8_t **g, const uint8_t **u, const uint8_t **d) {
    const uint64_t gb = (uint64_t)n_total_expert * mid_dim * (in_dim / QK) * Q3B;
    const uint64_t db = (uint64_t)n_total_expert * out_dim * (mid_dim / QK) * Q2B;
    if (!mapped_range_ok(model_size, gate_offset, gb) || !mapped_range_ok(model_size, up_offset, gb) ||
        !mapped_range_ok(model_size, down_offset, db))
        return 0;
    *g = (const uint8_t *)model_ptr(model_map, gate_offset, gb, "moe_gate");
    *u = (const uint8_t *)model_ptr(model_map, up_offset, gb, "moe_up");
    *d = (const uint8_t *)model_ptr(model_map, down_offset, db, "moe_down");
    return *g && *u && *d;
}

int sf37_hip_routed_moe_one_mapped(sf37_hip_tensor *out, sf37_hip_tensor *gate, sf37_hip_tensor *up,
                                   sf37_hip_tensor *mid, sf37_hip_tensor *down, const void *model_map,
                                   uint64_t model_size, uint64_t gate_offset, uint64_t up_offset,
                                   uint64_t down_offset, const sf37_hip_tensor *selected,
                                   const sf37_hip_tensor *weights, uint32_t n_total_expert, uint32_t topk,
                                   uint32_t in_dim, uint32_t expert_mid_dim, uint32_t out_dim, float clamp,
                                   const sf37_hip_tensor *x) {
    if (!model_map || !ensure_init() ||
        !routed_common_checks(out, gate, up, mid, down, selected, weights, n_total_expert, topk, in_dim,
                              expert_mid_dim, out_dim, x, 1))
        return 0;
    routed_args a = {NULL, NULL, NULL, (const int32_t *)selected->ptr, (const float *)weights->ptr, n_total_expert,
                     topk, in_dim, expert_mid_dim, out_dim, clamp, (const float *)x->ptr, 1, NULL, NULL, NULL};
    if (!resolve_experts(model_map, model_size, gate_offset, up_offset, down_offset, n_total_expert, in_dim,
                         expert_mid_dim, out_dim, &a.gate_w, &a.up_w, &a.down_w))
        return 0;
    return routed_one_impl(out, gate, up, mid, down, &a);
}

int sf37_hip_routed_moe_batch_mapped(sf37_hip_tensor *out, sf37_hip_tensor *gate, sf37_hip_tensor *up,
                                     sf37_hip_tensor *mid, sf37_hip_tensor *down, const void *model_map,
                                     uint64_t model_size, uint64_t gate_offset, uint64_t up_offset,
                                     uint64_t down_offset, const sf37_hip_tensor *selected,
                                     const sf37_hip_tensor *weights, uint32_t n_total_expert, uint32_t topk,
                                     uint32_t in_dim, uint32_t expert_mid_dim, uint32_t out_dim, float clamp,
                                     const sf37_hip_tensor *x, uint32_t n_tok) {
    if (!model_map || !ensure_init() ||
        !routed_common_checks(out, gate, up, mid, down, selected, weights, n_total_expert, topk, in_dim,
                              expert_mid_dim, out_dim, x, n_tok))
        return 0;
    routed_args a = {NULL, NULL, NULL, (const int32_t *)selected->ptr, (const float *)weights->ptr, n_total_expert,
                     topk, in_dim, expert_mid_dim, out_dim, clamp, (const float *)x->ptr, n_tok, NULL, NULL, NULL};
    if (!resolve_experts(model_map, model_size, gate_offset, up_offset, down_offset, n_total_expert, in_dim,
                         expert_mid_dim, out_dim, &a.gate_w, &a.up_w, &a.down_w))
        return 0;
    const uint64_t pairs = (uint64_t)n_tok * topk;
    if (n_tok > 1u && pairs <= 0xffffffffu && n_total_expert <= DISPATCH_MAX_EXPERTS &&
        q8k_use_for(expert_mid_dim) && q8k_use_for(out_dim)) {
        /* the caller's mid receives the per-pair SwiGLU output when it is big
         * enough (sf37_cuda.cu:5665-5674) */
        float *mid_pair = mid->bytes >= pairs * expert_mid_dim * 4u ? (float *)mid->ptr : NULL;
        if (decode_eligible(&a, 0)) {
            dec_extra ex;
            memset(&ex, 0, sizeof(ex));
            return decode_run(&a, &ex, (float *)out->ptr, mid_pair, NULL, NULL, NULL);
        }
        return routed_q8k(&a, (float *)out->ptr, mid_pair, NULL, NULL, NULL, 0);
    }
    /* per-token loop, as the reference's fallback (sf37_cuda.cu:5734-5780) */
    for (uint32_t t = 0; t < n_tok; t++) {
        sf37_hip_tensor ov = {(char *)out->ptr + (uint64_t)t * out_dim * 4u, (uint64_t)out_dim * 4u, 0};
        const uint64_t mp = (uint64_t)topk * expert_mid_dim * 4u;
        sf37_hip_tensor mv = {mid->bytes >= (uint64_t)n_tok * mp ? (char *)mid->ptr + (uint64_t)t * mp : mid->ptr, mp,
                              0};
        routed_args at = a;
        at.selected = a.selected + (uint64_t)t * topk;
        at.weights = a.weights + (uint64_t)t * topk;
        at.x = a.x + (uint64_t)t * in_dim;
        at.n_tok = 1;
        if (!routed_one_impl(&ov, gate, up, &mv, down, &at)) return 0;
    }
    return 1;
}

/* ------------------------------------------------------------------------ */
/* extensions                                                                */
/* ------------------------------------------------------------------------ */

int sf37_hip_q8k_quantize(sf37_hip_tensor *out, const sf37_hip_tensor *x, uint32_t in_dim, uint32_t n_rows) {
    if (!out || !x || in_dim % QK != 0 || !ensure_init()) return 0;
    if (out->bytes < (uint64_t)n_rows * (in_dim / QK) * Q8KB || x->bytes < (uint64_t)n_rows * in_dim * 4u) return 0;
    return LAUNCH(SF37_HIP_STAGE_Q8K_X, sf37k_q8k_quantize(out->ptr, (const float *)x->ptr, in_dim, n_rows, (sf37_stream_t)g_stream),
                     "q8k quantize launch");
}

int sf37_hip_moe_dispatch(sf37_hip_tensor *counts, sf37_hip_tensor *offsets, sf37_hip_tensor *sorted_pairs,
                          const sf37_hip_tensor *selected, uint32_t n_pairs, uint32_t n_expert) {
    if (!counts || !offsets || !sorted_pairs || !selected || n_expert == 0 || n_expert > DISPATCH_MAX_EXPERTS ||
        !ensure_init())
        return 0;
    if (counts->bytes < (uint64_t)n_expert * 4u || offsets->bytes < ((uint64_t)n_expert + 1u) * 4u ||
        sorted_pairs->bytes < (uint64_t)n_pairs * 4u || selected->bytes < (uint64_t)n_pairs * 4u)
        return 0;
    const uint64_t gbytes = align256((3u + 2u * (uint64_t)n_expert) * 4u);
    char *scr = scratch_get(gbytes + sf37k_moe_dispatch_scratch_bytes(n_pairs, n_expert), "dispatch groups");
    if (!scr) return 0;
    uint32_t *ginfo = (uint32_t *)scr, *hist = (uint32_t *)(scr + gbytes);
    return LAUNCH(SF37_HIP_STAGE_DISPATCH, sf37k_moe_dispatch(ginfo, (uint32_t *)sorted_pairs->ptr, (uint32_t *)counts->ptr,
                                        (uint32_t *)offsets->ptr, (const int32_t *)selected->ptr, n_pairs,
                                        n_expert, hist, (sf37_stream_t)g_stream),
                     "dispatch launch");
}

/* Whole layer: the layer buffers (layer_buf) hold logits, selection, the
 * shared expert's activations and, on the fp32 path, the routed output; the
 * routed pipeline then takes the scratch area. */
/* The RMSNorm and residual of an FFN block around the layer (sf37_hip_moe_block). */
typedef struct {
    const uint16_t *norm_w;
    float eps;
    float *xn;
} block_norm;

static int moe_layer_impl(sf37_hip_tensor *out, sf37_hip_tensor *selected, sf37_hip_tensor *weights,
                          const sf37_hip_moe_layer_weights *w, const sf37_hip_tensor *logits_in,
                          const sf37_hip_tensor *x, uint32_t n_tok, const block_norm *bn, float *resid);

int sf37_hip_moe_layer(sf37_hip_tensor *out, sf37_hip_tensor *selected, sf37_hip_tensor *weights,
                       const sf37_hip_moe_layer_weights *w, const sf37_hip_tensor *logits_in,
                       const sf37_hip_tensor *x, uint32_t n_tok) {
    return moe_layer_impl(out, selected, weights, w, logits_in, x, n_tok, NULL, NULL);
}

static sf37_hip_tensor *g_block_buf[2];
static uint64_t g_block_buf_bytes[2];

/* Layer buffer i of at least bytes (kept and grown across calls). */
static void *layer_buf(int i, uint64_t bytes) {
    g_mem_requests++;
    if (!g_layer_bufs[i] || g_layer_buf_bytes[i] < bytes) {
        /* a buffer the side stream may still read or write is freed only
         * after both streams' queued work */
        if (g_layer_bufs[i] && (!hip_ok(hipStreamSynchronize(g_stream), "layer buffer sync") ||
                                (g_side && !hip_ok(hipStreamSynchronize(g_side), "side stream sync"))))
            return NULL;
        if (g_layer_bufs[i]) sf37_hip_tensor_free(g_layer_bufs[i]);
        g_layer_bufs[i] = sf37_hip_tensor_alloc(bytes);
        g_layer_buf_bytes[i] = g_layer_bufs[i] ? bytes : 0;
        if (!g_layer_bufs[i]) return NULL;
    }
    return g_layer_bufs[i]->ptr;
}

static int tensor_holds(const sf37_hip_tensor *t, uint64_t bytes, const char *what) {
    if (t && t->bytes >= bytes) return 1;
    fprintf(stderr, "sf37: HIP moe layer: %s tensor holds %llu bytes, %llu needed\n", what,
            (unsigned long long)(t ? t->bytes : 0), (unsigned long long)bytes);
    return 0;
}

/* Every weight tensor of a layer is at least as large as its shape, in the
 * formats the layer names. */
static int layer_weights_ok(const sf37_hip_moe_layer_weights *w, int run_router) {
    const uint64_t E = w->n_expert, D = w->in_dim, F = w->mid_dim;
    const uint64_t q3 = E * F * (D / QK) * Q3B, q2 = E * D * (F / QK) * Q2B;
    const uint32_t rt = w->router_type, st = w->shared_type;
    if ((rt != SF37_HIP_TYPE_F32 && rt != SF37_HIP_TYPE_BF16 && rt != SF37_HIP_TYPE_Q8_0) ||
        (st != 0u && st != SF37_HIP_TYPE_Q8_0 && st != SF37_HIP_TYPE_Q3GU)) {
        fprintf(stderr, "sf37: HIP moe layer: router type %u / shared type %u not supported\n", rt, st);
        return 0;
    }
    const uint64_t rb = rt == SF37_HIP_TYPE_F32 ? E * D * 4u
                        : rt == SF37_HIP_TYPE_BF16 ? E * D * 2u : E * ((D + 31u) / 32u) * Q8B;
    const int sq3 = st == SF37_HIP_TYPE_Q3GU;
    const uint64_t s_gu = sq3 ? F * (D / QK) * Q3B : F * ((D + 31u) / 32u) * Q8B;
    const uint64_t s_d = sq3 ? D * (F / QK) * Q2B : D * ((F + 31u) / 32u) * Q8B;
    return (!run_router || tensor_holds(w->router, rb, "router")) &&
           tensor_holds(w->router_bias, E * 4u, "router bias") && tensor_holds(w->gate, q3, "gate") &&
           tensor_holds(w->up, q3, "up") && tensor_holds(w->down, q2, "down") &&
           tensor_holds(w->sh_gate, s_gu, "shared gate") && tensor_holds(w->sh_up, s_gu, "shared up") &&
           tensor_holds(w->sh_down, s_d, "shared down");
}

/* Is [p, p + bytes) inside a registered (non-cache) map range?  Weights there
 * stay put until the range is dropped, so derived copies may be kept. */
static int dev_registered(const void *p, uint64_t bytes) {
    for (size_t i = 0; i < g_nranges; i++) {
        const uintptr_t a = (uintptr_t)p, lo = (uintptr_t)g_ranges[i].dev;
        if (!g_ranges[i].cache && a >= lo && bytes <= g_ranges[i].bytes && a - lo <= g_ranges[i].bytes - bytes)
            return 1;
    }
    return 0;
}

/* Router logits of a BF16 or Q8_0 router (the F32 router runs inside the
 * decode launches or through router_matmul below). */
static int layer_router_typed(float *logits, const sf37_hip_moe_layer_weights *w, const float *x, uint32_t n_tok) {
    const uint64_t E = w->n_expert, D = w->in_dim;
    if (w->router_type == SF37_HIP_TYPE_Q8_0)
        return q8_0_run(logits, NULL, (const uint8_t *)w->router->ptr, NULL, D, E, x, n_tok);
    const float *f;
    if (dev_registered(w->router->ptr, E * D * 2u)) {
        f = bf16_resident_f32(w->router->ptr, E * D);
    } else {
        f = (const float *)layer_buf(7, E * D * 4u);
        if (f && !LAUNCH(SF37_HIP_STAGE_OTHER, sf37k_bf16_widen((float *)f, (const uint16_t *)w->router->ptr, E * D,
                                                                 (sf37_stream_t)g_stream),
                         "router bf16 widen launch"))
            return 0;
    }
    return f && LAUNCH(SF37_HIP_STAGE_ROUTER, router_matmul(logits, f, x, D, E, n_tok, (sf37_stream_t)g_stream),
                       "moe_layer bf16 router launch");
}

/* One decode_run_in on the side stream with scratch of its own (layer
 * buffer 9: the counters, then the decode scratch), forked from the library
 * stream now; *joined names the event the launch that uses its output must
 * wait for. */
static int decode_run_side(const routed_args *a, const dec_extra *ex, float *out, hipEvent_t *joined) {
    uint64_t need = 0;
    if (!decode_run_in(a, ex, out, NULL, NULL, NULL, NULL, NULL, 0, NULL, &need)) return 0;
    const uint64_t cnt_bytes =
        align256((uint64_t)sf37k_decode_counters(a->n_tok, a->topk, a->n_expert, a->in_dim, a->mid_dim) * 4u);
    const int fresh = !g_layer_bufs[9] || g_layer_buf_bytes[9] < cnt_bytes + need;
    char *buf = (char *)layer_buf(9, cnt_bytes + need);
    /* the kernels leave their counters zero; a new buffer starts so */
    if (!buf || (fresh && !hip_ok(hipMemset(buf, 0, cnt_bytes), "side counters clear")) || !side_stream_ready() ||
        !hip_ok(hipEventRecord(g_ev_fork, g_stream), "side fork") ||
        !hip_ok(hipStreamWaitEvent(g_side, g_ev_fork, 0), "side fork wait"))
        return 0;
    hipStream_t main = g_stream;
    g_stream = g_side;   /* the library's launches of this call go to the side stream */
    const int ok = decode_run_in(a, ex, out, NULL, NULL, NULL, NULL, buf + cnt_bytes, need, (uint32_t *)buf, NULL) &&
                   hip_ok(hipEventRecord(g_ev_join, g_side), "side join record");
    g_stream = main;
    *joined = ok ? g_ev_join : NULL;
    return ok;
}

/* The Q3GU/Q2D shared expert of n_tok rows: one expert, every token selects
 * it with weight 1.0, the shared clamp (the Q8_K routed pipeline).  With
 * joined (decode batches of several tokens, option shared_stream) it runs
 * on the side stream with scratch of its own (layer buffer 9: its decode
 * scratch, the counters after it), forked after the rows are ready, beside
 * the routed launches; *joined then names the event the launch that adds
 * the rows must wait for (8 tokens: 147 -> 129 us per layer; one token
 * measured 56 -> 59 us, so a single token stays in order). */
static int layer_shared_q3q2(float *out, const sf37_hip_moe_layer_weights *w, const float *x, uint32_t n_tok,
                             hipEvent_t *joined) {
    const uint32_t D = w->in_dim, F = w->mid_dim;
    char *sw = (char *)layer_buf(6, align256((uint64_t)n_tok * 4u) + (uint64_t)n_tok * 4u);
    if (!sw) return 0;
    int32_t *sel = (int32_t *)sw;
    float *wts = (float *)(sw + align256((uint64_t)n_tok * 4u));
    routed_args a = {(const uint8_t *)w->sh_gate->ptr, (const uint8_t *)w->sh_up->ptr,
                     (const uint8_t *)w->sh_down->ptr, sel, wts, 1u, 1u, D, F, D, w->clamp_shared, x, n_tok, NULL, NULL,
                     NULL};
    const int dec = decode_eligible(&a, 0);
    dec_extra ex;
    memset(&ex, 0, sizeof(ex));
    if (joined) *joined = NULL;
    if (dec && joined && g_opt_shared_stream && n_tok > 1u) {
        /* the fills go to the library stream, before the fork */
        return hip_ok(hipMemsetAsync(sel, 0, (uint64_t)n_tok * 4u, g_stream), "shared selection fill") &&
               hip_ok(hipMemsetD32Async((hipDeviceptr_t)wts, 0x3f800000, n_tok, g_stream), "shared weight fill") &&
               decode_run_side(&a, &ex, out, joined);
    }
    if (!hip_ok(hipMemsetAsync(sel, 0, (uint64_t)n_tok * 4u, g_stream), "shared selection fill") ||
        !hip_ok(hipMemsetD32Async((hipDeviceptr_t)wts, 0x3f800000, n_tok, g_stream), "shared weight fill"))
        return 0;
    if (dec) return decode_run(&a, &ex, out, NULL, NULL, NULL, NULL);
    return routed_q8k(&a, out, NULL, NULL, NULL, NULL, 0);
}

/* The fused decode launches' inputs for a whole layer: top-k from the
 * logits (computed by the route launch with f32_router, else given), the
 * Q8_0 shared expert (or, with sh_out, a Q3GU/Q2D shared expert's rows
 * computed before), the block's norm and residual with bn. */
static void layer_fused_extra(dec_extra *ex, const sf37_hip_moe_layer_weights *w, const float *logits,
                              sf37_hip_tensor *selected, sf37_hip_tensor *weights, const block_norm *bn,
                              int f32_router, float *sh_out) {
    memset(ex, 0, sizeof(*ex));
    ex->flags = SF37_DEC_SELECT | (sh_out ? SF37_DEC_SHBASE : SF37_DEC_SHARED) | (f32_router ? SF37_DEC_ROUTER : 0u);
    if (bn) {
        ex->flags |= SF37_DEC_NORM | SF37_DEC_RESID;
        ex->norm_w = bn->norm_w;
        ex->eps = bn->eps;
        ex->xn = bn->xn;
    }
    ex->router_w = f32_router ? (const float *)w->router->ptr : NULL;
    ex->router_bias = (const float *)w->router_bias->ptr;
    ex->logits_sel = logits;
    ex->sh_gate = (const uint8_t *)w->sh_gate->ptr;
    ex->sh_up = (const uint8_t *)w->sh_up->ptr;
    ex->sh_down = (const uint8_t *)w->sh_down->ptr;
    ex->sh_out = sh_out;
    ex->scale = w->scale;
    ex->clamp_shared = w->clamp_shared;
    ex->sel = selected ? (int32_t *)selected->ptr : NULL;
    ex->wts = weights ? (float *)weights->ptr : NULL;
}

/* The decode launches of a layer whose shared expert is in the routed
 * formats (Q3GU gate/up, Q2D down) with that expert as one more slot of
 * every token (SH9): the top-k fills slots 0..K-1 of K + 1 per token, slot K
 * is the shared expert (id E, weight 1, the shared clamp), so it is one more
 * group of n_tok pairs in the same up, mid and down launches, and the
 * combine's slot-order sum adds its row last - (slots 0..K-1) + shared,
 * the same single addition as shared + (slots 0..K-1).  The K + 1 slots
 * live in a layer buffer; the caller's selections and weights receive
 * slots 0..K-1. */
static int layer_fused_sh9(const routed_args *a9, const sf37_hip_moe_layer_weights *w, const float *logits,
                           sf37_hip_tensor *selected, sf37_hip_tensor *weights, const block_norm *bn, int f32_router,
                           float *out) {
    const uint32_t T = a9->n_tok, S = a9->topk, K = S - 1u;
    const uint64_t slots = (uint64_t)T * S * 4u;
    char *buf = (char *)layer_buf(10, 2u * align256(slots));
    if (!buf) return 0;
    int32_t *sel9 = (int32_t *)buf;
    float *wts9 = (float *)(buf + align256(slots));
    dec_extra ex;
    layer_fused_extra(&ex, w, logits, NULL, NULL, bn, f32_router, NULL);
    ex.flags = (ex.flags & ~SF37_DEC_SHARED) | SF37_DEC_SH9;
    ex.sel = sel9;
    ex.wts = wts9;
    if (!decode_run(a9, &ex, out, NULL, NULL, NULL, NULL)) return 0;
    return (!selected || hip_ok(hipMemcpy2DAsync(selected->ptr, (size_t)K * 4u, sel9, (size_t)S * 4u, (size_t)K * 4u, T,
                                                 hipMemcpyDeviceToDevice, g_stream),
                                "selection copy")) &&
           (!weights || hip_ok(hipMemcpy2DAsync(weights->ptr, (size_t)K * 4u, wts9, (size_t)S * 4u, (size_t)K * 4u, T,
                                                hipMemcpyDeviceToDevice, g_stream),
                               "routing weight copy"));
}

/* With bn, out is the hidden state (and x the same tensor): out += layer(
 * RMSNorm(out)).  The fused decode launches take the norm and residual
 * themselves; otherwise rms_norm into a block buffer and the layer into
 * another, whose last add then writes resid = resid + (shared + routed)
 * (resid given: out keeps the shared expert's rows only). */
static int moe_layer_impl(sf37_hip_tensor *out, sf37_hip_tensor *selected, sf37_hip_tensor *weights,
                          const sf37_hip_moe_layer_weights *w, const sf37_hip_tensor *logits_in,
                          const sf37_hip_tensor *x, uint32_t n_tok, const block_norm *bn, float *resid) {
    if (!out || !w || !x || n_tok == 0 || !ensure_init()) return 0;
    const uint32_t E = w->n_expert, K = w->topk, D = w->in_dim, F = w->mid_dim;
    if (!w->router_bias || !w->gate || !w->up || !w->down || !w->sh_gate || !w->sh_up || !w->sh_down || E == 0 ||
        K == 0 || K > 16u || D % QK != 0 || F % QK != 0 || (!logits_in && !w->router))
        return 0;
    if (out->bytes < (uint64_t)n_tok * D * 4u || x->bytes < (uint64_t)n_tok * D * 4u ||
        (logits_in && logits_in->bytes < (uint64_t)n_tok * E * 4u) ||
        (selected && selected->bytes < (uint64_t)n_tok * K * 4u) ||
        (weights && weights->bytes < (uint64_t)n_tok * K * 4u))
        return 0;
    const int run_router = !logits_in || (g_opt_router_always && w->router);
    /* weight tensors hold the shapes they are read at (the kernels do not
     * bound their reads by the tensors' sizes) */
    if (!layer_weights_ok(w, run_router)) return 0;
    const int router_f32 = w->router_type == SF37_HIP_TYPE_F32;
    const int shared_q3 = w->shared_type == SF37_HIP_TYPE_Q3GU;
    if (shared_q3 && (!q8k_use_for(F) || !q8k_use_for(D))) {
        fprintf(stderr, "sf37: HIP moe layer: the Q3GU/Q2D shared expert takes the Q8_K path (rows >= q8k_min_rows)\n");
        return 0;
    }
    const sf37_stream_t st = (sf37_stream_t)g_stream;
    routed_args a = {(const uint8_t *)w->gate->ptr, (const uint8_t *)w->up->ptr, (const uint8_t *)w->down->ptr, NULL,
                     NULL, E, K, D, F, D, w->clamp_routed, (const float *)x->ptr, n_tok, NULL, NULL, NULL};
    const int fused = decode_eligible(&a, SF37_DEC_SELECT | (shared_q3 ? 0u : SF37_DEC_SHARED));
    /* a Q3GU/Q2D shared expert as one more slot inside the routed decode
     * launches (its pairs grouped two at a time, so its up and down items
     * weigh what a routed expert's do: as one group of n_tok pairs the 8-token
     * layer measured 163 against 125 us with its own launches) */
    routed_args a9 = a;
    a9.topk = K + 1u;
    /* (pairs <= experts: then the launch plan's group count, the pair
     * count, is the same with the shared expert's groups) */
    const int sh9 = shared_q3 && g_opt_shared_slot && fused && K + 1u <= 16u &&
                    (uint64_t)n_tok * (K + 1u) <= E && decode_eligible(&a9, SF37_DEC_SELECT);
    if (bn && !fused) {
        const uint64_t bytes = (uint64_t)n_tok * D * 4u;
        for (int i = 0; i < 2; i++) {
            if (!g_block_buf[i] || g_block_buf_bytes[i] < bytes) {
                if (g_block_buf[i]) sf37_hip_tensor_free(g_block_buf[i]);
                g_block_buf[i] = sf37_hip_tensor_alloc(bytes);
                g_block_buf_bytes[i] = bytes;
                if (!g_block_buf[i]) return 0;
            }
        }
        float *xn = bn->xn ? bn->xn : (float *)g_block_buf[0]->ptr;
        sf37_hip_tensor xnt = {xn, bytes, 0}, *y = g_block_buf[1];
        return LAUNCH(SF37_HIP_STAGE_OTHER, sf37k_rms_norm(xn, (const float *)x->ptr, bn->norm_w, 1, D, n_tok, bn->eps, st),
                      "moe block rms_norm launch") &&
               moe_layer_impl(y, selected, weights, w, logits_in, &xnt, n_tok, NULL, (float *)out->ptr);
    }
    /* the rows the router and shared expert read: x, or with a block's norm
     * on the fused path (whose launches normalise x themselves), the rows
     * normalised here for the steps that run before those launches */
    const float *xl = (const float *)x->ptr;
    if (bn && ((run_router && !router_f32) || (shared_q3 && !sh9))) {
        float *xn = bn->xn ? bn->xn : (float *)layer_buf(5, (uint64_t)n_tok * D * 4u);
        if (!xn || !LAUNCH(SF37_HIP_STAGE_OTHER, sf37k_rms_norm(xn, (const float *)x->ptr, bn->norm_w, 1, D, n_tok,
                                                                bn->eps, st),
                           "moe block rms_norm launch"))
            return 0;
        xl = xn;
    }
    /* the Q8_0 shared expert of a prefill batch on the side stream, from
     * here to the routed combine: it depends on the rows alone, so it runs
     * beside the router, top-k, dispatch and routed experts */
    const int side = !fused && !shared_q3 && g_opt_shared_stream && shared_mfma_eligible(n_tok, D, F);
    if (side) {
        float *sh = (float *)layer_buf(3, (uint64_t)n_tok * F * 4u);
        if (!sh || !side_stream_ready() || !hip_ok(hipEventRecord(g_ev_fork, g_stream), "shared expert fork") ||
            !hip_ok(hipStreamWaitEvent(g_side, g_ev_fork, 0), "shared expert fork wait") ||
            !shared_mfma((float *)out->ptr, sh, (const uint8_t *)w->sh_gate->ptr, (const uint8_t *)w->sh_up->ptr,
                         (const uint8_t *)w->sh_down->ptr, D, F, xl, n_tok, w->clamp_shared, g_side) ||
            !hip_ok(hipEventRecord(g_ev_join, g_side), "shared expert join record"))
            return 0;
    }
    /* logits: injected, or a BF16 / Q8_0 router computed here; the F32
     * router runs in the decode route launch or below */
    float *lg_buf = (float *)layer_buf(0, (uint64_t)n_tok * E * 4u);
    if (!lg_buf) return 0;
    const float *logits = logits_in ? (const float *)logits_in->ptr : NULL;
    if (run_router && !router_f32) {
        if (!layer_router_typed(lg_buf, w, xl, n_tok)) return 0;
        if (!logits) logits = lg_buf;
    }
    if (sh9) return layer_fused_sh9(&a9, w, logits, selected, weights, bn, run_router && router_f32, (float *)out->ptr);
    if (fused) {
        /* a Q3GU/Q2D shared expert first, then the routed launches add it */
        float *sh_out = NULL;
        hipEvent_t join = NULL;
        if (shared_q3) {
            sh_out = (float *)layer_buf(4, (uint64_t)n_tok * D * 4u);
            if (!sh_out || !layer_shared_q3q2(sh_out, w, xl, n_tok, &join)) return 0;
        }
        dec_extra ex;
        layer_fused_extra(&ex, w, logits, selected, weights, bn, run_router && router_f32, sh_out);
        ex.comb_wait = join;
        return decode_run(&a, &ex, (float *)out->ptr, NULL, NULL, NULL, NULL);
    }
    /* layer-owned buffers (separate from the routed scratch): selection,
     * routing weights, the Q8_0 shared expert's gate | up | mid */
    int32_t *sel = selected ? (int32_t *)selected->ptr : (int32_t *)layer_buf(1, (uint64_t)n_tok * K * 4u);
    float *wts = weights ? (float *)weights->ptr : (float *)layer_buf(2, (uint64_t)n_tok * K * 4u);
    if (!sel || !wts) return 0;
    /* logits computed here feed only the top-8: a K-split router leaves its
     * slices for the top-8 launch to add (no launch of its own) */
    uint32_t slices = 1;
    double *rpart = NULL;
    if (run_router && router_f32 &&
        !LAUNCH(SF37_HIP_STAGE_ROUTER, router_matmul_part(lg_buf, (const float *)w->router->ptr, xl, D, E, n_tok,
                                                          logits ? NULL : &slices, &rpart, st),
                "moe_layer router launch"))
        return 0;
    if (!logits) logits = lg_buf;
    if (E > ROUTER_MAX_EXPERTS ||
        !LAUNCH(SF37_HIP_STAGE_SELECT, sf37k_router_select_part(sel, wts, NULL, logits, rpart, slices,
                                       (const float *)w->router_bias->ptr, E, K, w->scale, n_tok, st),
                   "moe_layer router_select launch"))
        return 0;
    /* shared expert into out: Q3GU/Q2D on the Q8_K path, or Q8_0 gate/up
     * pair -> SwiGLU -> Q8_0 down */
    if (shared_q3) {
        if (!layer_shared_q3q2((float *)out->ptr, w, xl, n_tok, NULL)) return 0;
    } else if (side) {
        a.comb_wait = g_ev_join;   /* launched above; the routed combine joins it */
    } else if (shared_mfma_eligible(n_tok, D, F)) {
        float *sh = (float *)layer_buf(3, (uint64_t)n_tok * F * 4u);
        if (!sh || !shared_mfma((float *)out->ptr, sh, (const uint8_t *)w->sh_gate->ptr, (const uint8_t *)w->sh_up->ptr,
                                (const uint8_t *)w->sh_down->ptr, D, F, xl, n_tok, w->clamp_shared, g_stream))
            return 0;
    } else {
        float *sh = (float *)layer_buf(3, (uint64_t)n_tok * F * 4u * 3u);   /* gate | up | mid */
        if (!sh ||
            !q8_0_run(sh, sh + (uint64_t)n_tok * F, (const uint8_t *)w->sh_gate->ptr, (const uint8_t *)w->sh_up->ptr, D,
                      F, xl, n_tok) ||
            !LAUNCH(SF37_HIP_STAGE_SWIGLU, sf37k_swiglu(sh + 2u * (uint64_t)n_tok * F, sh, sh + (uint64_t)n_tok * F,
                                                        (uint64_t)n_tok * F, w->clamp_shared, st),
                    "moe_layer shared swiglu launch") ||
            !q8_0_run((float *)out->ptr, NULL, (const uint8_t *)w->sh_down->ptr, NULL, F, D,
                      sh + 2u * (uint64_t)n_tok * F, n_tok))
            return 0;
    }
    a.selected = sel;
    a.weights = wts;
    const int slots = n_tok == 1u;
    if (!slots && E > DISPATCH_MAX_EXPERTS) return 0;
    /* the fp32-activation path (one token, small shapes) */
    float *routed = NULL;
    if (!q8k_use_for(F) || !q8k_use_for(D)) {
        if (n_tok != 1u) return 0;
        if (side && !hip_ok(hipStreamWaitEvent(g_stream, g_ev_join, 0), "shared expert join")) return 0;
        routed = (float *)layer_buf(4, (uint64_t)D * 4u);
        float *mid_down = (float *)layer_buf(5, (uint64_t)K * ((uint64_t)F + D) * 4u);
        if (!routed || !mid_down || !routed_f32(&a, routed, mid_down, mid_down + (uint64_t)K * F, NULL, NULL))
            return 0;
    } else {
        /* the routed combine adds the shared rows (and the residual) itself */
        a.comb_base = (const float *)out->ptr;
        a.comb_resid = resid;
        return routed_q8k(&a, (float *)out->ptr, NULL, NULL, NULL, NULL, slots);
    }
    if (resid)
        return LAUNCH(SF37_HIP_STAGE_ADD, sf37k_add2_inplace(resid, (const float *)out->ptr, routed, (uint64_t)n_tok * D, st),
                      "moe block residual launch");
    return LAUNCH(SF37_HIP_STAGE_ADD, sf37k_add_inplace((float *)out->ptr, routed, (uint64_t)n_tok * D, st), "moe_layer add launch");
}

/* sf37_hip_moe_layer for decode batches without any allocation: the fused
 * decode launches with their scratch (activation blocks, group tables,
 * per-pair rows, queues) in the library's static device array.  Calls that
 * overlap on one GPU share that array and race. */
int sf37_hip_moe_layer_noalloc(sf37_hip_tensor *out, sf37_hip_tensor *selected, sf37_hip_tensor *weights,
                               const sf37_hip_moe_layer_weights *w, const sf37_hip_tensor *logits_in,
                               const sf37_hip_tensor *x, uint32_t n_tok) {
    if (!out || !w || !x || n_tok == 0 || !ensure_init()) return 0;
    const uint32_t E = w->n_expert, K = w->topk, D = w->in_dim, F = w->mid_dim;
    if (!w->router_bias || !w->gate || !w->up || !w->down || !w->sh_gate || !w->sh_up || !w->sh_down || E == 0 ||
        K == 0 || K > 16u || D % QK != 0 || F % QK != 0 || (!logits_in && !w->router))
        return 0;
    if (out->bytes < (uint64_t)n_tok * D * 4u || x->bytes < (uint64_t)n_tok * D * 4u ||
        (logits_in && logits_in->bytes < (uint64_t)n_tok * E * 4u) ||
        (selected && selected->bytes < (uint64_t)n_tok * K * 4u) ||
        (weights && weights->bytes < (uint64_t)n_tok * K * 4u))
        return 0;
    const int run_router = !logits_in || (g_opt_router_always && w->router);
    if (!layer_weights_ok(w, run_router)) return 0;
    routed_args a = {(const uint8_t *)w->gate->ptr, (const uint8_t *)w->up->ptr, (const uint8_t *)w->down->ptr, NULL,
                     NULL, E, K, D, F, D, w->clamp_routed, (const float *)x->ptr, n_tok, NULL, NULL, NULL};
    if ((run_router && w->router_type != SF37_HIP_TYPE_F32) || w->shared_type == SF37_HIP_TYPE_Q3GU ||
        !decode_eligible(&a, SF37_DEC_SELECT | SF37_DEC_SHARED)) {
        fprintf(stderr, "sf37: HIP moe_layer_noalloc takes decode batches of 1..%u tokens on the Q8_K path with an "
                        "F32 router (or injected logits) and a Q8_0 shared expert\n", SF37_DEC_MAX_TOK);
        return 0;
    }
    /* the array's address on the current device, looked up on the first
     * call there (sf37_hip_init looks it up for device 0) */
    char *base = (char *)sf37k_noalloc_scratch();
    if (!base && hip_ok((hipError_t)sf37k_noalloc_scratch_init(), "no-alloc scratch address"))
        base = (char *)sf37k_noalloc_scratch();
    if (!base) {
        fprintf(stderr, "sf37: HIP moe_layer_noalloc: the static scratch of this device has no address\n");
        return 0;
    }
    dec_extra ex;
    layer_fused_extra(&ex, w, logits_in ? (const float *)logits_in->ptr : NULL, selected, weights, NULL, run_router,
                      NULL);
    return decode_run_in(&a, &ex, (float *)out->ptr, NULL, NULL, NULL, NULL, base + SF37_NOALLOC_QUEUE_BYTES,
                         SF37_NOALLOC_SCRATCH_BYTES - SF37_NOALLOC_QUEUE_BYTES, (uint32_t *)base, NULL);
}

int sf37_hip_moe_block(sf37_hip_tensor *hidden, sf37_hip_tensor *normed, sf37_hip_tensor *selected,
                       sf37_hip_tensor *weights, const sf37_hip_moe_layer_weights *w, const void *model_map,
                       uint64_t model_size, uint64_t norm_offset, float eps, const sf37_hip_tensor *logits_in,
                       uint32_t n_tok) {
    if (!hidden || !w || !model_map || n_tok == 0 || !ensure_init()) return 0;
    const uint64_t bytes = (uint64_t)n_tok * w->in_dim * 4u;
    if (hidden->bytes < bytes || (normed && normed->bytes < bytes) ||
        !mapped_range_ok(model_size, norm_offset, (uint64_t)w->in_dim * 2u))
        return 0;
    const void *nw = model_ptr(model_map, norm_offset, (uint64_t)w->in_dim * 2u, "ffn norm weight");
    if (!nw) return 0;
    const block_norm bn = {(const uint16_t *)nw, eps, normed ? (float *)normed->ptr : NULL};
    return moe_layer_impl(hidden, selected, weights, w, logits_in, hidden, n_tok, &bn, NULL);
}

int sf37_hip_moe_stack(sf37_hip_tensor *hidden, uint32_t n_layers, const sf37_hip_moe_layer_weights *layers,
                       const void *model_map, uint64_t model_size, const uint64_t *norm_offsets, float eps,
                       const sf37_hip_tensor *const *logits, sf37_hip_tensor *const *selected, uint32_t n_tok) {
    if (!hidden || !layers || !norm_offsets || n_layers == 0) return 0;
    for (uint32_t l = 0; l < n_layers; l++) {
        if (!sf37_hip_moe_block(hidden, NULL, selected ? selected[l] : NULL, NULL, &layers[l], model_map, model_size,
                                norm_offsets[l], eps, logits ? logits[l] : NULL, n_tok)) {
            fprintf(stderr, "sf37_hip: moe stack layer %u failed\n", l);
            return 0;
        }
    }
    return 1;
}

int sf37_hip_synth_normal(sf37_hip_tensor *dst, uint64_t n, uint64_t seed, uint64_t stream, uint64_t index0,
                          float sigma) {
    if (!dst || dst->bytes < n * 4u || !ensure_init()) return 0;
    return LAUNCH(SF37_HIP_STAGE_OTHER, sf37k_synth_normal((float *)dst->ptr, n, seed, stream, index0, sigma, (sf37_stream_t)g_stream),
                     "synth normal launch");
}

int sf37_hip_synth_quant_rows(int type, sf37_hip_tensor *dst, uint64_t row0, uint64_t nrows, uint64_t ncols,
                              uint64_t seed, uint64_t stream, float sigma) {
    if (!dst || !ensure_init() || (type != 0 && type != 2 && type != 3)) return 0;
    const uint64_t qk = type == 0 ? 32u : QK;
    const uint64_t bs = type == 0 ? Q8B : (type == 3 ? Q3B : Q2B);
    if (ncols % qk != 0 || dst->bytes < nrows * (ncols / qk) * bs) return 0;
    return LAUNCH(SF37_HIP_STAGE_OTHER, sf37k_synth_quant_rows(type, (uint8_t *)dst->ptr, row0, nrows, ncols, seed, stream, sigma,
                                            (sf37_stream_t)g_stream),
                     "synth quant launch");
}

int sf37_hip_sigmoid_array(sf37_hip_tensor *out, const sf37_hip_tensor *x, uint64_t n, int mode) {
    if (!out || !x || out->bytes < n * 4u || x->bytes < n * 4u || !ensure_init()) return 0;
    return LAUNCH(SF37_HIP_STAGE_OTHER, sf37k_sigmoid_array((float *)out->ptr, (const float *)x->ptr, n, mode, (sf37_stream_t)g_stream),
                     "sigmoid array launch");
}
