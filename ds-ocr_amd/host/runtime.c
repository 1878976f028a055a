/* runtime.c — device/stream bring-up, error reporting, staging buffers and the host->device weight
 * registry of libds_ocr_hip. The registry plays the role of the Metal backend's
 * ds_metal_register_expert_block (reference ds_metal.m:244-258): weights are uploaded once and
 * stay resident. */
#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "dsr.h"
#include "ds_hip.h"
#include "ds_kernels.h"

/* Mode globals; the reference defines them in ds_ocr.c:26-27, which wins when linked. */
__attribute__((weak)) int ds_verbose = 0;
__attribute__((weak)) int ds_bf16_simulate_python = 0;

hipStream_t dsr_stream = NULL;
static int g_init = 0; /* 0 = not tried, 1 = ok, -1 = failed */
static char g_err[512] = "";
static int g_threads = 1;

int dsr_failf(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  fprintf(stderr, "ds_ocr_hip: %s\n", g_err);
  return -1;
}

int dsr_fail(const char *what, hipError_t e) { return dsr_failf("%s: %s", what, hipGetErrorString(e)); }

const char *ds_hip_last_error(void) { return g_err; }

/* The device error words (DSR_DERR_*): one 64-byte line each of mapped, coherent pinned memory. */
static int *g_derr_host = NULL, *g_derr_dev = NULL;
#define DERR_STRIDE 16

int *dsr_derr_dev(int kind) {
  return g_derr_dev && kind >= 0 && kind < DSR_DERR_N ? g_derr_dev + DERR_STRIDE * kind : NULL;
}

/* Counters of the certified CFG routing ([0] routings, [1] recomputed in ds_linear's order, [2]
 * one-kernel layers whose output was corrected to the certified selection) and the routing log
 * (ds_hip_set_route_log). */
static unsigned long long *g_rstat = NULL;
static int *g_rlog = NULL, g_rlog_cap = 0;

dsh_rcert_t dsr_rcert(int tag) {
  dsh_rcert_t r;
  r.stats = g_rstat;
  r.log = g_rlog;
  r.log_cap = g_rlog_cap;
  r.tag = tag;
  return r;
}

int ds_hip_route_stats(unsigned long long *counts, int reset) {
  if (dsr_init()) return -1;
  if (!counts) return dsr_failf("ds_hip_route_stats: NULL argument");
  DSR_TRY(hipStreamSynchronize(dsr_stream), "synchronize");
  DSR_TRY(hipMemcpy(counts, g_rstat, 3 * sizeof(unsigned long long), hipMemcpyDeviceToHost), "route counters");
  if (reset) DSR_TRY(hipMemset(g_rstat, 0, 3 * sizeof(unsigned long long)), "route counters");
  return 0;
}

int ds_hip_set_route_log(int *log_dev, int capacity) {
  if (dsr_init()) return -1;
  if ((log_dev == NULL) != (capacity == 0) || capacity < 0)
    return dsr_failf("ds_hip_set_route_log: a buffer needs a capacity (NULL and 0 switch the log off)");
  g_rlog = log_dev;
  g_rlog_cap = capacity;
  return 0;
}

int dsr_derr_check(void) {
  static const char *what[DSR_DERR_N] = {
      "prefill: a down tile's bounded wait for its gate_up tiles gave up; that call's output is not valid",
      "decode: a certified layer's bounded wait for its verdict on the expert selection gave up; the "
      "step's output is not valid",
  };
  if (!g_derr_host) return 0;
  int rc = 0;
  for (int k = 0; k < DSR_DERR_N; k++) {
    if (__atomic_load_n(g_derr_host + DERR_STRIDE * k, __ATOMIC_ACQUIRE)) {
      __atomic_store_n(g_derr_host + DERR_STRIDE * k, 0, __ATOMIC_RELEASE);
      rc = dsr_failf("%s", what[k]);
    }
  }
  return rc;
}

int dsr_init(void) {
  if (g_init == 1) return 0;
  if (g_init == -1) return dsr_failf("HIP device unavailable (initialisation failed earlier)");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n < 1) {
    g_init = -1;
    return dsr_failf("no HIP device: %s", e != hipSuccess ? hipGetErrorString(e) : "device count is 0");
  }
  e = hipSetDevice(0);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&dsr_stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    g_init = -1;
    return dsr_fail("HIP init", e);
  }
  /* the device error words: host memory the kernels write directly */
  if (e == hipSuccess)
    e = hipHostMalloc((void **)&g_derr_host, (size_t)DSR_DERR_N * DERR_STRIDE * sizeof(int),
                      hipHostMallocMapped | hipHostMallocCoherent);
  if (e == hipSuccess) {
    memset(g_derr_host, 0, (size_t)DSR_DERR_N * DERR_STRIDE * sizeof(int));
    e = hipHostGetDevicePointer((void **)&g_derr_dev, g_derr_host, 0);
  }
  if (e != hipSuccess) {
    g_init = -1;
    return dsr_fail("HIP init (device error words)", e);
  }
  if (hipMalloc((void **)&g_rstat, 256) != hipSuccess || hipMemset(g_rstat, 0, 256) != hipSuccess) {
    g_init = -1;
    return dsr_failf("HIP init: routing counters");
  }
  /* the device address of the allocation-free entry points' scratch array (device 0 is current) */
  if (dsh_static_scratch_init()) {
    g_init = -1;
    return dsr_failf("HIP init: the device address of the static scratch array is not available");
  }
  g_init = 1;
  return 0;
}

int dsr_ready(void) { return g_init == 1; }

int ds_hip_init(void) { return dsr_init(); }

/* ---------------------------------------------------------------- staging */

static void *g_slot[DSR_NSLOTS];
static size_t g_slot_cap[DSR_NSLOTS];

void *dsr_scratch(int slot, size_t bytes) {
  if (bytes == 0) bytes = 16;
  if (bytes <= g_slot_cap[slot]) return g_slot[slot];
  if (g_slot[slot]) {
    hipStreamSynchronize(dsr_stream);
    hipFree(g_slot[slot]);
    g_slot[slot] = NULL;
    g_slot_cap[slot] = 0;
  }
  size_t cap = bytes < 65536 ? 65536 : bytes + bytes / 4;
  void *p = NULL;
  hipError_t e = hipMalloc(&p, cap);
  if (e != hipSuccess) {
    dsr_fail("staging allocation", e);
    return NULL;
  }
  g_slot[slot] = p;
  g_slot_cap[slot] = cap;
  return p;
}

int dsr_h2d(void *dst, const void *src, size_t n) {
  if (n == 0) return 0;
  DSR_TRY(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, dsr_stream), "copy to device");
  return 0;
}

int dsr_d2h(void *dst, const void *src, size_t n) {
  if (n) DSR_TRY(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, dsr_stream), "copy to host");
  DSR_TRY(hipStreamSynchronize(dsr_stream), "stream synchronize");
  return 0;
}

/* ---------------------------------------------------------------- registry */

static uint64_t fnv(uint64_t h, const void *p, size_t n) {
  const unsigned char *b = (const unsigned char *)p;
  for (size_t i = 0; i < n; i++) h = (h ^ b[i]) * 1099511628211ull;
  return h;
}

/* Weights are registered once: a host array is keyed by its address and size, like the reference's
 * read-only mmap'd weights and INT8 blocks that are never rewritten (ds_ocr.c:611-622; the Metal
 * backend registers expert blocks the same way, ds_metal.m:244-258). To notice a new array placed at
 * a freed one's address, each key also keeps a sampled fingerprint: 16 windows of 256 bytes spread
 * evenly over the array (the whole array when it is at most 4 KiB), about 4 KiB read per call
 * whatever the size. A caller that edits registered weights in place calls ds_hip_weights_changed. */
#define FP_WINDOWS 16
#define FP_WINDOW 256

static uint64_t fingerprint(const void *p, size_t n) {
  const unsigned char *b = (const unsigned char *)p;
  uint64_t h = fnv(1469598103934665603ull, &n, sizeof n);
  if (n <= (size_t)FP_WINDOWS * FP_WINDOW) return fnv(h, b, n);
  const size_t step = (n - FP_WINDOW) / (FP_WINDOWS - 1);
  for (int i = 0; i < FP_WINDOWS; i++) h = fnv(h, b + (size_t)i * step, FP_WINDOW);
  return h;
}

typedef struct {
  const void *key;
  uint64_t fp;
  size_t bytes;
  void *dev; /* weights: the copy; blocks: q (scale, offset follow in sdev/odev) */
  void *aux; /* weights: device data derived from them (dsr_weight_set_aux), freed with the entry */
  float *sdev, *odev;
  int out_dim, in_dim;
  int is_block;
} entry_t;

static entry_t *g_ent = NULL;
static int g_nent = 0, g_cap = 0;

static entry_t *find(const void *key, int is_block) {
  for (int i = 0; i < g_nent; i++)
    if (g_ent[i].key == key && g_ent[i].is_block == is_block) return &g_ent[i];
  return NULL;
}

static void drop(entry_t *e) {
  hipStreamSynchronize(dsr_stream);
  if (e->dev) hipFree(e->dev);
  if (e->aux) hipFree(e->aux);
  *e = g_ent[--g_nent];
}

static entry_t *add(void) {
  if (g_nent == g_cap) {
    int nc = g_cap ? 2 * g_cap : 64;
    entry_t *ne = (entry_t *)realloc(g_ent, (size_t)nc * sizeof(entry_t));
    if (!ne) return NULL;
    g_ent = ne;
    g_cap = nc;
  }
  entry_t *e = &g_ent[g_nent++];
  memset(e, 0, sizeof *e);
  return e;
}

static uint64_t block_fp(const ds_int4_block_t *b) {
  size_t nq = (size_t)b->out_dim * b->in_dim;
  uint64_t h = fingerprint(b->qweight, nq);
  h = fnv(h, &(uint64_t){fingerprint(b->scale, (size_t)b->out_dim * 4)}, 8);
  h = fnv(h, &(uint64_t){fingerprint(b->offset, (size_t)b->out_dim * 4)}, 8);
  h = fnv(h, &b->out_dim, sizeof(int));
  return fnv(h, &b->in_dim, sizeof(int));
}

/* One allocation per block: codes, then scales, then offsets (each 256-byte aligned). */
static size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }

static int block_alloc(entry_t *e, int out_dim, int in_dim) {
  size_t nq = al256((size_t)out_dim * in_dim), ns = al256((size_t)out_dim * 4);
  void *p = NULL;
  DSR_TRY(hipMalloc(&p, nq + 2 * ns), "block allocation");
  e->dev = p;
  e->sdev = (float *)((char *)p + nq);
  e->odev = (float *)((char *)p + nq + ns);
  e->out_dim = out_dim;
  e->in_dim = in_dim;
  e->is_block = 1;
  return 0;
}

int dsr_block_device(const ds_int4_block_t *b, dsr_dblock_t *out) {
  if (dsr_init()) return -1;
  uint64_t fp = block_fp(b);
  entry_t *e = find(b->qweight, 1);
  if (e && (e->fp != fp || e->out_dim != b->out_dim || e->in_dim != b->in_dim)) {
    drop(e);
    e = NULL;
  }
  if (!e) {
    e = add();
    if (!e) return dsr_failf("registry allocation failed");
    if (block_alloc(e, b->out_dim, b->in_dim)) {
      g_nent--;
      return -1;
    }
    e->key = b->qweight;
    e->fp = fp;
    if (dsr_h2d(e->dev, b->qweight, (size_t)b->out_dim * b->in_dim) ||
        dsr_h2d(e->sdev, b->scale, (size_t)b->out_dim * 4) || dsr_h2d(e->odev, b->offset, (size_t)b->out_dim * 4)) {
      drop(e);
      return -1;
    }
  }
  out->q = (int8_t *)e->dev;
  out->scale = e->sdev;
  out->offset = e->odev;
  out->out_dim = e->out_dim;
  out->in_dim = e->in_dim;
  return 0;
}

/* Allocates the device arrays of a block about to be produced on the device. */
int dsr_block_new(const ds_int4_block_t *b, dsr_dblock_t *out) {
  if (dsr_init()) return -1;
  entry_t *e = find(b->qweight, 1);
  if (e) drop(e);
  e = add();
  if (!e) return dsr_failf("registry allocation failed");
  if (block_alloc(e, b->out_dim, b->in_dim)) {
    g_nent--;
    return -1;
  }
  e->key = b->qweight;
  out->q = (int8_t *)e->dev;
  out->scale = e->sdev;
  out->offset = e->odev;
  out->out_dim = b->out_dim;
  out->in_dim = b->in_dim;
  return 0;
}

/* Seals a block produced by dsr_block_new once its host arrays hold the same values. */
int dsr_block_adopt(const ds_int4_block_t *b, int8_t *q, float *scale, float *offset) {
  (void)q;
  (void)scale;
  (void)offset;
  entry_t *e = find(b->qweight, 1);
  if (!e) return dsr_failf("internal: block not registered");
  e->fp = block_fp(b);
  return 0;
}

void dsr_block_forget(const void *qweight) {
  if (!qweight) return;
  entry_t *e = find(qweight, 1);
  if (e) drop(e);
}

int ds_hip_register_block(const ds_int4_block_t *block) {
  if (!block || !block->qweight || !block->scale || !block->offset || block->out_dim <= 0 || block->in_dim <= 0)
    return dsr_failf("ds_hip_register_block: invalid block");
  dsr_dblock_t db;
  return dsr_block_device(block, &db);
}

int ds_hip_register_weights(const void *host, size_t bytes) {
  if (!host || !bytes) return dsr_failf("ds_hip_register_weights: invalid arguments");
  return dsr_weight_device(host, bytes) ? 0 : -1;
}

int ds_hip_weights_changed(const void *host_ptr) {
  if (!host_ptr) return dsr_failf("ds_hip_weights_changed: NULL pointer");
  if (g_init != 1) return 0; /* nothing registered yet */
  int dropped = 0;
  for (int is_block = 0; is_block < 2; is_block++) {
    entry_t *e = find(host_ptr, is_block);
    if (e) {
      drop(e);
      dropped++;
    }
  }
  return dropped;
}

void *dsr_weight_aux(const void *host) {
  entry_t *e = find(host, 0);
  return e ? e->aux : NULL;
}

int dsr_weight_set_aux(const void *host, void *aux_dev) {
  entry_t *e = find(host, 0);
  if (!e) return -1;
  if (e->aux && e->aux != aux_dev) hipFree(e->aux);
  e->aux = aux_dev;
  return 0;
}

const void *dsr_weight_device(const void *host, size_t bytes) {
  if (dsr_init()) return NULL;
  uint64_t fp = fingerprint(host, bytes);
  entry_t *e = find(host, 0);
  if (e && (e->fp != fp || e->bytes != bytes)) {
    drop(e);
    e = NULL;
  }
  if (e) return e->dev;
  e = add();
  if (!e) {
    dsr_failf("registry allocation failed");
    return NULL;
  }
  void *p = NULL;
  hipError_t err = hipMalloc(&p, bytes ? bytes : 16);
  if (err != hipSuccess) {
    g_nent--;
    dsr_fail("weight allocation", err);
    return NULL;
  }
  e->key = host;
  e->fp = fp;
  e->bytes = bytes;
  e->dev = p;
  if (dsr_h2d(p, host, bytes)) {
    drop(e);
    return NULL;
  }
  return p;
}

/* ---------------------------------------------------------------- threads */

/* ds_kernels.c:517-543: clamp to [1, 16]. */
void ds_set_threads(int n) {
  if (n < 1) n = 1;
  if (n > 16) n = 16;
  g_threads = n;
}
int ds_get_threads(void) { return g_threads; }
int dsr_threads(void) { return g_threads; }

int ds_get_num_cpus(void) {
  long n = sysconf(_SC_NPROCESSORS_ONLN);
  return n > 0 ? (int)n : 1;
}

void ds_dispatch_ensure_init(void) { (void)dsr_init(); }

void ds_parallel_for(ds_parallel_fn_t fn, void *arg) {
  if (fn) fn(0, 1, arg);
}

/* ---------------------------------------------------------------- public memory helpers */

void *ds_hip_malloc(size_t bytes) {
  if (dsr_init()) return NULL;
  void *p = NULL;
  hipError_t e = hipMalloc(&p, bytes ? bytes : 16);
  if (e != hipSuccess) {
    dsr_fail("ds_hip_malloc", e);
    return NULL;
  }
  return p;
}

void ds_hip_free(void *p) {
  if (!p || g_init != 1) return;
  hipStreamSynchronize(dsr_stream);
  hipFree(p);
}

int ds_hip_memcpy_h2d(void *dst, const void *src, size_t n) {
  if (dsr_init()) return -1;
  if (dsr_h2d(dst, src, n)) return -1;
  DSR_TRY(hipStreamSynchronize(dsr_stream), "synchronize");
  return 0;
}

int ds_hip_memcpy_d2h(void *dst, const void *src, size_t n) {
  if (dsr_init()) return -1;
  return dsr_d2h(dst, src, n);
}

int ds_hip_memcpy_d2d(void *dst, const void *src, size_t n) {
  if (dsr_init()) return -1;
  if (n) DSR_TRY(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, dsr_stream), "device copy");
  return 0;
}

int ds_hip_time_stream_read(const void *src_dev, size_t bytes, int n, float *ms) {
  if (dsr_init()) return -1;
  if (!src_dev || bytes < 16 || n <= 0 || !ms) return dsr_failf("ds_hip_time_stream_read: invalid arguments");
  unsigned *sink = (unsigned *)dsr_scratch(DSR_SLOT_IDX, 1024 * sizeof(unsigned));
  if (!sink) return -1;
  hipEvent_t a, b;
  DSR_TRY(hipEventCreate(&a), "event");
  DSR_TRY(hipEventCreate(&b), "event");
  hipError_t e = dsh_launch_stream_read(src_dev, bytes & ~(size_t)15, sink, dsr_stream); /* warm-up */
  if (e == hipSuccess) e = hipEventRecord(a, dsr_stream);
  for (int i = 0; i < n && e == hipSuccess; i++) e = dsh_launch_stream_read(src_dev, bytes & ~(size_t)15, sink, dsr_stream);
  if (e == hipSuccess) e = hipEventRecord(b, dsr_stream);
  if (e == hipSuccess) e = hipEventSynchronize(b);
  float t = 0;
  if (e == hipSuccess) e = hipEventElapsedTime(&t, a, b);
  hipEventDestroy(a);
  hipEventDestroy(b);
  if (e != hipSuccess) return dsr_fail("stream read timing", e);
  *ms = t / n;
  return 0;
}

int ds_hip_sync(void) {
  if (dsr_init()) return -1;
  DSR_TRY(hipStreamSynchronize(dsr_stream), "synchronize");
  return dsr_derr_check();
}
