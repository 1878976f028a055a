/* runtime.c — device/stream bring-up, error reporting, staging buffers and the host->device weight
 * registry of libds_ocr_hip. The registry plays the role of the Metal backend's
 * ds_metal_register_expert_block (reference ds_metal.m:244-258): weights are uploaded once and
 * stay resident. */
#define _GNU_SOURCE
#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
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
      "expert: the down rows' bounded wait for the gate_up rows' h gave up; that call's output is not valid",
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

static void *g_hbuf = NULL;
static size_t g_hbuf_n = 0;
static unsigned g_epoch = 0;

void *dsr_expert_hbuf(size_t n) {
  if (n <= g_hbuf_n) return g_hbuf;
  if (g_hbuf) {
    hipStreamSynchronize(dsr_stream);
    hipFree(g_hbuf);
    g_hbuf = NULL;
    g_hbuf_n = 0;
  }
  const size_t cap = n < 4096 ? 4096 : n;
  if (hipMalloc(&g_hbuf, cap * 8) != hipSuccess || hipMemset(g_hbuf, 0, cap * 8) != hipSuccess) {
    dsr_failf("expert h buffer allocation failed");
    if (g_hbuf) hipFree(g_hbuf);
    g_hbuf = NULL;
    return NULL;
  }
  g_hbuf_n = cap;
  return g_hbuf;
}

unsigned dsr_expert_epoch(void) {
  if (++g_epoch == 0) g_epoch = 1;
  return g_epoch;
}

static unsigned char *g_xin = NULL;
static size_t g_xin_n = 0, g_xin_cap = 0;
static int g_xin_valid = 0;

int dsr_input_cached(const void *x, size_t n) {
  if (g_xin_valid && n == g_xin_n && memcmp(g_xin, x, n) == 0) return 1;
  if (n > g_xin_cap) {
    free(g_xin);
    g_xin = (unsigned char *)malloc(n);
    g_xin_cap = g_xin ? n : 0;
  }
  g_xin_valid = g_xin != NULL;
  if (g_xin_valid) {
    memcpy(g_xin, x, n);
    g_xin_n = n;
  }
  return 0;
}

void dsr_input_forget(void) { g_xin_valid = 0; }

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

static void *g_pin_host[DSR_NPIN], *g_pin_dev[DSR_NPIN];
static size_t g_pin_cap[DSR_NPIN];

static int pin_reserve(int slot, size_t n) {
  if (slot < 0 || slot >= DSR_NPIN) return dsr_failf("pinned staging: bad slot");
  if (n <= g_pin_cap[slot]) return 0;
  if (g_pin_host[slot]) {
    hipStreamSynchronize(dsr_stream);
    hipHostFree(g_pin_host[slot]);
    g_pin_host[slot] = g_pin_dev[slot] = NULL;
    g_pin_cap[slot] = 0;
  }
  const size_t cap = n < 65536 ? 65536 : n + n / 4;
  void *h = NULL, *d = NULL;
  DSR_TRY(hipHostMalloc(&h, cap, hipHostMallocMapped | hipHostMallocCoherent), "pinned staging");
  if (hipHostGetDevicePointer(&d, h, 0) != hipSuccess) {
    hipHostFree(h);
    return dsr_failf("pinned staging: no device address");
  }
  g_pin_host[slot] = h;
  g_pin_dev[slot] = d;
  g_pin_cap[slot] = cap;
  return 0;
}

const void *dsr_pin_in(int slot, const void *src, size_t n) {
  if (pin_reserve(slot, n ? n : 16)) return NULL;
  if (n) memcpy(g_pin_host[slot], src, n);
  return g_pin_dev[slot];
}

void *dsr_pin_buf(int slot, size_t n) { return pin_reserve(slot, n ? n : 16) ? NULL : g_pin_dev[slot]; }

int dsr_pin_out(void *dst, int slot, size_t n) {
  DSR_TRY(hipStreamSynchronize(dsr_stream), "stream synchronize");
  if (n) memcpy(dst, g_pin_host[slot], n);
  return 0;
}

int dsr_pin_out_done(void *dst, int slot, size_t n, int n_words, unsigned epoch) {
  const volatile unsigned *w = (const volatile unsigned *)g_pin_host[DSR_PIN_DONE];
  struct timespec t0, t1;
  clock_gettime(CLOCK_MONOTONIC, &t0);
  for (int i = 0; i < n_words;) {
    if (__atomic_load_n(&w[i], __ATOMIC_ACQUIRE) == epoch) {
      i++;
      continue;
    }
    clock_gettime(CLOCK_MONOTONIC, &t1);
    if (t1.tv_sec - t0.tv_sec > 1) { /* not done: the launch failed or stalls; let the stream say why */
      DSR_TRY(hipStreamSynchronize(dsr_stream), "stream synchronize");
      return dsr_failf("a kernel did not report completion");
    }
  }
  if (n) memcpy(dst, g_pin_host[slot], n);
  return 0;
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

/* 64-bit mixing hash, eight bytes per step (the tail zero-padded, the length mixed in). */
static uint64_t mix64(uint64_t h, uint64_t v) {
  h = (h ^ v) * 0x9E3779B97F4A7C15ull;
  return h ^ (h >> 29);
}

static uint64_t fnv(uint64_t h, const void *p, size_t n) {
  const unsigned char *b = (const unsigned char *)p;
  size_t i = 0;
  for (; i + 8 <= n; i += 8) {
    uint64_t v;
    memcpy(&v, b + i, 8);
    h = mix64(h, v);
  }
  uint64_t t = 0;
  memcpy(&t, b + i, n - i);
  return mix64(h, t ^ ((uint64_t)n << 56));
}

/* Weights are registered once: a host array is keyed by its address and size, like the reference's
 * read-only mmap'd weights and INT8 blocks that are never rewritten (ds_ocr.c:611-622; the Metal
 * backend registers expert blocks the same way, ds_metal.m:244-258). To notice a new array placed at
 * a freed one's address, each key also keeps a sampled fingerprint: 16 windows of 64 bytes spread
 * evenly over the array (the whole array when it is at most 1 KiB), about 1 KiB read per call
 * whatever the size, hashed eight bytes at a time. Keys are found through a hash index on the
 * address. A caller that edits registered weights in place calls ds_hip_weights_changed. */
#define FP_WINDOWS 16
#define FP_WINDOW 64

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
/* open-addressing index: slot -> entry index + 1 (0: empty), 4 slots per entry of capacity */
static int *g_idx = NULL;
static size_t g_idx_n = 0;

static size_t idx_slot(const void *key, int is_block) {
  return (size_t)(mix64((uint64_t)(uintptr_t)key, (uint64_t)is_block) & (g_idx_n - 1));
}

static void idx_insert(int i) {
  size_t s = idx_slot(g_ent[i].key, g_ent[i].is_block);
  while (g_idx[s]) s = (s + 1) & (g_idx_n - 1);
  g_idx[s] = i + 1;
}

static void idx_rebuild(void) {
  memset(g_idx, 0, g_idx_n * sizeof(int));
  for (int i = 0; i < g_nent; i++) idx_insert(i);
}

static entry_t *find(const void *key, int is_block) {
  if (!g_idx) return NULL;
  for (size_t s = idx_slot(key, is_block);; s = (s + 1) & (g_idx_n - 1)) {
    const int i = g_idx[s] - 1;
    if (i < 0) return NULL;
    if (g_ent[i].key == key && g_ent[i].is_block == is_block) return &g_ent[i];
  }
}

static void drop(entry_t *e) {
  hipStreamSynchronize(dsr_stream);
  if (e->dev) hipFree(e->dev);
  if (e->aux) hipFree(e->aux);
  *e = g_ent[--g_nent];
  idx_rebuild();
}

/* A new zeroed entry; the caller sets key and is_block, then calls add_done. */
static entry_t *add(void) {
  if (g_nent == g_cap) {
    int nc = g_cap ? 2 * g_cap : 64;
    entry_t *ne = (entry_t *)realloc(g_ent, (size_t)nc * sizeof(entry_t));
    int *ni = (int *)calloc((size_t)nc * 4, sizeof(int));
    if (!ne || !ni) {
      if (ne) g_ent = ne;
      free(ni);
      return NULL;
    }
    g_ent = ne;
    g_cap = nc;
    free(g_idx);
    g_idx = ni;
    g_idx_n = (size_t)nc * 4;
    idx_rebuild();
  }
  entry_t *e = &g_ent[g_nent++];
  memset(e, 0, sizeof *e);
  return e;
}

static void add_done(entry_t *e) { idx_insert((int)(e - g_ent)); }

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
    add_done(e);
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
  add_done(e);
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
  add_done(e);
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
