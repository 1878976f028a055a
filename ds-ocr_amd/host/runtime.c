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

/* Content hash of every byte: four lanes of the xxHash64 round (acc = rotl(acc + w*P2, 31) * P1)
 * over 32-byte stripes, the tail through FNV-1a. Any change of a cached host array is seen, also
 * when a new array reuses a freed one's address; arrays of 32 MiB and more are hashed in parallel
 * slices. */
#define XXP1 11400714785092567791ull
#define XXP2 14029467366897019727ull
static uint64_t rotl64(uint64_t v, int r) { return (v << r) | (v >> (64 - r)); }

static uint64_t hash_slice(const unsigned char *b, size_t n, uint64_t seed) {
  uint64_t v[4] = {seed + XXP1 + XXP2, seed + XXP2, seed, seed - XXP1};
  size_t i = 0;
  for (; i + 32 <= n; i += 32) {
    for (int l = 0; l < 4; l++) {
      uint64_t w;
      memcpy(&w, b + i + 8 * l, 8);
      v[l] = rotl64(v[l] + w * XXP2, 31) * XXP1;
    }
  }
  uint64_t h = rotl64(v[0], 1) + rotl64(v[1], 7) + rotl64(v[2], 12) + rotl64(v[3], 18);
  return fnv(h ^ (uint64_t)n, b + i, n - i);
}

typedef struct {
  const unsigned char *b;
  size_t n;
  uint64_t h;
} slice_t;

static void *hash_worker(void *arg) {
  slice_t *s = (slice_t *)arg;
  s->h = hash_slice(s->b, s->n, 0x9E3779B97F4A7C15ull);
  return NULL;
}

static uint64_t fingerprint(const void *p, size_t n) {
  const unsigned char *b = (const unsigned char *)p;
  uint64_t h = fnv(1469598103934665603ull, &n, sizeof n);
  enum { MAXS = 8 };
  long ncpu = sysconf(_SC_NPROCESSORS_ONLN);
  int ns = n >= ((size_t)32 << 20) ? (int)(ncpu < MAXS ? (ncpu < 1 ? 1 : ncpu) : MAXS) : 1;
  slice_t sl[MAXS];
  pthread_t th[MAXS];
  int started[MAXS] = {0};
  size_t per = ((n / (size_t)ns) + 31) & ~(size_t)31;
  for (int i = 0; i < ns; i++) {
    size_t s0 = per * (size_t)i < n ? per * (size_t)i : n;
    size_t s1 = i == ns - 1 ? n : (per * (size_t)(i + 1) < n ? per * (size_t)(i + 1) : n);
    sl[i].b = b + s0;
    sl[i].n = s1 - s0;
    if (i > 0 && pthread_create(&th[i], NULL, hash_worker, &sl[i]) == 0) started[i] = 1;
  }
  hash_worker(&sl[0]);
  for (int i = 1; i < ns; i++) {
    if (started[i])
      pthread_join(th[i], NULL);
    else
      hash_worker(&sl[i]);
  }
  for (int i = 0; i < ns; i++) h = fnv(h, &sl[i].h, sizeof sl[i].h);
  return h;
}

typedef struct {
  const void *key;
  uint64_t fp;
  size_t bytes;
  void *dev; /* weights: the copy; blocks: q (scale, offset follow in sdev/odev) */
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
  return 0;
}
