/* ds_hip_st.c — DeepSeek-OCR safetensors checkpoints straight into device MoE layers (ds_hip.h).
 *
 * The reference maps its safetensors shards (ds_safetensors.h:50-75, multi_safetensors_find), loads
 * the decoder's BF16 expert weights by name (ds_ocr.c:653-686), fuses each expert's gate and up
 * rows (ds_ocr.c:696-768) and quantizes every block on the host at each load
 * (ds_quantize_moe_int4, ds_ocr.c:781-841). Here the shards are mapped read-only, each tensor is
 * copied to the device once, and the quantizer kernel (bit-identical to ds_int4_quantize_bf16)
 * writes the codes straight into the layer arena. With ds_hip_arena_save the result can be kept
 * and reloaded without the BF16 checkpoint.
 *
 * A safetensors file is an 8-byte little-endian header length N, N bytes of JSON mapping each
 * tensor name to {"dtype", "shape", "data_offsets": [begin, end)} (offsets relative to the byte
 * after the header; an optional "__metadata__" object holds strings), then the data.
 */
#define _DEFAULT_SOURCE
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "dsr.h"
#include "ds_hip.h"

#define ST_MAX_DIMS 8
#define ST_NAME 256

typedef struct {
  char name[ST_NAME];
  int dtype; /* DS_HIP_ST_* */
  int ndim;
  int64_t shape[ST_MAX_DIMS];
  const uint8_t *data;
  size_t bytes;
} st_tensor_t;

typedef struct {
  int nfiles;
  void **maps;
  size_t *sizes;
  int n, cap;
  st_tensor_t *t;
} st_set_t;

/* ---------------------------------------------------------------- JSON header parsing */
typedef struct {
  const char *p, *end;
} jcur_t;

static void jws(jcur_t *c) {
  while (c->p < c->end && (*c->p == ' ' || *c->p == '\t' || *c->p == '\n' || *c->p == '\r')) c->p++;
}
static int jch(jcur_t *c, char ch) {
  jws(c);
  if (c->p < c->end && *c->p == ch) {
    c->p++;
    return 1;
  }
  return 0;
}
/* A string into out (escapes other than \" and \\ are kept verbatim; names never use them). */
static int jstr(jcur_t *c, char *out, size_t cap) {
  jws(c);
  if (c->p >= c->end || *c->p != '"') return -1;
  c->p++;
  size_t k = 0;
  while (c->p < c->end && *c->p != '"') {
    char ch = *c->p++;
    if (ch == '\\' && c->p < c->end) ch = *c->p++;
    if (k + 1 >= cap) return -1;
    out[k++] = ch;
  }
  if (c->p >= c->end) return -1;
  c->p++;
  out[k] = 0;
  return 0;
}
static int jint(jcur_t *c, int64_t *v) {
  jws(c);
  const char *q = c->p;
  int neg = 0;
  if (q < c->end && *q == '-') {
    neg = 1;
    q++;
  }
  if (q >= c->end || *q < '0' || *q > '9') return -1;
  uint64_t x = 0;
  while (q < c->end && *q >= '0' && *q <= '9') {
    if (x > (UINT64_MAX - 9) / 10) return -1;
    x = x * 10 + (uint64_t)(*q++ - '0');
  }
  if (x > (uint64_t)INT64_MAX) return -1;
  c->p = q;
  *v = neg ? -(int64_t)x : (int64_t)x;
  return 0;
}
static int jskip(jcur_t *c, int depth);
static int jskip_seq(jcur_t *c, char close, int depth, int keyed) {
  if (jch(c, close)) return 0;
  for (;;) {
    if (keyed) {
      char k[ST_NAME];
      if (jstr(c, k, sizeof k) || !jch(c, ':')) return -1;
    }
    if (jskip(c, depth + 1)) return -1;
    if (jch(c, close)) return 0;
    if (!jch(c, ',')) return -1;
  }
}
static int jskip(jcur_t *c, int depth) {
  if (depth > 16) return -1;
  jws(c);
  if (c->p >= c->end) return -1;
  char ch = *c->p;
  if (ch == '"') {
    char tmp[1024];
    return jstr(c, tmp, sizeof tmp);
  }
  if (ch == '{') {
    c->p++;
    return jskip_seq(c, '}', depth, 1);
  }
  if (ch == '[') {
    c->p++;
    return jskip_seq(c, ']', depth, 0);
  }
  /* number, true, false, null */
  const char *q = c->p;
  while (q < c->end && *q != ',' && *q != '}' && *q != ']' && *q != ' ' && *q != '\n' && *q != '\r' && *q != '\t')
    q++;
  if (q == c->p) return -1;
  c->p = q;
  return 0;
}
static int dtype_code(const char *s, size_t *elem) {
  if (!strcmp(s, "BF16")) {
    *elem = 2;
    return DS_HIP_ST_BF16;
  }
  if (!strcmp(s, "F32")) {
    *elem = 4;
    return DS_HIP_ST_F32;
  }
  if (!strcmp(s, "F16")) {
    *elem = 2;
    return DS_HIP_ST_F16;
  }
  *elem = 0;
  return DS_HIP_ST_OTHER;
}

static int st_push(st_set_t *S, const st_tensor_t *t) {
  if (S->n == S->cap) {
    int cap = S->cap ? 2 * S->cap : 256;
    st_tensor_t *nt = (st_tensor_t *)realloc(S->t, (size_t)cap * sizeof *nt);
    if (!nt) return dsr_failf("safetensors: out of host memory");
    S->t = nt;
    S->cap = cap;
  }
  S->t[S->n++] = *t;
  return 0;
}

/* Parses one mapped file's header and appends its tensors. */
static int st_parse(st_set_t *S, const uint8_t *base, size_t size, const char *path) {
  if (size < 8) return dsr_failf("safetensors: %s is too short", path);
  uint64_t hl = 0;
  for (int i = 7; i >= 0; i--) hl = (hl << 8) | base[i];
  if (hl > size - 8) return dsr_failf("safetensors: %s header length %llu exceeds the file", path, (unsigned long long)hl);
  const uint8_t *data0 = base + 8 + hl;
  const size_t data_bytes = size - 8 - hl;
  jcur_t c = {(const char *)base + 8, (const char *)base + 8 + hl};
  if (!jch(&c, '{')) return dsr_failf("safetensors: %s header is not a JSON object", path);
  if (jch(&c, '}')) return 0;
  for (;;) {
    st_tensor_t t;
    memset(&t, 0, sizeof t);
    if (jstr(&c, t.name, sizeof t.name) || !jch(&c, ':')) return dsr_failf("safetensors: %s: bad header key", path);
    if (!strcmp(t.name, "__metadata__")) {
      if (jskip(&c, 0)) return dsr_failf("safetensors: %s: bad __metadata__", path);
    } else {
      if (!jch(&c, '{')) return dsr_failf("safetensors: %s: entry %s is not an object", path, t.name);
      int64_t b = -1, e = -1;
      size_t elem = 0;
      int have_dt = 0, have_sh = 0;
      if (!jch(&c, '}')) {
        for (;;) {
          char key[64];
          if (jstr(&c, key, sizeof key) || !jch(&c, ':')) return dsr_failf("safetensors: %s: bad field in %s", path, t.name);
          if (!strcmp(key, "dtype")) {
            char dt[32];
            if (jstr(&c, dt, sizeof dt)) return dsr_failf("safetensors: %s: bad dtype in %s", path, t.name);
            t.dtype = dtype_code(dt, &elem);
            have_dt = 1;
          } else if (!strcmp(key, "shape")) {
            if (!jch(&c, '[')) return dsr_failf("safetensors: %s: bad shape in %s", path, t.name);
            if (!jch(&c, ']')) {
              for (;;) {
                int64_t v;
                if (t.ndim >= ST_MAX_DIMS || jint(&c, &v) || v < 0)
                  return dsr_failf("safetensors: %s: bad shape in %s", path, t.name);
                t.shape[t.ndim++] = v;
                if (jch(&c, ']')) break;
                if (!jch(&c, ',')) return dsr_failf("safetensors: %s: bad shape in %s", path, t.name);
              }
            }
            have_sh = 1;
          } else if (!strcmp(key, "data_offsets")) {
            if (!jch(&c, '[') || jint(&c, &b) || !jch(&c, ',') || jint(&c, &e) || !jch(&c, ']'))
              return dsr_failf("safetensors: %s: bad data_offsets in %s", path, t.name);
          } else if (jskip(&c, 1)) {
            return dsr_failf("safetensors: %s: bad field %s in %s", path, key, t.name);
          }
          if (jch(&c, '}')) break;
          if (!jch(&c, ',')) return dsr_failf("safetensors: %s: bad entry %s", path, t.name);
        }
      }
      if (!have_dt || !have_sh || b < 0 || e < b || (uint64_t)e > data_bytes)
        return dsr_failf("safetensors: %s: entry %s is incomplete or out of bounds", path, t.name);
      t.data = data0 + b;
      t.bytes = (size_t)(e - b);
      if (elem) {
        uint64_t numel = 1;
        for (int d = 0; d < t.ndim; d++) numel *= (uint64_t)t.shape[d];
        if (numel * elem != t.bytes)
          return dsr_failf("safetensors: %s: %s holds %zu bytes for %llu elements", path, t.name, t.bytes,
                           (unsigned long long)numel);
      }
      if (st_push(S, &t)) return -1;
    }
    if (jch(&c, '}')) return 0;
    if (!jch(&c, ',')) return dsr_failf("safetensors: %s: bad header", path);
  }
}

static void st_close(st_set_t *S) {
  if (!S) return;
  for (int i = 0; i < S->nfiles; i++)
    if (S->maps[i]) munmap(S->maps[i], S->sizes[i]);
  free(S->maps);
  free(S->sizes);
  free(S->t);
  free(S);
}

static st_set_t *st_open(const char *const *files, int n_files) {
  if (!files || n_files <= 0) {
    dsr_failf("safetensors: no files");
    return NULL;
  }
  st_set_t *S = (st_set_t *)calloc(1, sizeof *S);
  if (!S) return NULL;
  S->maps = (void **)calloc((size_t)n_files, sizeof(void *));
  S->sizes = (size_t *)calloc((size_t)n_files, sizeof(size_t));
  if (!S->maps || !S->sizes) {
    st_close(S);
    return NULL;
  }
  S->nfiles = n_files;
  for (int i = 0; i < n_files; i++) {
    int fd = files[i] ? open(files[i], O_RDONLY) : -1;
    struct stat sb;
    if (fd < 0 || fstat(fd, &sb) || sb.st_size <= 0) {
      if (fd >= 0) close(fd);
      dsr_failf("safetensors: cannot open %s", files[i] ? files[i] : "(null)");
      st_close(S);
      return NULL;
    }
    void *m = mmap(NULL, (size_t)sb.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) {
      dsr_failf("safetensors: cannot map %s", files[i]);
      st_close(S);
      return NULL;
    }
    S->maps[i] = m;
    S->sizes[i] = (size_t)sb.st_size;
    if (st_parse(S, (const uint8_t *)m, S->sizes[i], files[i])) {
      st_close(S);
      return NULL;
    }
  }
  return S;
}

static const st_tensor_t *st_find(const st_set_t *S, const char *name) {
  for (int i = 0; i < S->n; i++)
    if (!strcmp(S->t[i].name, name)) return &S->t[i];
  return NULL;
}

/* A 2-D BF16 tensor of shape [rows, cols] (cols, rows checked when > 0). */
static const st_tensor_t *st_bf16_2d(const st_set_t *S, const char *name, int64_t rows, int64_t cols) {
  const st_tensor_t *t = st_find(S, name);
  if (!t) {
    dsr_failf("safetensors: tensor %s not found", name);
    return NULL;
  }
  if (t->dtype != DS_HIP_ST_BF16 || t->ndim != 2 || (rows > 0 && t->shape[0] != rows) || (cols > 0 && t->shape[1] != cols)) {
    dsr_failf("safetensors: %s is not a BF16 [%lld, %lld] matrix", name, (long long)rows, (long long)cols);
    return NULL;
  }
  return t;
}

/* ---------------------------------------------------------------- public API */
int ds_hip_safetensors_info(const char *const *files, int n_files, const char *name, int *dtype, int64_t *shape,
                            int max_dims) {
  st_set_t *S = st_open(files, n_files);
  if (!S) return -1;
  const st_tensor_t *t = name ? st_find(S, name) : NULL;
  int rc;
  if (!t) {
    rc = dsr_failf("safetensors: tensor %s not found", name ? name : "(null)");
  } else {
    if (dtype) *dtype = t->dtype;
    for (int d = 0; d < t->ndim && d < max_dims && shape; d++) shape[d] = t->shape[d];
    rc = t->ndim;
  }
  st_close(S);
  return rc;
}

int ds_hip_load_moe_layers(const char *const *files, int n_files, int first_layer, int n_layers, int top_k,
                           ds_hip_layer_t **layers) {
  if (!layers || n_layers <= 0 || first_layer < 0 || top_k <= 0) return dsr_failf("ds_hip_load_moe_layers: invalid arguments");
  if (dsr_init()) return -1;
  st_set_t *S = st_open(files, n_files);
  if (!S) return -1;
  int made = 0, rc = 0;
  uint16_t *gu_dev = NULL, *dn_dev = NULL;
  float *rf = NULL;
  size_t stage = 0;
  char name[ST_NAME];
  for (int li = 0; li < n_layers && !rc; li++) {
    const int l = first_layer + li;
    snprintf(name, sizeof name, "model.layers.%d.mlp.gate.weight", l);
    const st_tensor_t *router = st_find(S, name);
    if (!router || router->ndim != 2 || (router->dtype != DS_HIP_ST_BF16 && router->dtype != DS_HIP_ST_F32)) {
      rc = dsr_failf("ds_hip_load_moe_layers: %s missing or not a BF16/F32 matrix (layer %d is not a MoE layer?)",
                     name, l);
      break;
    }
    const int E = (int)router->shape[0], H = (int)router->shape[1];
    snprintf(name, sizeof name, "model.layers.%d.mlp.experts.0.gate_proj.weight", l);
    const st_tensor_t *g0 = st_bf16_2d(S, name, -1, H);
    snprintf(name, sizeof name, "model.layers.%d.mlp.shared_experts.gate_proj.weight", l);
    const st_tensor_t *s0 = g0 ? st_bf16_2d(S, name, -1, H) : NULL;
    if (!g0 || !s0) {
      rc = -1;
      break;
    }
    const int I = (int)g0->shape[0], SI = (int)s0->shape[0];
    ds_hip_layer_t *L = ds_hip_layer_create(H, I, E, top_k, SI);
    if (!L) {
      rc = -1;
      break;
    }
    layers[made++] = L;
    /* router: BF16 → both forms (f32 = the bf16 value widened, as the reference's F32 load of a BF16
     * tensor gives); F32 → f32 only (the reference then has no bf16 router) */
    const size_t nr = (size_t)E * H;
    free(rf);
    rf = (float *)malloc(nr * 4);
    if (!rf) {
      rc = dsr_failf("ds_hip_load_moe_layers: out of host memory");
      break;
    }
    if (router->dtype == DS_HIP_ST_BF16) {
      const uint16_t *rb = (const uint16_t *)router->data;
      for (size_t i = 0; i < nr; i++) {
        const uint32_t u = (uint32_t)rb[i] << 16;
        memcpy(&rf[i], &u, 4);
      }
      rc = ds_hip_layer_set_router(L, rf, rb);
    } else {
      memcpy(rf, router->data, nr * 4);
      rc = ds_hip_layer_set_router(L, rf, NULL);
    }
    if (rc) break;
    const size_t need = (size_t)2 * (I > SI ? I : SI) * H * 2;
    if (need > stage) {
      ds_hip_free(gu_dev);
      ds_hip_free(dn_dev);
      gu_dev = (uint16_t *)ds_hip_malloc(need);
      dn_dev = (uint16_t *)ds_hip_malloc(need / 2);
      stage = need;
      if (!gu_dev || !dn_dev) {
        rc = dsr_failf("ds_hip_load_moe_layers: staging allocation failed");
        break;
      }
    }
    for (int e = -1; e < E && !rc; e++) {
      const int In = e < 0 ? SI : I;
      const st_tensor_t *g, *u, *d;
      if (e < 0) {
        snprintf(name, sizeof name, "model.layers.%d.mlp.shared_experts.gate_proj.weight", l);
        g = st_bf16_2d(S, name, In, H);
        snprintf(name, sizeof name, "model.layers.%d.mlp.shared_experts.up_proj.weight", l);
        u = st_bf16_2d(S, name, In, H);
        snprintf(name, sizeof name, "model.layers.%d.mlp.shared_experts.down_proj.weight", l);
        d = st_bf16_2d(S, name, H, In);
      } else {
        snprintf(name, sizeof name, "model.layers.%d.mlp.experts.%d.gate_proj.weight", l, e);
        g = st_bf16_2d(S, name, In, H);
        snprintf(name, sizeof name, "model.layers.%d.mlp.experts.%d.up_proj.weight", l, e);
        u = st_bf16_2d(S, name, In, H);
        snprintf(name, sizeof name, "model.layers.%d.mlp.experts.%d.down_proj.weight", l, e);
        d = st_bf16_2d(S, name, H, In);
      }
      if (!g || !u || !d) {
        rc = -1;
        break;
      }
      /* fused gate_up = [gate rows; up rows] (ds_ocr.c:724-735) */
      const size_t half = (size_t)In * H * 2;
      rc = ds_hip_memcpy_h2d(gu_dev, g->data, half) || ds_hip_memcpy_h2d((char *)gu_dev + half, u->data, half) ||
           ds_hip_memcpy_h2d(dn_dev, d->data, half) || ds_hip_layer_quantize_expert(L, e, gu_dev, dn_dev);
      if (!rc) rc = ds_hip_sync();  /* the staging buffers are reused by the next expert */
    }
  }
  ds_hip_free(gu_dev);
  ds_hip_free(dn_dev);
  free(rf);
  st_close(S);
  if (rc) {
    for (int i = 0; i < made; i++) ds_hip_layer_destroy(layers[i]);
    for (int i = 0; i < made; i++) layers[i] = NULL;
    return -1;
  }
  return n_layers;
}

int ds_hip_load_dense(const char *const *files, int n_files, int layer, ds_hip_dense_t **dense) {
  if (!dense || layer < 0) return dsr_failf("ds_hip_load_dense: invalid arguments");
  *dense = NULL;
  st_set_t *S = st_open(files, n_files);
  if (!S) return -1;
  char name[ST_NAME];
  snprintf(name, sizeof name, "model.layers.%d.mlp.gate_proj.weight", layer);
  const st_tensor_t *g = st_bf16_2d(S, name, -1, -1);
  const st_tensor_t *u = NULL, *d = NULL;
  if (g) {
    snprintf(name, sizeof name, "model.layers.%d.mlp.up_proj.weight", layer);
    u = st_bf16_2d(S, name, g->shape[0], g->shape[1]);
  }
  if (u) {
    snprintf(name, sizeof name, "model.layers.%d.mlp.down_proj.weight", layer);
    d = st_bf16_2d(S, name, g->shape[1], g->shape[0]);
  }
  if (d)
    *dense = ds_hip_dense_create((int)g->shape[1], (int)g->shape[0], (const uint16_t *)g->data,
                                 (const uint16_t *)u->data, (const uint16_t *)d->data);
  st_close(S);
  return *dense ? 0 : -1;
}

int ds_hip_load_lm_head(const char *const *files, int n_files, uint16_t **lm_head_dev, int *vocab, int *hidden) {
  if (!lm_head_dev) return dsr_failf("ds_hip_load_lm_head: invalid arguments");
  *lm_head_dev = NULL;
  if (dsr_init()) return -1;
  st_set_t *S = st_open(files, n_files);
  if (!S) return -1;
  const st_tensor_t *t = st_bf16_2d(S, "lm_head.weight", -1, -1);
  int rc = t ? 0 : -1;
  uint16_t *w = NULL;
  if (!rc) {
    w = (uint16_t *)ds_hip_malloc(t->bytes);
    rc = !w || ds_hip_memcpy_h2d(w, t->data, t->bytes) || ds_hip_sync();
  }
  if (!rc) {
    *lm_head_dev = w;
    if (vocab) *vocab = (int)t->shape[0];
    if (hidden) *hidden = (int)t->shape[1];
  } else {
    ds_hip_free(w);
  }
  st_close(S);
  return rc ? -1 : 0;
}
