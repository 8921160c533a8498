/*
 * pai_hip host layer (C11): device bring-up, packed-matrix handles,
 * argument validation, dispatch to the gfx950 kernels and HIP-error to
 * pai_status_t mapping. See include/pai_hip.h for the contract.
 *
 * No CPU fallback exists: without a usable gfx950 device every compute
 * entry point returns PAI_ERR_INIT.
 */
#define _GNU_SOURCE
#include "pai_hip.h"

#include <hip/hip_runtime_api.h>
#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "paik.h"

struct pai_qmat {
  uint32_t type;
  uint64_t n, k;
  uint64_t packed_bytes; /* N * type_bytes(K) */
  void *dev;             /* one allocation holding every plane */
  uint64_t dev_bytes;
  int device;
  paik_qview_t view;
  /* 16-bit copy of the activations for the MFMA path (see x16_workspace);
   * guarded by g_x16_lock */
  void *x16;
  uint64_t x16_bytes;
  /* the split parts of MFMA launches led by this handle (see part_workspace) */
  void *pw;
  uint64_t pw_bytes;
  /* workspaces replaced by larger ones: a HIP graph captured earlier may
   * still use them, so they are freed only with the handle */
  struct pai_retired *retired;
};

struct pai_retired {
  void *p;
  struct pai_retired *next;
};

/* ---------------------------------------------------------------------- */
/* Errors                                                                   */
/* ---------------------------------------------------------------------- */

static _Thread_local char t_err[256];

/* Shared with pai_gguf.c; not exported from the library. */
__attribute__((visibility("hidden"))) pai_status_t pai__fail(pai_status_t st, const char *fmt,
                                                             ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(t_err, sizeof t_err, fmt, ap);
  va_end(ap);
  return st;
}
#define fail pai__fail

const char *pai_hip_last_error(void) { return t_err; }

/* ---------------------------------------------------------------------- */
/* Measurement knobs                                                        */
/* ---------------------------------------------------------------------- */

paik_tune_t paik_tune;

pai_status_t pai_hip_set_tuning(uint32_t knob, int32_t value) {
  int32_t *f;
  switch (knob) {
  case PAI_TUNE_GEMM_SPLITS: f = &paik_tune.gemm_splits; break;
  case PAI_TUNE_GEMM_NO_X16: f = &paik_tune.gemm_no_x16; break;
  case PAI_TUNE_GEMM_ATOMIC_SPLITS: f = &paik_tune.gemm_atomic_splits; break;
  case PAI_TUNE_GEMV_WGS: f = &paik_tune.gemv_wgs; break;
  case PAI_TUNE_GEMV_ROWS: f = &paik_tune.gemv_rows; break;
  case PAI_TUNE_GEMV_NW: f = &paik_tune.gemv_nw; break;
  case PAI_TUNE_GEMV_NO_MX: f = &paik_tune.gemv_no_mx; break;
  case PAI_TUNE_MFMA_MIN_M: f = &paik_tune.mfma_min_m; break;
  case PAI_TUNE_GEMM_TILE: f = &paik_tune.gemm_tile; break;
  case PAI_TUNE_V0_SEQUENTIAL: f = &paik_tune.v0_sequential; break;
  default: return fail(PAI_ERR_INVALID_ARG, "unknown tuning knob %u", knob);
  }
  if (value < 0) return fail(PAI_ERR_INVALID_ARG, "tuning value %d < 0", (int)value);
  *f = value;
  return PAI_OK;
}

/* hipError_t -> pai_status_t (sdk/include/pai/error.h codes). */
static pai_status_t map_hip(hipError_t e, const char *what) {
  pai_status_t st;
  switch (e) {
  case hipSuccess:
    return PAI_OK;
  case hipErrorOutOfMemory:
    st = PAI_ERR_NOMEM;
    break;
  case hipErrorNoDevice:
  case hipErrorInvalidDevice:
  case hipErrorNotInitialized:
  case hipErrorInsufficientDriver:
  case hipErrorNoBinaryForGpu:
    st = PAI_ERR_INIT;
    break;
  case hipErrorLaunchTimeOut:
    st = PAI_ERR_TIMEOUT;
    break;
  default:
    st = PAI_ERR_INTERNAL;
    break;
  }
  return fail(st, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

#define HIP_TRY(call, what)                                                    \
  do {                                                                         \
    hipError_t e_ = (call);                                                    \
    if (e_ != hipSuccess) return map_hip(e_, what);                            \
  } while (0)

/* ---------------------------------------------------------------------- */
/* Lifecycle                                                                */
/* ---------------------------------------------------------------------- */

static pthread_mutex_t g_lock = PTHREAD_MUTEX_INITIALIZER;
static int g_ready;
static int g_device;

/* Device address of each device's copy of the no-allocation scratch array
 * (qscratch.hip), taken once per device with that device current: at
 * pai_hip_init for the init device, else at that device's first
 * no-allocation call. Guarded by g_lock. */
#define PAI_MAX_DEVICES 64
static void *g_scratch[PAI_MAX_DEVICES];

/* Host-pointer staging (grow-only), guarded by g_stage_lock. */
static pthread_mutex_t g_stage_lock = PTHREAD_MUTEX_INITIALIZER;
static void *g_stage;
static uint64_t g_stage_bytes;

pai_status_t pai_hip_init(void) {
  pthread_mutex_lock(&g_lock);
  if (g_ready) {
    pthread_mutex_unlock(&g_lock);
    return PAI_OK;
  }
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count <= 0) {
    pthread_mutex_unlock(&g_lock);
    return fail(PAI_ERR_INIT, "no HIP device (%s)", hipGetErrorString(e));
  }
  int dev = 0;
  e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    pthread_mutex_unlock(&g_lock);
    return map_hip(e, "hipGetDevice");
  }
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess) {
    pthread_mutex_unlock(&g_lock);
    return map_hip(e, "hipGetDeviceProperties");
  }
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    pthread_mutex_unlock(&g_lock);
    return fail(PAI_ERR_INIT, "device %d is %s; kernels are built for gfx950", dev,
                prop.gcnArchName);
  }
  if (dev >= 0 && dev < PAI_MAX_DEVICES && g_scratch[dev] == NULL) {
    const int se = paik_scratch_address(&g_scratch[dev]);
    if (se != 0) {
      pthread_mutex_unlock(&g_lock);
      return map_hip((hipError_t)se, "hipGetSymbolAddress(scratch)");
    }
  }
  g_device = dev;
  g_ready = 1;
  pthread_mutex_unlock(&g_lock);
  return PAI_OK;
}

/* The current device's scratch address (NULL with the status on failure). */
static void *scratch_here(pai_status_t *st) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    *st = map_hip(e, "hipGetDevice");
    return NULL;
  }
  if (dev < 0 || dev >= PAI_MAX_DEVICES) {
    *st = fail(PAI_ERR_UNSUPPORTED, "device %d above %d", dev, PAI_MAX_DEVICES - 1);
    return NULL;
  }
  pthread_mutex_lock(&g_lock);
  if (g_scratch[dev] == NULL) {
    const int se = paik_scratch_address(&g_scratch[dev]);
    if (se != 0) {
      pthread_mutex_unlock(&g_lock);
      *st = map_hip((hipError_t)se, "hipGetSymbolAddress(scratch)");
      return NULL;
    }
  }
  void *p = g_scratch[dev];
  pthread_mutex_unlock(&g_lock);
  *st = PAI_OK;
  return p;
}

pai_status_t pai_hip_shutdown(void) {
  pthread_mutex_lock(&g_stage_lock);
  if (g_stage != NULL) {
    (void)hipFree(g_stage);
    g_stage = NULL;
    g_stage_bytes = 0;
  }
  pthread_mutex_unlock(&g_stage_lock);
  pthread_mutex_lock(&g_lock);
  g_ready = 0;
  pthread_mutex_unlock(&g_lock);
  return PAI_OK;
}

static pai_status_t ensure_ready(void) {
  if (g_ready) return PAI_OK;
  return pai_hip_init();
}

/* ---------------------------------------------------------------------- */
/* Formats and layout                                                       */
/* ---------------------------------------------------------------------- */

static uint64_t block_elems(uint32_t type) {
  switch (type) {
  case PAI_QTYPE_Q4_0:
  case PAI_QTYPE_Q8_0:
    return 32u;
  case PAI_QTYPE_Q4_K:
  case PAI_QTYPE_Q6_K:
    return 256u;
  default:
    return 0u;
  }
}

static uint64_t block_bytes(uint32_t type) {
  switch (type) {
  case PAI_QTYPE_Q4_0: return 18u;
  case PAI_QTYPE_Q8_0: return 34u;
  case PAI_QTYPE_Q4_K: return 144u;
  case PAI_QTYPE_Q6_K: return 210u;
  default: return 0u;
  }
}

/* adapters/llama/gguf.c:562-597 semantics for the four supported types. */
uint64_t pai_qtype_bytes(uint32_t type, uint64_t numel) {
  const uint64_t qk = block_elems(type);
  if (qk == 0u || numel % qk != 0u) return 0u;
  return numel / qk * block_bytes(type);
}

static uint64_t align256(uint64_t v) { return (v + 255u) & ~(uint64_t)255u; }

uint64_t paik_plan_layout(uint32_t type, uint64_t n, uint64_t k, uint64_t *off_q,
                          uint64_t *off_aux, uint64_t *off_meta, uint64_t *off_d) {
  const uint64_t qk = block_elems(type);
  if (qk == 0u || n == 0u || k == 0u || k % qk != 0u) return 0u;
  const uint64_t nb = k / qk;
  uint64_t q_bytes = 0, aux_bytes = 0, meta_bytes = 0, d_bytes = 0;
  switch (type) {
  case PAI_QTYPE_Q8_0: q_bytes = n * k; d_bytes = n * nb * 2u; break;
  case PAI_QTYPE_Q4_0: q_bytes = n * k / 2u; d_bytes = n * nb * 2u; break;
  case PAI_QTYPE_Q4_K: q_bytes = n * k / 2u; meta_bytes = n * nb * 16u; break;
  case PAI_QTYPE_Q6_K:
    q_bytes = n * k / 2u;
    aux_bytes = n * k / 4u;
    meta_bytes = n * nb * 16u;
    d_bytes = n * nb * 2u;
    break;
  default: return 0u;
  }
  uint64_t off = 0;
  *off_q = off;
  off = align256(off + q_bytes);
  *off_aux = off;
  off = align256(off + aux_bytes);
  *off_meta = off;
  off = align256(off + meta_bytes);
  *off_d = off;
  off = align256(off + d_bytes);
  return off;
}

/* Kernel index math is 32-bit in rows/columns; byte offsets are 64-bit. */
#define PAI_MAX_DIM ((uint64_t)1 << 30)

static pai_status_t check_shape(uint32_t type, uint64_t n, uint64_t k) {
  if (n == 0u || k == 0u) return fail(PAI_ERR_INVALID_ARG, "zero dimension");
  if (block_elems(type) == 0u) return fail(PAI_ERR_UNSUPPORTED, "ggml type %u not supported", type);
  if (k % block_elems(type) != 0u)
    return fail(PAI_ERR_UNSUPPORTED, "K=%llu is not a whole number of %llu-element blocks",
                (unsigned long long)k, (unsigned long long)block_elems(type));
  if (n > PAI_MAX_DIM || k > PAI_MAX_DIM) return fail(PAI_ERR_UNSUPPORTED, "dimension above 2^30");
  return PAI_OK;
}

static pai_status_t make_qmat(pai_qmat_t **out, uint32_t type, uint64_t n, uint64_t k,
                              const void *dev_native, void *stream) {
  uint64_t oq, oa, om, od;
  const uint64_t bytes = paik_plan_layout(type, n, k, &oq, &oa, &om, &od);
  pai_qmat_t *w = (pai_qmat_t *)calloc(1, sizeof *w);
  if (w == NULL) return fail(PAI_ERR_NOMEM, "host allocation");
  hipError_t e = hipMalloc(&w->dev, bytes);
  if (e != hipSuccess) {
    free(w);
    return map_hip(e, "hipMalloc(weights)");
  }
  w->type = type;
  w->n = n;
  w->k = k;
  w->packed_bytes = n * pai_qtype_bytes(type, k);
  w->dev_bytes = bytes;
  w->device = g_device;
  uint8_t *base = (uint8_t *)w->dev;
  w->view.q = base + oq;
  w->view.aux = base + oa;
  w->view.meta = base + om;
  w->view.d = (const uint16_t *)(base + od);
  w->view.type = type;
  w->view.n = (uint32_t)n;
  w->view.k = (uint32_t)k;
  w->view.nb = (uint32_t)(k / block_elems(type));
  w->view.q_stride = (uint32_t)(type == PAI_QTYPE_Q8_0 ? k : k / 2u);
  int le = paik_repack(&w->view, (const uint8_t *)dev_native, stream);
  if (le == 0) le = (int)hipStreamSynchronize((hipStream_t)stream);
  if (le != 0) {
    (void)hipFree(w->dev);
    free(w);
    return map_hip((hipError_t)le, "repack");
  }
  *out = w;
  return PAI_OK;
}

pai_status_t pai_qmat_upload(pai_qmat_t **out, uint32_t type, uint64_t n, uint64_t k,
                             const void *blocks, uint64_t nbytes) {
  if (out == NULL || blocks == NULL) return fail(PAI_ERR_INVALID_ARG, "NULL argument");
  *out = NULL;
  pai_status_t st = check_shape(type, n, k);
  if (st != PAI_OK) return st;
  if (nbytes != n * pai_qtype_bytes(type, k))
    return fail(PAI_ERR_MISMATCH, "nbytes=%llu, expected %llu", (unsigned long long)nbytes,
                (unsigned long long)(n * pai_qtype_bytes(type, k)));
  st = ensure_ready();
  if (st != PAI_OK) return st;
  void *staging = NULL;
  HIP_TRY(hipMalloc(&staging, nbytes), "hipMalloc(staging)");
  hipError_t e = hipMemcpy(staging, blocks, nbytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(staging);
    return map_hip(e, "hipMemcpy(blocks)");
  }
  st = make_qmat(out, type, n, k, staging, NULL);
  (void)hipFree(staging);
  return st;
}

pai_status_t pai_qmat_upload_device(pai_qmat_t **out, uint32_t type, uint64_t n, uint64_t k,
                                    const void *dev_blocks, uint64_t nbytes, void *stream) {
  if (out == NULL || dev_blocks == NULL) return fail(PAI_ERR_INVALID_ARG, "NULL argument");
  *out = NULL;
  pai_status_t st = check_shape(type, n, k);
  if (st != PAI_OK) return st;
  if (nbytes != n * pai_qtype_bytes(type, k))
    return fail(PAI_ERR_MISMATCH, "nbytes=%llu, expected %llu", (unsigned long long)nbytes,
                (unsigned long long)(n * pai_qtype_bytes(type, k)));
  st = ensure_ready();
  if (st != PAI_OK) return st;
  return make_qmat(out, type, n, k, dev_blocks, stream);
}

/* Shared with pai_llama.c; not exported from the library. */
__attribute__((visibility("hidden"))) const paik_qview_t *pai__qmat_view(const pai_qmat_t *w) {
  return &w->view;
}
__attribute__((visibility("hidden"))) pai_status_t pai__map_hip(int e, const char *what) {
  return map_hip((hipError_t)e, what);
}
__attribute__((visibility("hidden"))) pai_status_t pai__ready(void) { return ensure_ready(); }

pai_status_t pai_qmat_free(pai_qmat_t *w) {
  if (w == NULL) return PAI_OK;
  if (w->x16 != NULL) (void)hipFree(w->x16);
  if (w->pw != NULL) (void)hipFree(w->pw);
  while (w->retired != NULL) {
    struct pai_retired *r = w->retired;
    w->retired = r->next;
    (void)hipFree(r->p);
    free(r);
  }
  hipError_t e = hipFree(w->dev);
  free(w);
  return e == hipSuccess ? PAI_OK : map_hip(e, "hipFree(weights)");
}

pai_status_t pai_qmat_shape(const pai_qmat_t *w, uint32_t *type, uint64_t *n, uint64_t *k) {
  if (w == NULL) return fail(PAI_ERR_INVALID_ARG, "NULL handle");
  if (type != NULL) *type = w->type;
  if (n != NULL) *n = w->n;
  if (k != NULL) *k = w->k;
  return PAI_OK;
}

uint64_t pai_qmat_bytes(const pai_qmat_t *w) { return w != NULL ? w->packed_bytes : 0u; }

/* ---------------------------------------------------------------------- */
/* Compute                                                                  */
/* ---------------------------------------------------------------------- */

#define PAI_MFMA_MIN_M 8u
/* Token count from which calls take the 16-bit MFMA GEMM; below it the
 * GEMV kernels (PAI_MFMA_MIN_M, or the mfma_min_m tuning field). */
static uint64_t mfma_min_m(void) {
  const int32_t r = paik_tune.mfma_min_m;
  return r >= 2 && r <= 4096 ? (uint64_t)r : PAI_MFMA_MIN_M;
}

/* Calls that take the GEMV kernels: under mfma_min_m() tokens, the
 * PAI_QGEMM_FP32 flag, or up to 8 tokens that one launch of the
 * matrix-core GEMV covers (its weight operands serve every token, so it
 * streams W once where the 16-bit GEMM adds conversion and fill launches). */
static int gemv_call(const pai_qmat_t *w, uint64_t m, uint32_t flags) {
  if (m < mfma_min_m() || (flags & PAI_QGEMM_FP32) != 0u) return 1;
  return m <= 8u && paik_gemv_mx_tokens((uint32_t)w->k, (uint32_t)m) >= m;
}

/* Workspace of the MFMA path: a 16-bit copy of up to PAI_X16_TOKENS tokens
 * of activations, owned by the matrix handle (calls on one handle do not
 * overlap, so they can share it). Allocated, or grown, by the first call
 * that needs it outside stream capture; a call made during capture uses
 * what is there (larger inputs run in token blocks of that size) or, with
 * nothing there, the kernels that stage the activations through registers.
 * Both give the same results. */
#define PAI_X16_TOKENS 1024u
static pthread_mutex_t g_x16_lock = PTHREAD_MUTEX_INITIALIZER;

/* A handle-owned device buffer of at least `want` bytes, grown outside
 * stream capture only (NULL with *bytes = 0, or the smaller buffer, during
 * capture). The buffer it replaces is not freed: a graph captured earlier
 * may still read and write it, so it joins the handle's retired list and is
 * freed by pai_qmat_free. Buffers only grow, and the largest size is
 * bounded (PAI_X16_TOKENS tokens), so the list stays short. Caller holds
 * g_x16_lock. */
static void *grow_workspace(pai_qmat_t *w, void **slot, uint64_t *slot_bytes, uint64_t want,
                            hipStream_t s, uint64_t *bytes) {
  if (*slot == NULL || *slot_bytes < want) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) == hipSuccess && cs == hipStreamCaptureStatusNone) {
      void *p = NULL;
      struct pai_retired *r = *slot != NULL ? (struct pai_retired *)malloc(sizeof *r) : NULL;
      if ((*slot == NULL || r != NULL) && hipMalloc(&p, want) == hipSuccess) {
        if (r != NULL) {
          r->p = *slot;
          r->next = w->retired;
          w->retired = r;
        }
        *slot = p;
        *slot_bytes = want;
      } else {
        free(r);
        (void)hipGetLastError(); /* keep the old buffer: the caller fits its work to it */
      }
    }
  }
  *bytes = *slot_bytes;
  return *slot;
}

static void *x16_workspace(const pai_qmat_t *cw, uint64_t m, hipStream_t s, uint64_t *bytes) {
  pai_qmat_t *w = (pai_qmat_t *)cw;
  const uint64_t tok = ((m < PAI_X16_TOKENS ? m : PAI_X16_TOKENS) + 255u) & ~(uint64_t)255u;
  pthread_mutex_lock(&g_x16_lock);
  void *p = grow_workspace(w, &w->x16, &w->x16_bytes, tok * w->k * 2u, s, bytes);
  pthread_mutex_unlock(&g_x16_lock);
  return p;
}

/* The split parts of a multi-matrix MFMA launch (matrices vs sharing x,
 * m tokens), owned by the first matrix's handle: parts summed in a fixed
 * order by one reduce launch, in place of a zero fill per matrix and
 * atomic adds (q/k/v at 32 tokens: 20.4 -> 18.0 us), and repeatable bit for
 * bit. Single-matrix launches keep the zero fill and atomics: there the
 * reduce launch, which reads every part, measured slower (down at 8
 * tokens: 19.0 -> 23.4 us; prefill down unchanged). NULL when the launch
 * does not split, or inside a capture without a large enough buffer. */
static void *part_workspace(const pai_qmat_t *cw, const paik_qview_t *const *vs, uint32_t count,
                            uint64_t m, hipStream_t s, uint64_t *bytes) {
  pai_qmat_t *w = (pai_qmat_t *)cw;
  *bytes = 0;
  if (count < 2u || paik_tune.gemm_atomic_splits != 0) return NULL;
  const uint64_t want = paik_gemm_part_bytes(vs, count, (uint32_t)m);
  if (want == 0u) return NULL;
  pthread_mutex_lock(&g_x16_lock);
  void *p = grow_workspace(w, &w->pw, &w->pw_bytes, want, s, bytes);
  pthread_mutex_unlock(&g_x16_lock);
  return p;
}

/* MFMA calls of up to this many tokens round x to 16 bits inside the GEMM
 * (register-staged activations: same tiles, split plan, rounding and
 * MFMA order, so the same bits) instead of in a conversion launch before
 * it. Measured on the Q4_K batched decode step at 32 tokens: o 15.5 ->
 * 14.1 us, down 24.0 -> 23.0, the q/k/v launch 18.5 -> 16.9; at 16 tokens
 * q/k/v 17.3 -> 15.6. Larger calls take the 16-bit copy, which the
 * activation tiles of many token tiles share. */
#define PAI_DIRECT_TOKENS 32u

/* Matrices sharing x in one MFMA launch. */
static pai_status_t launch_mfma_multi(const pai_qmat_t *const *ws, uint32_t count, uint64_t m,
                                      const float *x, float *const *ys, const float *gate,
                                      uint32_t flags, hipStream_t s) {
  uint64_t wb = 0, pb = 0;
  void *x16 = paik_tune.gemm_no_x16 != 0 || m <= PAI_DIRECT_TOKENS
                  ? NULL
                  : x16_workspace(ws[0], m, s, &wb);
  const paik_qview_t *vs[4];
  for (uint32_t i = 0; i < count; ++i) vs[i] = &ws[i]->view;
  void *part = gate != NULL ? NULL : part_workspace(ws[0], vs, count, m, s, &pb);
  const int e = paik_gemm_mfma_multi(vs, ys, count, (uint32_t)m, x, gate,
                                     (flags & PAI_QGEMM_MFMA_BF16) != 0u, x16, wb, part, pb, 0, s);
  return e == 0 ? PAI_OK : map_hip((hipError_t)e, "kernel launch");
}

static pai_status_t launch_mfma(const pai_qmat_t *w, uint64_t m, const float *x, float *y,
                                const float *gate, uint32_t flags, hipStream_t s) {
  return launch_mfma_multi(&w, 1u, m, x, &y, gate, flags, s);
}


static pai_status_t launch(const pai_qmat_t *w, uint64_t m, const float *x, float *y,
                           uint32_t flags, hipStream_t s) {
  if (gemv_call(w, m, flags)) {
    const int e = paik_gemv(&w->view, (uint32_t)m, x, y, s);
    return e == 0 ? PAI_OK : map_hip((hipError_t)e, "kernel launch");
  }
  return launch_mfma(w, m, x, y, NULL, flags, s);
}

static pai_status_t check_call(const pai_qmat_t *w, uint64_t m, const void *x, const void *y) {
  if (w == NULL || x == NULL || y == NULL) return fail(PAI_ERR_INVALID_ARG, "NULL argument");
  if (m == 0u) return fail(PAI_ERR_INVALID_ARG, "m == 0");
  if (m > PAI_MAX_DIM) return fail(PAI_ERR_UNSUPPORTED, "m above 2^30");
  return ensure_ready();
}

pai_status_t pai_qgemm_f32_async(const pai_qmat_t *w, uint64_t m, const float *x, float *y,
                                 uint32_t flags, void *stream) {
  pai_status_t st = check_call(w, m, x, y);
  if (st != PAI_OK) return st;
  if (((uintptr_t)x & 15u) != 0u || ((uintptr_t)y & 3u) != 0u)
    return fail(PAI_ERR_INVALID_ARG, "x must be 16-byte aligned, y 4-byte aligned");
  return launch(w, m, x, y, flags, (hipStream_t)stream);
}

/* pai_qgemm_f32_async without allocations: the 16-bit MFMA path takes its
 * copy of x from the current device's scratch array (PAIK_SCRATCH_BYTES,
 * shared by every call on that device) in token blocks that fit it, in
 * place of the handle's workspace; single-matrix launches split over K
 * zero-fill y with a kernel and add their parts with atomics, as in
 * pai_qgemm_f32_async. The GEMV paths use no scratch. Nothing here
 * allocates or frees device or host memory. */
pai_status_t pai_qgemm_f32_noalloc_async(const pai_qmat_t *w, uint64_t m, const float *x,
                                         float *y, uint32_t flags, void *stream) {
  pai_status_t st = check_call(w, m, x, y);
  if (st != PAI_OK) return st;
  if (((uintptr_t)x & 15u) != 0u || ((uintptr_t)y & 3u) != 0u)
    return fail(PAI_ERR_INVALID_ARG, "x must be 16-byte aligned, y 4-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  if (gemv_call(w, m, flags)) {
    const int e = paik_gemv(&w->view, (uint32_t)m, x, y, s);
    return e == 0 ? PAI_OK : map_hip((hipError_t)e, "kernel launch");
  }
  /* the smallest token block of the 16-bit path is 256 tokens */
  if (w->k * 2u * 256u > (uint64_t)PAIK_SCRATCH_BYTES)
    return fail(PAI_ERR_UNSUPPORTED,
                "K=%llu above %u: the no-allocation scratch (%u bytes) holds 256 tokens of "
                "16-bit activations up to that K",
                (unsigned long long)w->k, PAIK_SCRATCH_BYTES / 512u, PAIK_SCRATCH_BYTES);
  void *scratch = scratch_here(&st);
  if (scratch == NULL) return st;
  const paik_qview_t *v = &w->view;
  const int e = paik_gemm_mfma_multi(&v, &y, 1u, (uint32_t)m, x, NULL,
                                     (flags & PAI_QGEMM_MFMA_BF16) != 0u, scratch,
                                     PAIK_SCRATCH_BYTES, NULL, 0u, 0, s);
  return e == 0 ? PAI_OK : map_hip((hipError_t)e, "kernel launch");
}

#define PAI_MULTI_MAX 4u

pai_status_t pai_qgemm_f32_multi_async(const pai_qmat_t *const *ws, uint32_t count, uint64_t m,
                                       const float *x, float *const *ys, uint32_t flags,
                                       void *stream) {
  if (ws == NULL || ys == NULL || x == NULL) return fail(PAI_ERR_INVALID_ARG, "NULL argument");
  if (count == 0u || count > PAI_MULTI_MAX)
    return fail(PAI_ERR_INVALID_ARG, "count=%u, expected 1..%u", count, PAI_MULTI_MAX);
  for (uint32_t i = 0; i < count; ++i) {
    pai_status_t st = check_call(ws[i], m, x, ys[i]);
    if (st != PAI_OK) return st;
    if (((uintptr_t)ys[i] & 3u) != 0u) return fail(PAI_ERR_INVALID_ARG, "y must be 4-byte aligned");
    if (ws[i]->type != ws[0]->type || ws[i]->k != ws[0]->k)
      return fail(PAI_ERR_MISMATCH, "matrix %u differs from matrix 0 in type or K", i);
  }
  if (((uintptr_t)x & 15u) != 0u) return fail(PAI_ERR_INVALID_ARG, "x must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  if (gemv_call(ws[0], m, flags)) {
    const paik_qview_t *vs[PAI_MULTI_MAX];
    for (uint32_t i = 0; i < count; ++i) vs[i] = &ws[i]->view;
    const int e = paik_gemv_multi(vs, ys, count, (uint32_t)m, x, s);
    return e == 0 ? PAI_OK : map_hip((hipError_t)e, "kernel launch");
  }
  return launch_mfma_multi(ws, count, m, x, ys, NULL, flags, s);
}

pai_status_t pai_qgemm_f32_gate_up_async(const pai_qmat_t *w_gate, const pai_qmat_t *w_up,
                                         uint64_t m, const float *x, float *h, uint32_t flags,
                                         void *stream) {
  pai_status_t st = check_call(w_gate, m, x, h);
  if (st != PAI_OK) return st;
  st = check_call(w_up, m, x, h);
  if (st != PAI_OK) return st;
  if (w_up->type != w_gate->type || w_up->n != w_gate->n || w_up->k != w_gate->k)
    return fail(PAI_ERR_MISMATCH, "gate and up differ in type or shape");
  if (((uintptr_t)x & 15u) != 0u || ((uintptr_t)h & 3u) != 0u)
    return fail(PAI_ERR_INVALID_ARG, "x must be 16-byte aligned, h 4-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  if (gemv_call(w_gate, m, flags)) {
    /* one token, or a K the matrix-core GEMV does not take: the integer-dot
     * kernel, which needs whole rows in one launch */
    const int mx = m >= 2u && paik_gemv_mx_tokens((uint32_t)w_gate->k, (uint32_t)m) != 0u;
    if (!mx && w_gate->k > paik_gemv_pair_max_k())
      return fail(PAI_ERR_UNSUPPORTED, "K=%llu above %u for the fused gate/up product at M < %u",
                  (unsigned long long)w_gate->k, paik_gemv_pair_max_k(), PAI_MFMA_MIN_M);
    const int e = paik_gemv_silu_mul(&w_gate->view, &w_up->view, (uint32_t)m, x, h, s);
    return e == 0 ? PAI_OK : map_hip((hipError_t)e, "kernel launch");
  }
  /* When the up product would split over K (few tiles: batched decode),
   * gate and up run as one two-matrix launch whose split parts go to a
   * workspace, and the reduce launch that sums them forms silu(gate) * up.
   * Otherwise (or without the workspaces, inside a capture) the gate
   * product lands in h and the up product's epilogue forms silu(gate) * up
   * in place (whole sums, no split). */
  if (m <= PAI_X16_TOKENS && paik_tune.gemm_no_x16 == 0 &&
      paik_gemm_x16_splits(&w_up->view, (uint32_t)m) > 1u) {
    uint64_t wb = 0, pb = 0;
    const int direct = m <= PAI_DIRECT_TOKENS; /* x rounded inside the GEMM */
    void *x16 = direct ? NULL : x16_workspace(w_gate, m, s, &wb);
    const paik_qview_t *vs[2] = {&w_gate->view, &w_up->view};
    const uint64_t need = paik_gemm_part_bytes(vs, 2u, (uint32_t)m);
    void *part = part_workspace(w_gate, vs, 2u, m, s, &pb);
    if ((direct || (x16 != NULL && wb >= m * w_gate->k * 2u)) && part != NULL && need > 0u &&
        pb >= need) {
      float *outs[2] = {h, h};
      const int e = paik_gemm_mfma_multi(vs, outs, 2u, (uint32_t)m, x, NULL,
                                         (flags & PAI_QGEMM_MFMA_BF16) != 0u, x16, wb, part, pb,
                                         1, s);
      return e == 0 ? PAI_OK : map_hip((hipError_t)e, "kernel launch");
    }
  }
  st = launch_mfma(w_gate, m, x, h, NULL, flags, s);
  if (st != PAI_OK) return st;
  /* the up launch reads the 16-bit copy of x the gate launch just made,
   * when that holds every token (one conversion instead of two) */
  if (m > PAI_DIRECT_TOKENS && m <= PAI_X16_TOKENS && paik_tune.gemm_no_x16 == 0) {
    uint64_t wb = 0;
    void *x16 = x16_workspace(w_gate, m, s, &wb);
    if (x16 != NULL && wb >= ((m + 255u) & ~(uint64_t)255u) * w_gate->k * 2u) {
      const paik_qview_t *vu = &w_up->view;
      const int e = paik_gemm_mfma_multi(&vu, &h, 1u, (uint32_t)m, NULL, h,
                                         (flags & PAI_QGEMM_MFMA_BF16) != 0u, x16, wb, NULL, 0u,
                                         0, s);
      return e == 0 ? PAI_OK : map_hip((hipError_t)e, "kernel launch");
    }
  }
  return launch_mfma(w_up, m, x, h, h, flags, s);
}

pai_status_t pai_qgemm_f32(const pai_qmat_t *w, uint64_t m, const float *x, float *y,
                           uint32_t flags) {
  pai_status_t st = check_call(w, m, x, y);
  if (st != PAI_OK) return st;
  if ((flags & PAI_QGEMM_DEVICE_PTRS) != 0u) {
    st = pai_qgemm_f32_async(w, m, x, y, flags, NULL);
    if (st != PAI_OK) return st;
    HIP_TRY(hipStreamSynchronize(NULL), "qgemm");
    return PAI_OK;
  }
  const uint64_t xb = align256(m * w->k * sizeof(float));
  const uint64_t yb = align256(m * w->n * sizeof(float));
  pthread_mutex_lock(&g_stage_lock);
  if (g_stage_bytes < xb + yb) {
    if (g_stage != NULL) (void)hipFree(g_stage);
    g_stage = NULL;
    g_stage_bytes = 0;
    hipError_t e = hipMalloc(&g_stage, xb + yb);
    if (e != hipSuccess) {
      pthread_mutex_unlock(&g_stage_lock);
      return map_hip(e, "hipMalloc(x/y staging)");
    }
    g_stage_bytes = xb + yb;
  }
  float *dx = (float *)g_stage;
  float *dy = (float *)((uint8_t *)g_stage + xb);
  hipError_t e = hipMemcpy(dx, x, m * w->k * sizeof(float), hipMemcpyHostToDevice);
  if (e == hipSuccess) {
    st = launch(w, m, dx, dy, flags, NULL);
    if (st == PAI_OK) {
      e = hipMemcpy(y, dy, m * w->n * sizeof(float), hipMemcpyDeviceToHost);
      if (e != hipSuccess) st = map_hip(e, "hipMemcpy(y)");
    }
  } else {
    st = map_hip(e, "hipMemcpy(x)");
  }
  pthread_mutex_unlock(&g_stage_lock);
  return st;
}

pai_status_t pai_qdequant_f32(const pai_qmat_t *w, float *out, uint32_t flags) {
  if (w == NULL || out == NULL) return fail(PAI_ERR_INVALID_ARG, "NULL argument");
  pai_status_t st = ensure_ready();
  if (st != PAI_OK) return st;
  const uint64_t bytes = w->n * w->k * sizeof(float);
  float *dst = out;
  if ((flags & PAI_QGEMM_DEVICE_PTRS) == 0u) {
    HIP_TRY(hipMalloc((void **)&dst, bytes), "hipMalloc(dequant out)");
  } else if (((uintptr_t)out & 15u) != 0u) {
    return fail(PAI_ERR_INVALID_ARG, "out must be 16-byte aligned");
  }
  int le = paik_dequant(&w->view, dst, NULL);
  if (le == 0) le = (int)hipStreamSynchronize(NULL);
  if (le == 0 && dst != out) le = (int)hipMemcpy(out, dst, bytes, hipMemcpyDeviceToHost);
  if (dst != out) (void)hipFree(dst);
  return le == 0 ? PAI_OK : map_hip((hipError_t)le, "dequant");
}

/* ---------------------------------------------------------------------- */
/* The executor's GEMM branch (scheduler/scheduler.c:280-343)               */
/* ---------------------------------------------------------------------- */

pai_status_t pai_qgemm_shape_check(int is_gemv, uint32_t a_rank, const uint64_t *a,
                                   uint32_t b_rank, const uint64_t *b, uint32_t c_rank,
                                   const uint64_t *c, uint64_t w_n, uint64_t w_k,
                                   uint64_t *m_tokens) {
  if (a == NULL || b == NULL || c == NULL || m_tokens == NULL)
    return fail(PAI_ERR_INVALID_ARG, "NULL shape or output");
  if (is_gemv) {
    /* y[m] = A[m,k] * x[k], A the weight ([N][K] rows) */
    if (a_rank != 2u || b_rank != 1u || c_rank != 1u)
      return fail(PAI_ERR_MISMATCH, "GEMV ranks %u, %u, %u", a_rank, b_rank, c_rank);
    if (b[0] != a[1] || c[0] != a[0]) return fail(PAI_ERR_MISMATCH, "GEMV extents");
    if (a[0] != w_n || a[1] != w_k) return fail(PAI_ERR_MISMATCH, "GEMV matrix is not the weight");
    *m_tokens = 1u;
    return PAI_OK;
  }
  uint64_t m, k, n;
  if (a_rank == 1u) {
    /* row vector: y[n] = x[k] * W[k,n] */
    m = 1u;
    k = a[0];
    if (b_rank != 2u || b[0] != k) return fail(PAI_ERR_MISMATCH, "row-vector operand b");
    n = b[1];
    if (c_rank == 1u) {
      if (c[0] != n) return fail(PAI_ERR_MISMATCH, "row-vector output");
    } else if (c_rank == 2u) {
      if (c[0] != 1u || c[1] != n) return fail(PAI_ERR_MISMATCH, "row-vector output");
    } else {
      return fail(PAI_ERR_MISMATCH, "row-vector output rank %u", c_rank);
    }
  } else {
    /* C[m,n] = A[m,k] * B[k,n] */
    if (a_rank != 2u || b_rank != 2u) return fail(PAI_ERR_MISMATCH, "GEMM ranks");
    m = a[0];
    k = a[1];
    n = b[1];
    if (b[0] != k || c_rank != 2u || c[0] != m || c[1] != n)
      return fail(PAI_ERR_MISMATCH, "GEMM extents");
  }
  if (k != w_k || n != w_n) return fail(PAI_ERR_MISMATCH, "operand b is not the weight");
  *m_tokens = m;
  return PAI_OK;
}

pai_status_t pai_qgemm_run(const pai_qmat_t *w, int is_gemv, uint32_t a_rank,
                           const uint64_t *a_shape, uint32_t b_rank, const uint64_t *b_shape,
                           uint32_t c_rank, const uint64_t *c_shape, const float *act,
                           float *out, uint32_t flags) {
  if (w == NULL) return fail(PAI_ERR_INVALID_ARG, "NULL weight");
  uint64_t m = 0;
  const pai_status_t st = pai_qgemm_shape_check(is_gemv, a_rank, a_shape, b_rank, b_shape,
                                                c_rank, c_shape, w->n, w->k, &m);
  if (st != PAI_OK) return st;
  if (m == 0u) return fail(PAI_ERR_INVALID_ARG, "zero tokens");
  return pai_qgemm_f32(w, m, act, out, flags);
}

/* ---------------------------------------------------------------------- */
/* Registry descriptors                                                     */
/* ---------------------------------------------------------------------- */

/* caps: PAI_OP_CAP_CPU_REF (sdk/include/pai/op.h:59) | PAI_OP_CAP_GPU_HIP */
#define PAI_QGEMM_CAPS ((1u << 0) | PAI_OP_CAP_GPU_HIP)
#define PAI_QGEMM_REF ((pai_status_t(*)(void))pai_qgemm_ref_f32)
static const pai_hip_op_descriptor_t k_ops[] = {
    {"qgemm_q4_0_f32", 1u, 2u, 1u, 0, 0, PAI_QGEMM_CAPS, PAI_QGEMM_REF, 0, {0u, 0u}},
    {"qgemm_q8_0_f32", 1u, 2u, 1u, 0, 0, PAI_QGEMM_CAPS, PAI_QGEMM_REF, 0, {0u, 0u}},
    {"qgemm_q4_k_f32", 1u, 2u, 1u, 0, 0, PAI_QGEMM_CAPS, PAI_QGEMM_REF, 0, {0u, 0u}},
    {"qgemm_q6_k_f32", 1u, 2u, 1u, 0, 0, PAI_QGEMM_CAPS, PAI_QGEMM_REF, 0, {0u, 0u}},
    {"qgemm_w8_f32", 1u, 3u, 1u, 0, 0, PAI_QGEMM_CAPS, (pai_status_t(*)(void))pai_gemm_w8_ref_f32,
     0, {0u, 0u}},
    {"qgemm_w4_f32", 1u, 3u, 1u, 0, 0, PAI_QGEMM_CAPS, (pai_status_t(*)(void))pai_gemm_w4_ref_f32,
     0, {0u, 0u}},
};

const pai_hip_op_descriptor_t *pai_hip_op_descriptors(uint32_t *count) {
  if (count != NULL) *count = (uint32_t)(sizeof k_ops / sizeof k_ops[0]);
  return k_ops;
}

const char *pai_hip_op_name(uint32_t type) {
  switch (type) {
  case PAI_QTYPE_Q4_0: return k_ops[0].name;
  case PAI_QTYPE_Q8_0: return k_ops[1].name;
  case PAI_QTYPE_Q4_K: return k_ops[2].name;
  case PAI_QTYPE_Q6_K: return k_ops[3].name;
  default: return NULL;
  }
}

/* ---------------------------------------------------------------------- */
/* IR quantization tag                                                      */
/* ---------------------------------------------------------------------- */

/* (type, bits, signed, group, zero-point repr) of the four formats; the
 * scale repr is f16 (1) for all. */
static const struct {
  uint32_t type;
  uint8_t bits, is_signed, zp_repr;
  uint16_t group;
} k_tags[] = {
    {PAI_QTYPE_Q8_0, 8u, 1u, 0u, 32u},
    {PAI_QTYPE_Q4_0, 4u, 0u, 0u, 32u},
    {PAI_QTYPE_Q4_K, 4u, 0u, 1u, 256u},
    {PAI_QTYPE_Q6_K, 6u, 1u, 0u, 256u},
};

pai_status_t pai_hip_quant_tag(uint32_t type, pai_hip_ir_quant_t *out) {
  if (out == NULL) return fail(PAI_ERR_INVALID_ARG, "NULL argument");
  for (size_t i = 0; i < sizeof k_tags / sizeof k_tags[0]; ++i) {
    if (k_tags[i].type != type) continue;
    memset(out, 0, sizeof *out);
    out->present = 1u;
    out->bit_width = k_tags[i].bits;
    out->scale_repr = 1u; /* PAI_IR_QUANT_REPR_F16 */
    out->zero_point_repr = k_tags[i].zp_repr;
    out->is_signed = k_tags[i].is_signed;
    out->block_structure = (uint8_t)PAI_IR_QUANT_BLOCK_GGUF;
    out->group_size = k_tags[i].group;
    return PAI_OK;
  }
  return fail(PAI_ERR_UNSUPPORTED, "ggml type %u has no GGUF tag here", type);
}

uint32_t pai_hip_quant_type(const pai_hip_ir_quant_t *q) {
  if (q == NULL || q->present == 0u || q->block_structure != PAI_IR_QUANT_BLOCK_GGUF) return 0u;
  for (size_t i = 0; i < sizeof k_tags / sizeof k_tags[0]; ++i)
    if (k_tags[i].bits == q->bit_width && k_tags[i].group == q->group_size &&
        k_tags[i].is_signed == q->is_signed)
      return k_tags[i].type;
  return 0u;
}
