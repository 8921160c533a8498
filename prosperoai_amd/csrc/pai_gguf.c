/*
 * GGUF tensor directory and device-resident upload.
 *
 * The reference imports a GGUF model by dequantizing and transposing every
 * weight on the host (adapters/llama/llama.c:408-470, reader in
 * adapters/llama/gguf.c). The GPU kernels consume the packed blocks
 * themselves, so this reader keeps only the tensor directory: it walks the
 * header and the metadata key/value section, resolves "general.alignment",
 * records every tensor's name, extents, type and offset, and
 * pai_qmat_upload_gguf copies one tensor's bytes to the device as they are
 * in the file.
 *
 * Accepted input is the reference reader's (pai_gguf_open,
 * adapters/llama/gguf.c:128-245), decision for decision:
 *   - shorter than 24 bytes, wrong magic           -> PROTOCOL
 *   - version outside 1..3                          -> UNSUPPORTED
 *   - more than 1024 tensors                        -> UNSUPPORTED
 *   - counts, string lengths and extents are u64 in every version
 *   - a metadata value of unknown type, or any read past the end,
 *     a tensor name of length 0 or >= 128, n_dims outside 1..4, an
 *     extent above 2^26                             -> PROTOCOL
 *   - alignment: the first "general.alignment" key with an integer, bool
 *     or f32 value type, truncated to 32 bits (other value types leave the
 *     default 32); it must be a power of two <= 4096 -> else PROTOCOL
 *   - the data section starts at the aligned end of the tensor infos,
 *     which must not lie past the end of the file   -> else PROTOCOL.
 * Tensor offsets are checked when a tensor is used, as pai_gguf_dequant
 * checks them (adapters/llama/gguf.c:984-996). One difference: arrays
 * nested deeper than 64 levels are rejected as PROTOCOL instead of being
 * followed recursively without a limit.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "pai_hip.h"

__attribute__((visibility("hidden"))) pai_status_t pai__fail(pai_status_t st, const char *fmt,
                                                             ...);

#define GGUF_MAGIC 0x46554747u /* "GGUF" */
#define GGUF_MAX_VERSION 3u
#define GGUF_ALIGN_DEFAULT 32u
#define GGUF_MAX_ALIGN 4096u
#define GGUF_MAX_TENSORS 1024u
#define GGUF_MAX_EXTENT (1ull << 26)
#define GGUF_NAME_CAP 128u
#define GGUF_MAX_NEST 64

typedef struct gguf_entry {
  char name[GGUF_NAME_CAP];
  uint32_t type;
  uint32_t n_dims;
  uint64_t dims[4]; /* unused extents are 0 */
  uint64_t offset;  /* from the start of the data section */
} gguf_entry_t;

struct pai_gguf_dir {
  const uint8_t *data; /* the caller's buffer, not owned */
  uint64_t size;
  uint32_t version;
  uint32_t alignment;
  uint64_t data_start; /* from the start of the buffer */
  uint64_t count;
  gguf_entry_t *t;
};

typedef struct cursor {
  const uint8_t *p;
  uint64_t size, pos;
  int bad;
} cursor_t;

static int avail(cursor_t *c, uint64_t n) {
  if (c->bad || n > c->size - c->pos) c->bad = 1;
  return !c->bad;
}
static uint64_t rd_le(cursor_t *c, unsigned n) {
  uint64_t v = 0;
  if (!avail(c, n)) return 0;
  for (unsigned i = 0; i < n; ++i) v |= (uint64_t)c->p[c->pos + i] << (8u * i);
  c->pos += n;
  return v;
}
static uint32_t rd_u32(cursor_t *c) { return (uint32_t)rd_le(c, 4); }
static uint64_t rd_u64(cursor_t *c) { return rd_le(c, 8); }

/* A string: u64 length, then the bytes (returned in place, no NUL) */
static const uint8_t *rd_str(cursor_t *c, uint64_t *len) {
  *len = rd_u64(c);
  if (!avail(c, *len)) return NULL;
  const uint8_t *s = c->p + c->pos;
  c->pos += *len;
  return s;
}

/* Metadata value types (gguf_type in the GGUF specification) */
enum { V_U8, V_I8, V_U16, V_I16, V_U32, V_I32, V_F32, V_BOOL, V_STR, V_ARR, V_U64, V_I64, V_F64 };

/* Bytes of a fixed-size value; 0 for strings, arrays and unknown types */
static unsigned fixed_bytes(uint32_t vt) {
  switch (vt) {
  case V_U8: case V_I8: case V_BOOL: return 1;
  case V_U16: case V_I16: return 2;
  case V_U32: case V_I32: case V_F32: return 4;
  case V_U64: case V_I64: case V_F64: return 8;
  default: return 0;
  }
}

static void skip_value(cursor_t *c, uint32_t vt, int depth) {
  const unsigned fb = fixed_bytes(vt);
  if (fb != 0u) {
    if (avail(c, fb)) c->pos += fb;
  } else if (vt == V_STR) {
    uint64_t n;
    (void)rd_str(c, &n);
  } else if (vt == V_ARR && depth < GGUF_MAX_NEST) {
    const uint32_t et = rd_u32(c);
    const uint64_t n = rd_u64(c);
    const unsigned eb = fixed_bytes(et);
    if (c->bad) return;
    if (eb != 0u) {
      /* n fixed-size elements: one bounds check covers them all */
      if (n > (c->size - c->pos) / eb) c->bad = 1;
      else c->pos += n * eb;
    } else {
      for (uint64_t i = 0; i < n && !c->bad; ++i) skip_value(c, et, depth + 1);
    }
  } else {
    c->bad = 1; /* unknown type, or nesting too deep */
  }
}

void pai_gguf_dir_close(pai_gguf_dir_t *d) {
  if (d == NULL) return;
  free(d->t);
  free(d);
}

pai_status_t pai_gguf_dir_open(const void *data, uint64_t size, pai_gguf_dir_t **out) {
  if (data == NULL || out == NULL) return pai__fail(PAI_ERR_INVALID_ARG, "NULL argument");
  *out = NULL;
  if (size < 24u) return pai__fail(PAI_ERR_PROTOCOL, "GGUF file of %llu bytes",
                                   (unsigned long long)size);
  cursor_t c = {(const uint8_t *)data, size, 0, 0};
  if (rd_u32(&c) != GGUF_MAGIC) return pai__fail(PAI_ERR_PROTOCOL, "not a GGUF file");
  const uint32_t version = rd_u32(&c);
  if (version < 1u || version > GGUF_MAX_VERSION)
    return pai__fail(PAI_ERR_UNSUPPORTED, "GGUF version %u", version);
  const uint64_t nt = rd_u64(&c), nkv = rd_u64(&c);
  if (nt > GGUF_MAX_TENSORS)
    return pai__fail(PAI_ERR_UNSUPPORTED, "%llu tensors (at most %u)", (unsigned long long)nt,
                     GGUF_MAX_TENSORS);

  uint32_t alignment = GGUF_ALIGN_DEFAULT;
  int have_alignment = 0;
  for (uint64_t i = 0; i < nkv && !c.bad; ++i) {
    uint64_t klen;
    const uint8_t *key = rd_str(&c, &klen);
    const uint32_t vt = rd_u32(&c);
    if (c.bad) break;
    const unsigned fb = fixed_bytes(vt);
    if (!have_alignment && klen == 17u && memcmp(key, "general.alignment", 17) == 0) {
      have_alignment = 1; /* the first such key decides, whatever its type */
      if (fb != 0u && avail(&c, fb)) alignment = (uint32_t)rd_le(&c, fb);
      else skip_value(&c, vt, 0);
    } else {
      skip_value(&c, vt, 0);
    }
  }
  if (c.bad) return pai__fail(PAI_ERR_PROTOCOL, "malformed GGUF metadata");

  pai_gguf_dir_t *d = (pai_gguf_dir_t *)calloc(1, sizeof *d);
  gguf_entry_t *t = (gguf_entry_t *)calloc(nt ? nt : 1u, sizeof *t);
  if (d == NULL || t == NULL) {
    free(d);
    free(t);
    return pai__fail(PAI_ERR_NOMEM, "GGUF directory");
  }
  d->t = t;
  for (uint64_t i = 0; i < nt && !c.bad; ++i) {
    gguf_entry_t *e = &t[i];
    uint64_t nlen;
    const uint8_t *name = rd_str(&c, &nlen);
    if (c.bad || nlen == 0u || nlen >= GGUF_NAME_CAP) {
      c.bad = 1;
      break;
    }
    memcpy(e->name, name, nlen);
    e->n_dims = rd_u32(&c);
    if (e->n_dims == 0u || e->n_dims > 4u) c.bad = 1;
    for (uint32_t j = 0; j < e->n_dims && !c.bad; ++j) {
      e->dims[j] = rd_u64(&c);
      if (e->dims[j] > GGUF_MAX_EXTENT) c.bad = 1;
    }
    e->type = rd_u32(&c);
    e->offset = rd_u64(&c);
  }
  if (!c.bad && (alignment == 0u || (alignment & (alignment - 1u)) != 0u ||
                 alignment > GGUF_MAX_ALIGN))
    c.bad = 1;
  const uint64_t start = c.bad ? 0u : (c.pos + alignment - 1u) / alignment * alignment;
  if (c.bad || start > size) {
    pai_gguf_dir_close(d);
    return pai__fail(PAI_ERR_PROTOCOL, "malformed GGUF tensor directory");
  }
  d->data = (const uint8_t *)data;
  d->size = size;
  d->version = version;
  d->alignment = alignment;
  d->data_start = start;
  d->count = nt;
  *out = d;
  return PAI_OK;
}

uint64_t pai_gguf_dir_count(const pai_gguf_dir_t *d) { return d == NULL ? 0u : d->count; }

pai_status_t pai_gguf_dir_layout(const pai_gguf_dir_t *d, uint32_t *version,
                                 uint32_t *alignment, uint64_t *data_start) {
  if (d == NULL) return pai__fail(PAI_ERR_INVALID_ARG, "NULL directory");
  if (version != NULL) *version = d->version;
  if (alignment != NULL) *alignment = d->alignment;
  if (data_start != NULL) *data_start = d->data_start;
  return PAI_OK;
}

pai_status_t pai_gguf_dir_tensor(const pai_gguf_dir_t *d, uint64_t index, const char **name,
                                 uint32_t *type, uint32_t *n_dims, uint64_t *dims,
                                 uint64_t *offset) {
  if (d == NULL) return pai__fail(PAI_ERR_INVALID_ARG, "NULL directory");
  if (index >= d->count)
    return pai__fail(PAI_ERR_INVALID_ARG, "tensor index %llu of %llu",
                     (unsigned long long)index, (unsigned long long)d->count);
  const gguf_entry_t *e = &d->t[index];
  if (name != NULL) *name = e->name;
  if (type != NULL) *type = e->type;
  if (n_dims != NULL) *n_dims = e->n_dims;
  if (dims != NULL) memcpy(dims, e->dims, sizeof e->dims);
  if (offset != NULL) *offset = e->offset;
  return PAI_OK;
}

pai_status_t pai_gguf_dir_find(const pai_gguf_dir_t *d, const char *name, uint64_t *index) {
  if (d == NULL || name == NULL || index == NULL)
    return pai__fail(PAI_ERR_INVALID_ARG, "NULL argument");
  for (uint64_t i = 0; i < d->count; ++i)
    if (strcmp(d->t[i].name, name) == 0) {
      *index = i;
      return PAI_OK;
    }
  return pai__fail(PAI_ERR_MISMATCH, "no tensor named %s", name);
}

pai_status_t pai_gguf_dir_blocks(const pai_gguf_dir_t *d, uint64_t index, const void **blocks,
                                 uint64_t *nbytes) {
  if (d == NULL || blocks == NULL || nbytes == NULL)
    return pai__fail(PAI_ERR_INVALID_ARG, "NULL argument");
  *blocks = NULL;
  *nbytes = 0;
  if (index >= d->count)
    return pai__fail(PAI_ERR_INVALID_ARG, "tensor index %llu of %llu",
                     (unsigned long long)index, (unsigned long long)d->count);
  const gguf_entry_t *e = &d->t[index];
  uint64_t numel = 1u; /* wraps like pai_gguf_tensor_numel (gguf.c:549-560) */
  for (uint32_t j = 0; j < e->n_dims; ++j) numel *= e->dims[j];
  if (numel == 0u) return pai__fail(PAI_ERR_PROTOCOL, "tensor %s has no elements", e->name);
  const uint64_t bytes = pai_qtype_bytes(e->type, numel);
  if (bytes == 0u)
    return pai__fail(PAI_ERR_UNSUPPORTED,
                     "tensor %s: ggml type %u is not Q4_0/Q8_0/Q4_K/Q6_K, or %llu elements "
                     "are not whole blocks", e->name, e->type, (unsigned long long)numel);
  const uint64_t region = d->size - d->data_start;
  if (e->offset > region || bytes > region - e->offset)
    return pai__fail(PAI_ERR_PROTOCOL, "tensor %s: bytes fall outside the file", e->name);
  *blocks = d->data + d->data_start + e->offset;
  *nbytes = bytes;
  return PAI_OK;
}

pai_status_t pai_qmat_upload_gguf(pai_qmat_t **out, const pai_gguf_dir_t *d, const char *name) {
  if (out == NULL || d == NULL || name == NULL)
    return pai__fail(PAI_ERR_INVALID_ARG, "NULL argument");
  *out = NULL;
  uint64_t i;
  pai_status_t st = pai_gguf_dir_find(d, name, &i);
  if (st != PAI_OK) return st;
  const void *blocks;
  uint64_t nbytes;
  st = pai_gguf_dir_blocks(d, i, &blocks, &nbytes);
  if (st != PAI_OK) return st;
  const gguf_entry_t *e = &d->t[i];
  if (e->n_dims != 2u)
    return pai__fail(PAI_ERR_MISMATCH, "tensor %s has %u dims, a weight matrix has 2", name,
                     e->n_dims);
  /* extents are innermost first: dims[0] = K (row length), dims[1] = N */
  return pai_qmat_upload(out, e->type, e->dims[1], e->dims[0], blocks, nbytes);
}
