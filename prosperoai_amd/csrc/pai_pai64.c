/*
 * The `.pai` container with 64-bit offsets and sizes (version 2) and the
 * uncapped tokenizer blob: writer, reader (versions 1 and 2), manifest
 * codec and the upload of GGUF-block tensors. See include/pai_pai64.h for
 * the format. Host C11.
 */
#define _GNU_SOURCE
#include "pai_pai64.h"

#include <fcntl.h>
#include <pthread.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

pai_status_t pai__fail(pai_status_t st, const char *fmt, ...);

/* ------------------------------------------------------------------ */
/* Little-endian fields and the checksum                               */
/* ------------------------------------------------------------------ */

static uint32_t le32(const uint8_t *p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
static uint64_t le64(const uint8_t *p) { return (uint64_t)le32(p) | ((uint64_t)le32(p + 4) << 32); }
static void put32(uint8_t *p, uint32_t v) {
  for (int i = 0; i < 4; ++i) p[i] = (uint8_t)(v >> (8 * i));
}
static void put64(uint8_t *p, uint64_t v) {
  for (int i = 0; i < 8; ++i) p[i] = (uint8_t)(v >> (8 * i));
}

/* Reflected CRC-32, polynomial 0xEDB88320, eight table lookups per 8
 * bytes (slicing-by-8). */
static uint32_t g_crc[8][256];
static pthread_once_t g_crc_once = PTHREAD_ONCE_INIT;
static void crc_tables(void) {
  for (uint32_t i = 0; i < 256; ++i) {
    uint32_t c = i;
    for (int k = 0; k < 8; ++k) c = (c & 1u) ? 0xEDB88320u ^ (c >> 1) : c >> 1;
    g_crc[0][i] = c;
  }
  for (uint32_t i = 0; i < 256; ++i)
    for (int t = 1; t < 8; ++t) g_crc[t][i] = (g_crc[t - 1][i] >> 8) ^ g_crc[0][g_crc[t - 1][i] & 0xFFu];
}
static uint32_t crc_run(uint32_t c, const uint8_t *p, uint64_t n) {
  while (n >= 8u) {
    const uint32_t a = c ^ le32(p), b = le32(p + 4);
    c = g_crc[7][a & 0xFFu] ^ g_crc[6][(a >> 8) & 0xFFu] ^ g_crc[5][(a >> 16) & 0xFFu] ^
        g_crc[4][a >> 24] ^ g_crc[3][b & 0xFFu] ^ g_crc[2][(b >> 8) & 0xFFu] ^
        g_crc[1][(b >> 16) & 0xFFu] ^ g_crc[0][b >> 24];
    p += 8;
    n -= 8u;
  }
  while (n-- > 0u) c = g_crc[0][(c ^ *p++) & 0xFFu] ^ (c >> 8);
  return c;
}
uint32_t pai64_crc32(uint32_t crc, const void *data, uint64_t nbytes) {
  pthread_once(&g_crc_once, crc_tables);
  if (data == NULL) return crc;
  return crc_run(crc ^ 0xFFFFFFFFu, (const uint8_t *)data, nbytes) ^ 0xFFFFFFFFu;
}

/* ------------------------------------------------------------------ */
/* Writer                                                              */
/* ------------------------------------------------------------------ */

static uint64_t align_up(uint64_t v) { return (v + PAI64_ALIGN - 1u) & ~(uint64_t)(PAI64_ALIGN - 1u); }

static int write_all(int fd, const void *p, uint64_t n, uint64_t off) {
  const uint8_t *b = (const uint8_t *)p;
  while (n > 0u) {
    const size_t chunk = n > (1u << 30) ? (1u << 30) : (size_t)n;
    const ssize_t w = pwrite(fd, b, chunk, (off_t)off);
    if (w <= 0) return -1;
    b += w;
    off += (uint64_t)w;
    n -= (uint64_t)w;
  }
  return 0;
}

pai_status_t pai64_write_file(const char *path, const pai64_section_in_t *sec, uint32_t count,
                              uint64_t *out_nbytes) {
  if (path == NULL || sec == NULL || count == 0u || count > PAI64_MAX_SECTIONS)
    return pai__fail(PAI_ERR_INVALID_ARG, "container: path, sections, 1..%u sections",
                     PAI64_MAX_SECTIONS);
  uint32_t seen = 0;
  for (uint32_t i = 0; i < count; ++i) {
    const uint32_t t = sec[i].type;
    if (t == 0u || t > PAI64_SEC_PROFILE || (seen & (1u << t)) != 0u)
      return pai__fail(PAI_ERR_INVALID_ARG, "container: section %u type %u", i, t);
    seen |= 1u << t;
    if (sec[i].flags != 0u && (t != PAI64_SEC_WEIGHTS || sec[i].flags != PAI64_SEC_FLAG_COMPRESSED))
      return pai__fail(PAI_ERR_INVALID_ARG, "container: section %u flags %#x", i, sec[i].flags);
  }
  /* layout */
  uint8_t head[PAI64_HEADER_BYTES + PAI64_MAX_SECTIONS * PAI64_ENTRY_BYTES];
  const uint64_t table_end = PAI64_HEADER_BYTES + (uint64_t)count * PAI64_ENTRY_BYTES;
  uint64_t cursor = align_up(table_end);
  memset(head, 0, sizeof head);
  for (uint32_t i = 0; i < count; ++i) {
    uint8_t *e = head + PAI64_HEADER_BYTES + i * PAI64_ENTRY_BYTES;
    const int has_crc = sec[i].data != NULL || sec[i].size == 0u;
    const uint32_t crc = has_crc ? pai64_crc32(0u, sec[i].data, sec[i].size) : 0u;
    put32(e, sec[i].type);
    put32(e + 4, sec[i].flags | (has_crc ? PAI64_SEC_FLAG_CRC : 0u));
    put64(e + 8, cursor);
    put64(e + 16, sec[i].size);
    put32(e + 24, crc);
    cursor = align_up(cursor + sec[i].size);
  }
  /* the last section ends the file (no trailing padding) */
  uint64_t total = PAI64_HEADER_BYTES;
  for (uint32_t i = 0; i < count; ++i) {
    const uint8_t *e = head + PAI64_HEADER_BYTES + i * PAI64_ENTRY_BYTES;
    const uint64_t end = le64(e + 8) + le64(e + 16);
    if (end > total) total = end;
  }
  if (total < table_end) total = table_end;
  put32(head, PAI64_MAGIC);
  head[4] = (uint8_t)PAI64_VERSION;
  put32(head + 8, count);
  put64(head + 16, total);
  uint32_t hcrc = pai64_crc32(0u, head, 12u);
  hcrc = pai64_crc32(hcrc, head + 16, table_end - 16u);
  put32(head + 12, hcrc);

  const int fd = open(path, O_WRONLY | O_CREAT | O_TRUNC, 0644);
  if (fd < 0) return pai__fail(PAI_ERR_IO, "container: cannot create %s", path);
  int bad = ftruncate(fd, (off_t)total) != 0; /* holes and padding read as zeros */
  if (!bad) bad = write_all(fd, head, table_end, 0u) != 0;
  for (uint32_t i = 0; i < count && !bad; ++i) {
    const uint8_t *e = head + PAI64_HEADER_BYTES + i * PAI64_ENTRY_BYTES;
    if (sec[i].data != NULL && sec[i].size > 0u)
      bad = write_all(fd, sec[i].data, sec[i].size, le64(e + 8)) != 0;
  }
  if (close(fd) != 0) bad = 1;
  if (bad) return pai__fail(PAI_ERR_IO, "container: write to %s failed", path);
  if (out_nbytes != NULL) *out_nbytes = total;
  return PAI_OK;
}

/* ------------------------------------------------------------------ */
/* Reader                                                              */
/* ------------------------------------------------------------------ */

#define PROTO(...) pai__fail(PAI_ERR_PROTOCOL, __VA_ARGS__)

/* The per-section rules shared by both versions (pai/pai.c:182-226). */
static pai_status_t check_sections(const pai64_container_t *c, uint64_t table_end) {
  for (uint32_t i = 0; i < c->num_sections; ++i) {
    const pai64_section_t *s = &c->sections[i];
    const uint32_t allowed = c->version == 1u ? 0u : PAI64_SEC_FLAG_CRC;
    if (s->type == 0u || s->type > PAI64_SEC_PROFILE) return PROTO("section type %u", s->type);
    const uint32_t fl = s->flags & ~allowed;
    if (fl != 0u && (s->type != PAI64_SEC_WEIGHTS || (fl & ~PAI64_SEC_FLAG_COMPRESSED) != 0u))
      return PROTO("section %u flags %#x", i, s->flags);
    if (s->offset < table_end) return PROTO("section %u overlaps the table", i);
    if (s->offset > c->nbytes || s->size > c->nbytes - s->offset)
      return PROTO("section %u leaves the file", i);
    if (c->version == 2u && (s->offset % PAI64_ALIGN) != 0u)
      return PROTO("section %u offset not %u-aligned", i, PAI64_ALIGN);
    for (uint32_t k = 0; k < i; ++k) {
      const pai64_section_t *p = &c->sections[k];
      if (p->type == s->type) return PROTO("section type %u repeated", s->type);
      if (s->offset < p->offset + p->size && p->offset < s->offset + s->size)
        return PROTO("sections %u and %u overlap", k, i);
    }
  }
  return PAI_OK;
}

pai_status_t pai64_open(const uint8_t *data, uint64_t nbytes, pai64_container_t *out) {
  if (data == NULL || out == NULL) return pai__fail(PAI_ERR_INVALID_ARG, "NULL argument");
  if (nbytes < 16u) return pai__fail(PAI_ERR_INVALID_ARG, "container of %llu bytes",
                                     (unsigned long long)nbytes);
  if (le32(data) != PAI64_MAGIC) return PROTO("not a .pai container");
  const uint32_t version = (uint32_t)data[4] | ((uint32_t)data[5] << 8);
  if ((version != 1u && version != 2u) || data[6] != 0u || data[7] != 0u)
    return PROTO(".pai version %u", version);
  const uint32_t n = le32(data + 8);
  if (n == 0u || n > PAI64_MAX_SECTIONS) return PROTO("%u sections", n);
  pai64_container_t c;
  memset(&c, 0, sizeof c);
  c.version = version;
  c.num_sections = n;
  c.data = data;
  c.nbytes = nbytes;
  uint64_t table_end;
  if (version == 1u) {
    table_end = 16u + 16u * (uint64_t)n;
    if (table_end > nbytes) return PROTO("truncated section table");
    for (uint32_t i = 0; i < n; ++i) {
      const uint8_t *e = data + 16 + 16 * i;
      c.sections[i].type = le32(e);
      c.sections[i].flags = le32(e + 4);
      c.sections[i].offset = le32(e + 8);
      c.sections[i].size = le32(e + 12);
    }
    pai_status_t st = check_sections(&c, table_end);
    if (st != PAI_OK) return st;
    /* version 1: one CRC over [0,12) and everything from byte 16 */
    uint32_t crc = pai64_crc32(0u, data, 12u);
    crc = pai64_crc32(crc, data + 16, nbytes - 16u);
    if (crc != le32(data + 12)) return PROTO("container checksum mismatch");
  } else {
    table_end = PAI64_HEADER_BYTES + PAI64_ENTRY_BYTES * (uint64_t)n;
    if (table_end > nbytes) return PROTO("truncated section table");
    uint32_t crc = pai64_crc32(0u, data, 12u);
    crc = pai64_crc32(crc, data + 16, table_end - 16u);
    if (crc != le32(data + 12)) return PROTO("header checksum mismatch");
    if (le64(data + 16) != nbytes) return PROTO("total size field %llu, file %llu bytes",
                                                (unsigned long long)le64(data + 16),
                                                (unsigned long long)nbytes);
    if (le64(data + 24) != 0u) return PROTO("reserved header field set");
    for (uint32_t i = 0; i < n; ++i) {
      const uint8_t *e = data + PAI64_HEADER_BYTES + PAI64_ENTRY_BYTES * i;
      c.sections[i].type = le32(e);
      c.sections[i].flags = le32(e + 4);
      c.sections[i].offset = le64(e + 8);
      c.sections[i].size = le64(e + 16);
      c.sections[i].crc = le32(e + 24);
      if (le32(e + 28) != 0u) return PROTO("reserved entry field set");
    }
    pai_status_t st = check_sections(&c, table_end);
    if (st != PAI_OK) return st;
  }
  *out = c;
  return PAI_OK;
}

static const pai64_section_t *find(const pai64_container_t *c, uint32_t type) {
  if (c == NULL) return NULL;
  for (uint32_t i = 0; i < c->num_sections; ++i)
    if (c->sections[i].type == type) return &c->sections[i];
  return NULL;
}

const uint8_t *pai64_section(const pai64_container_t *c, uint32_t type, uint64_t *out_size) {
  const pai64_section_t *s = find(c, type);
  if (out_size != NULL) *out_size = s != NULL ? s->size : 0u;
  return s != NULL ? c->data + s->offset : NULL;
}

pai_status_t pai64_verify_section(const pai64_container_t *c, uint32_t type) {
  const pai64_section_t *s = find(c, type);
  if (s == NULL) return pai__fail(PAI_ERR_MISMATCH, "no section of type %u", type);
  if (c->version != 2u || (s->flags & PAI64_SEC_FLAG_CRC) == 0u)
    return pai__fail(PAI_ERR_UNSUPPORTED, "section %u has no recorded checksum", type);
  if (pai64_crc32(0u, c->data + s->offset, s->size) != s->crc)
    return PROTO("section %u checksum mismatch", type);
  return PAI_OK;
}

pai_status_t pai64_map_file(const char *path, const uint8_t **data, uint64_t *nbytes) {
  if (path == NULL || data == NULL || nbytes == NULL)
    return pai__fail(PAI_ERR_INVALID_ARG, "NULL argument");
  const int fd = open(path, O_RDONLY);
  if (fd < 0) return pai__fail(PAI_ERR_IO, "cannot open %s", path);
  struct stat sb;
  if (fstat(fd, &sb) != 0 || sb.st_size <= 0) {
    close(fd);
    return pai__fail(PAI_ERR_IO, "cannot size %s", path);
  }
  void *p = mmap(NULL, (size_t)sb.st_size, PROT_READ, MAP_SHARED, fd, 0);
  close(fd);
  if (p == MAP_FAILED) return pai__fail(PAI_ERR_IO, "cannot map %s", path);
  *data = (const uint8_t *)p;
  *nbytes = (uint64_t)sb.st_size;
  return PAI_OK;
}

pai_status_t pai64_unmap_file(const uint8_t *data, uint64_t nbytes) {
  if (data == NULL) return PAI_OK;
  return munmap((void *)data, (size_t)nbytes) == 0 ? PAI_OK
                                                   : pai__fail(PAI_ERR_IO, "munmap failed");
}

/* ------------------------------------------------------------------ */
/* Manifest (the version-1 entry layout, pai/pai.h:16-18)              */
/* ------------------------------------------------------------------ */

#define ENTRY_FIXED (4u + 4u + 6u * 8u + 8u + 8u) /* after name_len + name */
#define DTYPE_COUNT 9u                            /* sdk/include/pai/dtype.h:12-23 */

uint64_t pai64_manifest_bytes(const pai64_tensor_t *t, uint32_t count) {
  if (t == NULL || count == 0u) return 0u;
  uint64_t total = 4u;
  for (uint32_t i = 0; i < count; ++i) {
    const size_t len = strnlen(t[i].name, sizeof t[i].name);
    if (len == 0u || len >= sizeof t[i].name) return 0u;
    total += 2u + len + ENTRY_FIXED;
  }
  return total;
}

pai_status_t pai64_manifest_encode(const pai64_tensor_t *t, uint32_t count, uint8_t *out,
                                   uint64_t cap, uint64_t *out_nbytes) {
  const uint64_t total = pai64_manifest_bytes(t, count);
  if (out == NULL || out_nbytes == NULL || total == 0u || total > cap)
    return pai__fail(PAI_ERR_INVALID_ARG, "manifest: entries, names or room");
  for (uint32_t i = 0; i < count; ++i)
    if (t[i].gguf_type > 0xFFFFu || t[i].rank == 0u || t[i].rank > 6u)
      return pai__fail(PAI_ERR_INVALID_ARG, "manifest entry %u", i);
  uint8_t *p = out;
  put32(p, count);
  p += 4;
  for (uint32_t i = 0; i < count; ++i) {
    const uint32_t len = (uint32_t)strlen(t[i].name);
    p[0] = (uint8_t)len;
    p[1] = (uint8_t)(len >> 8);
    memcpy(p + 2, t[i].name, len);
    p += 2u + len;
    put32(p, t[i].value_id);
    p[4] = (uint8_t)t[i].dtype;
    p[5] = (uint8_t)t[i].rank;
    p[6] = (uint8_t)t[i].gguf_type;
    p[7] = (uint8_t)(t[i].gguf_type >> 8);
    p += 8;
    for (int d = 0; d < 6; ++d, p += 8) put64(p, t[i].shape[d]);
    put64(p, t[i].offset);
    put64(p + 8, t[i].size_bytes);
    p += 16;
  }
  *out_nbytes = total;
  return PAI_OK;
}

pai_status_t pai64_manifest_decode(const uint8_t *data, uint64_t size, pai64_tensor_t *out,
                                   uint32_t max_tensors, uint32_t *out_count) {
  if (data == NULL || size < 4u || out == NULL || max_tensors == 0u || out_count == NULL)
    return pai__fail(PAI_ERR_INVALID_ARG, "manifest: NULL argument or size");
  const uint32_t count = le32(data);
  if (count == 0u || count > max_tensors) return PROTO("manifest of %u entries", count);
  uint64_t p = 4u;
  for (uint32_t i = 0; i < count; ++i) {
    pai64_tensor_t *t = &out[i];
    if (p + 2u > size) return PROTO("manifest entry %u truncated", i);
    const uint32_t len = (uint32_t)data[p] | ((uint32_t)data[p + 1] << 8);
    p += 2u;
    if (len == 0u || len >= sizeof t->name || p + len + ENTRY_FIXED > size)
      return PROTO("manifest entry %u name or size", i);
    memset(t, 0, sizeof *t);
    memcpy(t->name, data + p, len);
    p += len;
    t->value_id = le32(data + p);
    t->dtype = data[p + 4];
    t->rank = data[p + 5];
    t->gguf_type = (uint32_t)data[p + 6] | ((uint32_t)data[p + 7] << 8);
    p += 8u;
    if (t->rank == 0u || t->rank > 6u || t->dtype >= DTYPE_COUNT)
      return PROTO("manifest entry %u rank %u dtype %u", i, t->rank, t->dtype);
    for (int d = 0; d < 6; ++d, p += 8u) t->shape[d] = le64(data + p);
    t->offset = le64(data + p);
    t->size_bytes = le64(data + p + 8);
    p += 16u;
    if (t->size_bytes == 0u) return PROTO("manifest entry %u of 0 bytes", i);
  }
  *out_count = count;
  return PAI_OK;
}

pai_status_t pai64_qmat_upload(const pai64_container_t *c, const pai64_tensor_t *t,
                               pai_qmat_t **out) {
  if (c == NULL || t == NULL || out == NULL) return pai__fail(PAI_ERR_INVALID_ARG, "NULL argument");
  if (t->gguf_type == 0u || pai_hip_op_name(t->gguf_type) == NULL)
    return pai__fail(PAI_ERR_UNSUPPORTED, "tensor %s is not GGUF blocks of a supported type",
                     t->name);
  if (t->rank != 2u) return pai__fail(PAI_ERR_MISMATCH, "tensor %s of rank %u", t->name, t->rank);
  uint64_t wsize = 0;
  const uint8_t *w = pai64_section(c, PAI64_SEC_WEIGHTS, &wsize);
  if (w == NULL) return pai__fail(PAI_ERR_MISMATCH, "no WEIGHTS section");
  if (t->offset > wsize || t->size_bytes > wsize - t->offset)
    return pai__fail(PAI_ERR_MISMATCH, "tensor %s leaves the WEIGHTS section", t->name);
  /* logical [K][N]; the blocks are the native [N][K/blk] rows */
  return pai_qmat_upload(out, t->gguf_type, t->shape[1], t->shape[0], w + t->offset,
                         t->size_bytes);
}

/* ------------------------------------------------------------------ */
/* Tokenizer blob                                                      */
/* ------------------------------------------------------------------ */

uint64_t pai64_tok_bytes(const char *const *texts, uint32_t ntok, uint32_t nmerge) {
  if ((texts == NULL && ntok > 0u) || ntok > PAI64_TOK_MAX || nmerge > PAI64_TOK_MAX) return 0u;
  uint64_t total = 16u + 12u * (uint64_t)nmerge;
  for (uint32_t i = 0; i < ntok; ++i) {
    const size_t len = texts[i] != NULL ? strnlen(texts[i], 256u) : 0u;
    if (len == 0u || len > 255u) return 0u;
    total += 5u + len;
  }
  return total;
}

pai_status_t pai64_tok_encode(const uint32_t *ids, const char *const *texts, uint32_t ntok,
                              const uint32_t *merges, uint32_t nmerge, uint8_t *out,
                              uint64_t cap, uint64_t *out_nbytes) {
  const uint64_t total = pai64_tok_bytes(texts, ntok, nmerge);
  if ((ids == NULL && ntok > 0u) || (merges == NULL && nmerge > 0u) || out == NULL ||
      out_nbytes == NULL || total == 0u || total > cap)
    return pai__fail(PAI_ERR_INVALID_ARG, "tokenizer: arguments, texts or room");
  uint8_t *p = out;
  put32(p, PAI64_TOK_MAGIC);
  put32(p + 4, PAI64_TOK_VERSION);
  put32(p + 8, ntok);
  put32(p + 12, nmerge);
  p += 16;
  for (uint32_t i = 0; i < ntok; ++i) {
    const uint32_t len = (uint32_t)strlen(texts[i]);
    put32(p, ids[i]);
    p[4] = (uint8_t)len;
    memcpy(p + 5, texts[i], len);
    p += 5u + len;
  }
  for (uint32_t i = 0; i < nmerge; ++i, p += 12)
    for (int k = 0; k < 3; ++k) put32(p + 4 * k, merges[3u * i + (uint32_t)k]);
  *out_nbytes = total;
  return PAI_OK;
}

pai_status_t pai64_tok_index(const uint8_t *blob, uint64_t nbytes, uint32_t *out_ntok,
                             uint32_t *out_nmerge, uint64_t *entry_offsets, uint32_t cap,
                             uint64_t *merges_offset) {
  if (blob == NULL || out_ntok == NULL || out_nmerge == NULL || nbytes < 16u)
    return pai__fail(PAI_ERR_INVALID_ARG, "tokenizer: NULL argument or size");
  const uint32_t version = le32(blob + 4);
  if (le32(blob) != PAI64_TOK_MAGIC || (version != 1u && version != 2u))
    return PROTO("not a tokenizer blob (version %u)", version);
  const uint32_t ntok = le32(blob + 8), nmerge = le32(blob + 12);
  /* models/tokenizer.h:23-24 for version 1 */
  const uint32_t max_tok = version == 1u ? 65536u : PAI64_TOK_MAX;
  const uint32_t max_merge = version == 1u ? 8192u : PAI64_TOK_MAX;
  if (ntok > max_tok || nmerge > max_merge)
    return PROTO("tokenizer of %u tokens, %u merges (version %u)", ntok, nmerge, version);
  if (entry_offsets != NULL && cap < ntok)
    return pai__fail(PAI_ERR_INVALID_ARG, "index room for %u of %u tokens", cap, ntok);
  uint64_t p = 16u;
  for (uint32_t i = 0; i < ntok; ++i) {
    if (p + 5u > nbytes) return PROTO("token %u truncated", i);
    const uint32_t len = blob[p + 4];
    if (len == 0u || p + 5u + len > nbytes) return PROTO("token %u text", i);
    if (entry_offsets != NULL) entry_offsets[i] = p;
    p += 5u + len;
  }
  if (p + 12u * (uint64_t)nmerge > nbytes) return PROTO("merges truncated");
  if (merges_offset != NULL) *merges_offset = p;
  *out_ntok = ntok;
  *out_nmerge = nmerge;
  return PAI_OK;
}
