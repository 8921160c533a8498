/*
 * pai_pai64 — the `.pai` model container with 64-bit section offsets and
 * sizes (version 2), and a tokenizer blob without the 65 536-token cap,
 * so that a Llama-3-8B-size model (4.9 GB of packed weights, 128 256
 * tokens, 280 k merges) travels through the reference's own format.
 *
 * Version 1 (pai/pai.h:1-18) keeps every offset and size in 32 bits and
 * reads whole files into one buffer (pai_pai_read_file caps them at 4 GiB;
 * adapters/llama/llama.c:279 at 2 GiB); its tokenizer rejects more than
 * 65 536 tokens and 8 192 merges (models/tokenizer.h:23-24). Version 2
 * keeps the section types, the validation rules, the CRC-32 and the
 * manifest entry layout of version 1, and changes:
 *
 *   header  32 bytes: u32 magic "PAIC", u16 version 2, u16 flags 0,
 *           u32 num_sections, u32 crc32 of bytes [0,12) and [16, 32 +
 *           32 num_sections) (header tail and section table), u64 total
 *           file bytes, u64 reserved 0
 *   table   num_sections x 32 bytes: u32 type, u32 flags, u64 offset, u64
 *           size, u32 crc32 of the payload, u32 reserved 0
 *   payload each section at a 256-byte-aligned offset (direct uploads
 *           from a mapped file), zero padding between sections
 *
 * Payload CRCs are checked on request (pai64_verify_section), not on
 * open, so that opening a multi-gigabyte file maps it without reading it.
 * A section flag bit says whether its CRC was recorded (a section written
 * as a hole of zeros has none).
 *
 * The manifest payload keeps the version-1 entry layout (pai/pai.h:16-18)
 * and uses its reserved u16 for the GGUF block type of a tensor stored as
 * native blocks (0 for f32 or v0 data), with a u32 entry count without the
 * 512-tensor cap. Readers of version 1 are unchanged by this: the reserved
 * field is written as 0 there.
 *
 * All integers little-endian. Host code (C11); only pai64_qmat_upload
 * touches the GPU.
 */
#ifndef PAI_PAI64_H
#define PAI_PAI64_H

#include <stdint.h>

#include "pai_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

#define PAI64_MAGIC 0x43494150u /* "PAIC", as pai/pai.h:34 */
#define PAI64_VERSION 2u
#define PAI64_HEADER_BYTES 32u
#define PAI64_ENTRY_BYTES 32u
#define PAI64_MAX_SECTIONS 8u /* pai/pai.h:37 */
#define PAI64_ALIGN 256u
/* section types: pai_pai_section_type_t (pai/pai.h:41-49), META = 1 ..
 * PROFILE = 7 */
#define PAI64_SEC_META 1u
#define PAI64_SEC_MANIFEST 2u
#define PAI64_SEC_WEIGHTS 3u
#define PAI64_SEC_IR 4u
#define PAI64_SEC_TOKENIZER 5u
#define PAI64_SEC_TARGET 6u
#define PAI64_SEC_PROFILE 7u
/* section flags: the WEIGHTS-only compressed bit of version 1
 * (pai/pai.h:95), and the recorded-CRC bit of version 2 */
#define PAI64_SEC_FLAG_COMPRESSED 1u
#define PAI64_SEC_FLAG_CRC (1u << 31)

typedef struct pai64_section {
  uint32_t type;
  uint32_t flags;
  uint64_t offset; /* from the file start */
  uint64_t size;
  uint32_t crc; /* version 2 with PAI64_SEC_FLAG_CRC */
} pai64_section_t;

/* Parsed view of a version-1 or version-2 container; does not own data. */
typedef struct pai64_container {
  uint32_t version;
  uint32_t num_sections;
  pai64_section_t sections[PAI64_MAX_SECTIONS];
  const uint8_t *data;
  uint64_t nbytes;
} pai64_container_t;

/* A section to write: `size` bytes from `data`, or, with data NULL, a
 * hole of `size` zero bytes left unwritten in the file (no CRC). `flags`
 * takes PAI64_SEC_FLAG_COMPRESSED on WEIGHTS only. */
typedef struct pai64_section_in {
  uint32_t type;
  uint32_t flags;
  const void *data;
  uint64_t size;
} pai64_section_in_t;

/* CRC-32 (IEEE 802.3, reflected, the container's checksum,
 * protocol/crc32.c): pai64_crc32(0, p, n) is the checksum of n bytes, and
 * passing a previous result continues it. */
uint32_t pai64_crc32(uint32_t crc, const void *data, uint64_t nbytes);

/* Write a version-2 container to `path`: sections in the given order,
 * each at the next 256-byte boundary. INVALID_ARG for 0 or more than
 * PAI64_MAX_SECTIONS sections, a type outside 1..7, a repeated type,
 * flags other than COMPRESSED on WEIGHTS, or data NULL with size 0 only
 * where a section is empty; IO on a write failure. */
pai_status_t pai64_write_file(const char *path, const pai64_section_in_t *sections,
                              uint32_t count, uint64_t *out_nbytes);

/* Validate and view a container held in memory (a mapped file): version 2
 * by the rules above, version 1 by pai_pai_open's (pai/pai.c:147-255, its
 * whole-file CRC included). PROTOCOL for any violation: bad magic,
 * version or header flags, 0 or too many sections, a table or header
 * CRC mismatch, a section type outside 1..7 or repeated, flags other
 * than COMPRESSED on WEIGHTS (and CRC in version 2), a payload that
 * overlaps the header, the table or another payload, leaves the file, or
 * (version 2) is not 256-byte aligned, or a total-size field that differs
 * from nbytes. INVALID_ARG for NULL. */
pai_status_t pai64_open(const uint8_t *data, uint64_t nbytes, pai64_container_t *out);

/* Payload of the section of `type` (NULL when absent; size in
 * *out_size, 0 when absent), as pai_pai_section. */
const uint8_t *pai64_section(const pai64_container_t *c, uint32_t type, uint64_t *out_size);

/* Check a version-2 section's payload against its recorded CRC: OK,
 * PROTOCOL on a mismatch, UNSUPPORTED when none was recorded (a hole, or
 * a version-1 container, whose open already checked the whole file),
 * MISMATCH when the section is absent. */
pai_status_t pai64_verify_section(const pai64_container_t *c, uint32_t type);

/* Map a file read-only (no size limit); unmap with pai64_unmap_file. IO on
 * failure. */
pai_status_t pai64_map_file(const char *path, const uint8_t **data, uint64_t *nbytes);
pai_status_t pai64_unmap_file(const uint8_t *data, uint64_t nbytes);

/* ------------------------------------------------------------------ */
/* Manifest                                                            */
/* ------------------------------------------------------------------ */

/* One entry: pai_pai_tensor_t (pai/pai.h:64-73) plus the GGUF block type
 * carried in the entry's reserved u16. */
typedef struct pai64_tensor {
  char name[64];
  uint32_t value_id;
  uint32_t dtype; /* pai_dtype_t */
  uint32_t rank;  /* 1..6 */
  uint64_t shape[6];
  uint64_t offset; /* into the WEIGHTS section */
  uint64_t size_bytes;
  uint32_t gguf_type; /* PAI_QTYPE_* for native GGUF blocks, else 0 */
} pai64_tensor_t;

/* Bytes pai64_manifest_encode writes for these entries (0 on bad input). */
uint64_t pai64_manifest_bytes(const pai64_tensor_t *tensors, uint32_t count);
/* Encode as the version-1 manifest (pai_pai_manifest_encode,
 * pai/pai.c:411-471) with the GGUF type in the reserved field.
 * INVALID_ARG for NULL, count 0, an empty or over-long name (63 chars at
 * most), a GGUF type above 65535, or too little room. */
pai_status_t pai64_manifest_encode(const pai64_tensor_t *tensors, uint32_t count, uint8_t *out,
                                   uint64_t cap, uint64_t *out_nbytes);
/* Decode, with pai_pai_manifest_decode's checks (pai/pai.c:473-540):
 * PROTOCOL for count 0 or above max_tensors, a truncated entry, an empty
 * or over-long name, rank outside 1..6, a dtype id of 9 or more, or a
 * zero size. */
pai_status_t pai64_manifest_decode(const uint8_t *data, uint64_t size, pai64_tensor_t *out,
                                   uint32_t max_tensors, uint32_t *out_count);

/* Upload a manifest tensor stored as native GGUF blocks to the device:
 * shape [K][N] (the graph's logical weight, rank 2), gguf_type one of the
 * PAI_QTYPE_* formats, its bytes inside the WEIGHTS section.
 * UNSUPPORTED when gguf_type is 0 or not a supported format, MISMATCH for
 * a shape, size or offset that does not fit, and pai_qmat_upload's
 * errors. */
pai_status_t pai64_qmat_upload(const pai64_container_t *c, const pai64_tensor_t *t,
                               pai_qmat_t **out);

/* ------------------------------------------------------------------ */
/* Tokenizer blob                                                      */
/* ------------------------------------------------------------------ */

/* Version 2 of the tokenizer blob (models/tokenizer.c:292-356): the
 * version-1 layout (u32 magic "PTK1", u32 version, u32 num_tokens, u32
 * num_merges; per token u32 id, u8 text length 1..255, the text; per
 * merge u32 left, right, result), with counts up to PAI64_TOK_MAX. */
#define PAI64_TOK_MAGIC 0x314B5450u
#define PAI64_TOK_VERSION 2u
#define PAI64_TOK_MAX (1u << 24)

/* Blob bytes for these token texts and merge count (0 on bad input). */
uint64_t pai64_tok_bytes(const char *const *texts, uint32_t ntok, uint32_t nmerge);
/* Encode: ids[i] and texts[i] (1..255 bytes, NUL-terminated) per token,
 * merges as (left, right, result) triples. INVALID_ARG for NULL, a count
 * above PAI64_TOK_MAX, a text length outside 1..255, or too little room. */
pai_status_t pai64_tok_encode(const uint32_t *ids, const char *const *texts, uint32_t ntok,
                              const uint32_t *merges, uint32_t nmerge, uint8_t *out,
                              uint64_t cap, uint64_t *out_nbytes);
/* Validate a version-1 or version-2 blob and index it: token and merge
 * counts, and (when entry_offsets is not NULL) the byte offset of each
 * token's entry (id at +0, length at +4, text at +5) for up to `cap`
 * tokens; *merges_offset is where the merge triples start. PROTOCOL for a
 * bad magic or version, counts above the version's caps (65 536 / 8 192
 * for version 1, PAI64_TOK_MAX for 2), a text length of 0, or a
 * truncated entry; INVALID_ARG for NULL or cap below the token count. */
pai_status_t pai64_tok_index(const uint8_t *blob, uint64_t nbytes, uint32_t *out_ntok,
                             uint32_t *out_nmerge, uint64_t *entry_offsets, uint32_t cap,
                             uint64_t *merges_offset);

#ifdef __cplusplus
}
#endif

#endif /* PAI_PAI64_H */
