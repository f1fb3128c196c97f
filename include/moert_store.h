/*
 * moert_store.h -- the expert store v0 (experts.index + experts.pack).
 *
 * Replaces moert/include/moert/store.h: the same entry points, structs and
 * on-disk layout (moert/memmgr/store_format.h: a 96-byte index header,
 * 72-byte records, a 32-byte pack header, pages 256-aligned, FNV-1a 64
 * checksums), so stores written by either side are read by the other.
 * Host code; the pages go to device memory through llapis_store_upload
 * (llapis_moe.h).
 */
#ifndef MOERT_STORE_HIP_H
#define MOERT_STORE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOERT_STORE_INDEX_SUFFIX ".experts.index"
#define MOERT_STORE_PACK_SUFFIX  ".experts.pack"

/* store.h:32-37 */
enum moert_page_flags {
    MOERT_PAGE_REQUANTIZED = 1 << 0,
    MOERT_PAGE_IMATRIX     = 1 << 1,
    MOERT_PAGE_PADDED      = 1 << 2,
    MOERT_PAGE_SCALE       = 1 << 3,
};

/* store.h:40-50 (layout is ABI) */
typedef struct moert_store_info {
    uint32_t format_version;
    uint64_t source_uuid;
    char     arch[16];
    int32_t  n_layers;
    int32_t  n_expert;
    uint64_t n_embd;
    uint64_t n_ff_exp;
    uint64_t pack_uuid;
    uint64_t record_count;
} moert_store_info;

/* store.h:53: 1 = a valid index header was read into out, 0 = missing/invalid. */
int32_t moert_store_probe(const char * index_path, moert_store_info * out);
/* store.h:58: pages whose checksum fails (0 = clean), -1 on an I/O or format error. */
int64_t moert_store_verify(const char * index_path);

/* store.h:62-80: the writer (pack_uuid 0 = generated; 1 = ok / 0 = failed). */
typedef struct moert_store_writer moert_store_writer;
moert_store_writer * moert_store_writer_open(const char * index_path, const char * pack_path,
                                             const moert_store_info * info);
int32_t moert_store_writer_add_page(moert_store_writer * w,
                                    int32_t layer, int32_t expert_id, int32_t kind, int32_t is_scale,
                                    int32_t quant_type, int32_t source_quant, uint32_t extra_flags,
                                    const int64_t * shape, int32_t ndim,
                                    const void * bytes, uint64_t nbytes);
int32_t moert_store_writer_close(moert_store_writer * w);

/* store.h:84 */
uint64_t moert_store_fnv1a64(const void * data, uint64_t nbytes, uint64_t seed);
#define MOERT_STORE_FNV_SEED 14695981039346656037ull

/* store.h:92-120: per-page reads into host memory. */
typedef struct moert_store_reader moert_store_reader;
moert_store_reader * moert_store_reader_open(const char * index_path, uint64_t expect_source_uuid);
void     moert_store_reader_free(moert_store_reader * r);
int32_t  moert_store_reader_geometry(const moert_store_reader * r, int32_t * n_layers, int32_t * n_expert);
uint64_t moert_store_reader_page_nbytes(const moert_store_reader * r,
                                        int32_t layer, int32_t kind, int32_t is_scale, int32_t expert);
int32_t  moert_store_reader_page_info(const moert_store_reader * r,
                                      int32_t layer, int32_t kind, int32_t is_scale, int32_t expert,
                                      int32_t * quant_type, uint64_t * nbytes, int64_t shape[4]);
uint64_t moert_store_reader_read(moert_store_reader * r,
                                 int32_t layer, int32_t kind, int32_t is_scale, int32_t expert,
                                 void * dst, uint64_t dst_cap, int32_t verify);

#ifdef __cplusplus
}
#endif
#endif
