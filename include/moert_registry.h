/*
 * moert_registry.h -- where a (layer, expert)'s bytes can be copied from:
 * the same types, values and inline functions as the reference's
 * moert/include/moert/registry.h:21-49 (moert_rep, moert_source,
 * moert_expert_where, moert_source_for, moert_source_name), so host code
 * that composes a moert_expert_where and asks for a source compiles against
 * either header.  Header-only, no allocation, no device calls.
 *
 * Sources, cheapest first: a READY hot slot (a device-to-device copy), the
 * arena, a file.  A slot holds the HOT representation and the arena the COLD
 * one; either serves the other representation only when the two are the
 * same bytes.  On MI355X (one GPU, 288 GB) the arena is the HBM-resident
 * cold pool, and the "file" is an expert store or GGUF read through
 * llapis_store_upload / llapis_gguf_upload; the promotion engine's HBM
 * promotion source (every expert in the hot formats) answers a HOT request
 * as a device-to-device copy, which is the slot's cost class.
 */
#ifndef MOERT_REGISTRY_H
#define MOERT_REGISTRY_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum moert_rep { MOERT_REP_HOT = 0, MOERT_REP_COLD = 1 };
enum moert_source { MOERT_SRC_NONE = 0, MOERT_SRC_SLOT = 1, MOERT_SRC_ARENA = 2, MOERT_SRC_FILE = 3 };

typedef struct moert_expert_where {
    int32_t slot;          /* READY hot slot holding the expert's HOT bytes, or -1 */
    int32_t arena_valid;   /* the arena holds (or will hold, for a job queued now) the COLD bytes */
    int32_t same_bytes;    /* the HOT and COLD representations are byte-identical */
    int32_t file_hot;      /* a file holds the HOT representation */
    int32_t file_cold;     /* a file holds the COLD representation */
} moert_expert_where;

/* The cheapest source holding representation `rep` (a moert_rep) of the
 * expert, MOERT_SRC_NONE if no source does (or w is NULL). */
static inline int32_t moert_source_for(const moert_expert_where * w, int32_t rep) {
    if (w == 0) return MOERT_SRC_NONE;
    const int32_t want_hot = (rep == MOERT_REP_HOT);
    /* which representations each source can hand out */
    const int32_t slot_serves = (w->slot >= 0) && (want_hot || w->same_bytes);
    const int32_t arena_serves = (w->arena_valid != 0) && (!want_hot || w->same_bytes);
    const int32_t file_serves = want_hot ? (w->file_hot != 0) : (w->file_cold != 0);
    return slot_serves ? MOERT_SRC_SLOT : arena_serves ? MOERT_SRC_ARENA : file_serves ? MOERT_SRC_FILE
                                                                                          : MOERT_SRC_NONE;
}

/* "slot", "arena", "file", or "none" for any other value. */
static inline const char * moert_source_name(int32_t src) {
    static const char * const names[4] = {"none", "slot", "arena", "file"};
    return (src >= MOERT_SRC_SLOT && src <= MOERT_SRC_FILE) ? names[src] : names[0];
}

#ifdef __cplusplus
}
#endif
#endif
