/*
 * ecache_oracle.h -- CPU oracle (TEST INFRASTRUCTURE ONLY) of the expert
 * cache's policy: which record each get/hold/hint/prefetch reads, which slot
 * it lands in, and the hit/miss/eviction counters (src/ecache.c, declared at
 * src/ecache.h:95-123).  Only tests/ use it, as the checker of the GPU
 * library's HBM expert cache.
 *
 * The reference's reader threads are replaced by a deterministic model:
 * queued reads complete only when the caller drains the queue
 * (orc_ecache_drain, all of them in queue order) or when a get() meets a
 * record still in flight (the queue completes in order up to and including
 * that read).  Between those points every read the reference would have in
 * flight is in flight here too; a test that drains before each get sees the
 * same decisions from both.  A read fails, as expert_fetch (nn.c:1564-1567)
 * does, when the layer or expert is out of range.
 */
#ifndef ECACHE_ORACLE_H
#define ECACHE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_EC_EMPTY = 0, ORC_EC_READY, ORC_EC_INFLIGHT, ORC_EC_FAILED };
#define ORC_EC_PF_MAX 64
#define ORC_EC_SAMPLE 16
#define ORC_EC_QCAP 256

typedef struct {
    int32_t key;          /* layer << 16 | expert, -1 when empty */
    uint8_t state, fresh, birth;
    uint32_t hits;
    uint64_t last, pin;
} orc_eslot;

typedef struct {
    int slot, layer, expert, prio;
} orc_ejob;

typedef struct {
    orc_eslot *slot;
    int n_slots;
    size_t rec_bytes;
    int n_layer, n_expert;                 /* the fetch's valid range */
    uint64_t clock, hits, misses, bytes_read, evictions, prefetched, spec_issued;
    uint32_t rng;
    int policy;                            /* 0 LFRU, 1 LRU */
    int io_on, depth;
    uint64_t pf_gen;
    int pf_ids[ORC_EC_PF_MAX];
    int pf_layer, pf_n, pf_issued;
    int held[ORC_EC_PF_MAX];
    int n_held, last_used;
    orc_ejob q[ORC_EC_QCAP];
    int qhead, qn;
} orc_ecache;

int  orc_ecache_init(orc_ecache *c, size_t budget_bytes, size_t rec_bytes, int policy, int n_layer,
                     int n_expert);
void orc_ecache_free(orc_ecache *c);
void orc_ecache_clear(orc_ecache *c);
/* reader threads on (nthreads > 0): hint/prefetch become active */
int  orc_ecache_io_start(orc_ecache *c, int nthreads, int depth);
/* slot index of the record, or -1 (failed read, or no cache) */
int  orc_ecache_get(orc_ecache *c, int layer, int expert);
int  orc_ecache_hold(orc_ecache *c, int layer, int expert);
void orc_ecache_release(orc_ecache *c);
void orc_ecache_hint(orc_ecache *c, int layer, const int *ids, int n);
void orc_ecache_prefetch(orc_ecache *c, int layer, const int *ids, int n);
void orc_ecache_drain(orc_ecache *c);
/* slot holding (layer, expert) in any state, or -1 */
int  orc_ecache_lookup(const orc_ecache *c, int layer, int expert);
/* heap-allocated cache for bindings; counters out[0..6] = hits, misses,
   bytes_read, evictions, prefetched, spec_issued, n_slots */
orc_ecache *orc_ecache_create(size_t budget_bytes, size_t rec_bytes, int policy, int n_layer, int n_expert);
void orc_ecache_destroy(orc_ecache *c);
void orc_ecache_counters(const orc_ecache *c, uint64_t out[7]);

#ifdef __cplusplus
}
#endif
#endif
