/*
 * ecache_oracle.c -- CPU oracle (TEST INFRASTRUCTURE ONLY) of the expert
 * cache policy of src/ecache.c.  Only tests/ use it.  The restatement keeps
 * the reference's decisions -- slot claims, victim sampling, pins, counters
 * -- and replaces its reader threads with the deterministic completion model
 * described in ecache_oracle.h.  The record bytes are not modelled: a slot
 * index stands for the record.
 */
#include "ecache_oracle.h"

#include <stdlib.h>
#include <string.h>

static int32_t key_of(int layer, int expert) { return (int32_t)(((uint32_t)layer << 16) | (uint32_t)expert); }

/* a read succeeds when expert_fetch's range check passes (nn.c:1564-1567) */
static int fetch_ok(const orc_ecache *c, int layer, int expert)
{
    return layer >= 0 && layer < c->n_layer && expert >= 0 && expert < c->n_expert;
}

int orc_ecache_init(orc_ecache *c, size_t budget_bytes, size_t rec_bytes, int policy, int n_layer, int n_expert)
{
    /* ecache.c:194-229: no cache when the budget holds no record; else
       budget / rec slots, at least 4 */
    memset(c, 0, sizeof *c);
    c->rec_bytes = rec_bytes;
    c->policy = policy;
    c->rng = 0x9e3779b9u;
    c->pf_gen = 1;
    c->last_used = -1;
    c->n_layer = n_layer;
    c->n_expert = n_expert;
    if (!rec_bytes || budget_bytes < rec_bytes) return 0;
    c->n_slots = (int)(budget_bytes / rec_bytes);
    if (c->n_slots < 4) c->n_slots = 4;
    c->slot = (orc_eslot *)calloc((size_t)c->n_slots, sizeof *c->slot);
    if (!c->slot) return -1;
    for (int i = 0; i < c->n_slots; i++) c->slot[i].key = -1;
    return 0;
}

void orc_ecache_free(orc_ecache *c)
{
    free(c->slot);
    c->slot = NULL;
    c->n_slots = 0;
}

int orc_ecache_lookup(const orc_ecache *c, int layer, int expert)
{
    const int32_t k = key_of(layer, expert);
    for (int i = 0; i < c->n_slots; i++)
        if (c->slot[i].key == k) return i;
    return -1;
}

static int is_held(const orc_ecache *c, int i)
{
    for (int k = 0; k < c->n_held; k++)
        if (c->held[k] == i) return 1;
    return 0;
}

/* ecache.c:274-278: in flight, hinted in this generation, the last record
   handed out, or held */
static int pinned(const orc_ecache *c, int i)
{
    const orc_eslot *s = &c->slot[i];
    return s->state == ORC_EC_INFLIGHT || s->pin == c->pf_gen || i == c->last_used || is_held(c, i);
}

/* ecache.c:280-306: an empty slot (lowest index) if any; else the best of
   16 slots drawn with the LCG x <- 1664525 x + 1013904223 (mod 2^32), index
   x mod n_slots, pinned draws skipped; LFRU orders by (hits, last), LRU by
   last; if every draw was pinned, the lowest unpinned slot */
static int victim(orc_ecache *c)
{
    for (int i = 0; i < c->n_slots; i++)
        if (c->slot[i].state == ORC_EC_EMPTY) return i;
    int best = -1;
    uint32_t bh = 0;
    uint64_t bl = 0;
    for (int s = 0; s < ORC_EC_SAMPLE; s++) {
        c->rng = c->rng * 1664525u + 1013904223u;
        const int i = (int)(c->rng % (uint32_t)c->n_slots);
        if (pinned(c, i)) continue;
        const orc_eslot *sl = &c->slot[i];
        int better;
        if (c->policy == 1) better = best < 0 || sl->last < bl;
        else better = best < 0 || sl->hits < bh || (sl->hits == bh && sl->last < bl);
        if (better) {
            best = i;
            bh = sl->hits;
            bl = sl->last;
        }
    }
    if (best < 0)
        for (int i = 0; i < c->n_slots; i++)
            if (!pinned(c, i)) return i;
    return best;
}

static void set_key(orc_ecache *c, int vi, int32_t key)
{
    if (c->slot[vi].key >= 0) c->evictions++;
    c->slot[vi].key = key;
    c->slot[vi].state = ORC_EC_INFLIGHT;
}

/* speculative claim, ecache.c:308-323: immune through the next generation,
   zero hits, counted as spec_issued (not a miss) */
static void claim_spec(orc_ecache *c, int vi, int32_t key)
{
    set_key(c, vi, key);
    c->slot[vi].fresh = 0;
    c->slot[vi].pin = c->pf_gen + 1;
    c->slot[vi].birth = 0;
    c->slot[vi].hits = 0;
    c->slot[vi].last = c->clock;
    c->spec_issued++;
    c->bytes_read += c->rec_bytes;
}

/* demand claim, ecache.c:325-340: fresh (hinted) reads are pinned to the
   current generation and not yet a hit */
static void claim(orc_ecache *c, int vi, int32_t key, int fresh)
{
    set_key(c, vi, key);
    c->slot[vi].fresh = (uint8_t)fresh;
    c->slot[vi].pin = fresh ? c->pf_gen : 0;
    c->slot[vi].birth = fresh ? 1 : 2;
    c->slot[vi].hits = 1;
    c->slot[vi].last = c->clock;
    c->misses++;
    c->bytes_read += c->rec_bytes;
}

static void drop(orc_ecache *c, int vi)
{
    c->slot[vi].key = -1;
    c->slot[vi].state = ORC_EC_EMPTY;
    c->slot[vi].fresh = 0;
    c->slot[vi].pin = 0;
}

/* eio_push, ecache.c:113-138: demand reads go after the demand reads
   already queued and before every speculative one */
static int push(orc_ecache *c, int slot, int layer, int expert, int prio)
{
    if (c->qn == ORC_EC_QCAP) return -1;
    int pos = c->qn;
    if (prio) {
        pos = 0;
        while (pos < c->qn && c->q[(c->qhead + pos) % ORC_EC_QCAP].prio) pos++;
    }
    for (int i = c->qn; i > pos; i--) c->q[(c->qhead + i) % ORC_EC_QCAP] = c->q[(c->qhead + i - 1) % ORC_EC_QCAP];
    c->q[(c->qhead + pos) % ORC_EC_QCAP] = (orc_ejob){slot, layer, expert, prio};
    c->qn++;
    return 0;
}

static void complete_one(orc_ecache *c)
{
    const orc_ejob j = c->q[c->qhead];
    c->qhead = (c->qhead + 1) % ORC_EC_QCAP;
    c->qn--;
    c->slot[j.slot].state = fetch_ok(c, j.layer, j.expert) ? ORC_EC_READY : ORC_EC_FAILED;
}

void orc_ecache_drain(orc_ecache *c)
{
    while (c->qn > 0) complete_one(c);
}

/* ec_issue_next, ecache.c:352-376: start the next hinted read that is not
   resident (resident ones are re-pinned to this generation) */
static void issue_next(orc_ecache *c)
{
    if (!c->io_on) return;
    while (c->pf_issued < c->pf_n) {
        const int eid = c->pf_ids[c->pf_issued++];
        const int32_t key = key_of(c->pf_layer, eid);
        const int si = orc_ecache_lookup(c, c->pf_layer, eid);
        if (si >= 0) {
            c->slot[si].pin = c->pf_gen;
            continue;
        }
        const int vi = victim(c);
        if (vi < 0) {
            c->pf_issued--;
            return;
        }
        claim(c, vi, key, 1);
        c->prefetched++;
        if (push(c, vi, c->pf_layer, eid, 1) != 0) {
            c->prefetched--;
            c->misses--;
            c->bytes_read -= c->rec_bytes;
            drop(c, vi);
            c->pf_issued--;
        }
        return;
    }
}

int orc_ecache_io_start(orc_ecache *c, int nthreads, int depth)
{
    /* ecache.c:140-148: depth clamped to [1, n_slots / 4]; none fits -> off */
    if (c->io_on || nthreads <= 0 || c->n_slots <= 0) return 0;
    if (depth < 1) depth = 1;
    if (depth > c->n_slots / 4) depth = c->n_slots / 4;
    if (depth < 1) return 0;
    c->io_on = 1;
    c->depth = depth;
    return 0;
}

void orc_ecache_prefetch(orc_ecache *c, int layer, const int *ids, int n)
{
    /* ecache.c:378-397 */
    if (!c->io_on || c->n_slots <= 0 || n <= 0) return;
    for (int i = 0; i < n; i++) {
        if (ids[i] < 0) continue;
        if (orc_ecache_lookup(c, layer, ids[i]) >= 0) continue;
        const int vi = victim(c);
        if (vi < 0) break;
        claim_spec(c, vi, key_of(layer, ids[i]));
        if (push(c, vi, layer, ids[i], 0) != 0) {
            c->spec_issued--;
            c->bytes_read -= c->rec_bytes;
            drop(c, vi);
            break;
        }
    }
}

void orc_ecache_hint(orc_ecache *c, int layer, const int *ids, int n)
{
    /* ecache.c:399-412: a new generation; at most 64 ids and n_slots / 4;
       the first `depth` reads start now */
    if (!c->io_on || c->n_slots <= 0 || n <= 0) return;
    c->pf_gen++;
    c->pf_layer = layer;
    c->pf_n = n > ORC_EC_PF_MAX ? ORC_EC_PF_MAX : n;
    if (c->pf_n > c->n_slots / 4) c->pf_n = c->n_slots / 4;
    for (int i = 0; i < c->pf_n; i++) c->pf_ids[i] = ids[i];
    c->pf_issued = 0;
    for (int d = 0; d < c->depth; d++) issue_next(c);
}

int orc_ecache_get(orc_ecache *c, int layer, int expert)
{
    /* ecache.c:414-498 */
    const int32_t key = key_of(layer, expert);
    c->clock++;
    if (c->last_used >= 0 && c->slot[c->last_used].state == ORC_EC_READY) c->last_used = -1;
    if (c->n_slots > 0) {
        const int si = orc_ecache_lookup(c, layer, expert);
        if (si >= 0) {
            while (c->slot[si].state == ORC_EC_INFLIGHT && c->qn > 0) complete_one(c);
            if (c->slot[si].state != ORC_EC_READY) {
                drop(c, si);
                issue_next(c);
                return -1;
            }
            if (c->slot[si].fresh) c->slot[si].fresh = 0;     /* counted as a miss when issued */
            else {
                c->hits++;
                c->slot[si].hits++;
            }
            c->slot[si].last = c->clock;
            c->last_used = si;
            issue_next(c);
            return si;
        }
    }
    if (c->n_slots == 0) {
        c->misses++;
        c->bytes_read += c->rec_bytes;
        return -1;
    }
    /* not resident, not hinted: a synchronous read, through a slot */
    const int vi = victim(c);
    if (vi < 0) return -1;
    claim(c, vi, key, 0);
    if (!fetch_ok(c, layer, expert)) {
        drop(c, vi);
        return -1;
    }
    c->slot[vi].state = ORC_EC_READY;
    c->last_used = vi;
    issue_next(c);
    return vi;
}

int orc_ecache_hold(orc_ecache *c, int layer, int expert)
{
    /* ecache.c:500-514: as get, and the slot stays pinned until release */
    if (c->n_slots <= 0 || c->n_held >= ORC_EC_PF_MAX) return -1;
    const int r = orc_ecache_get(c, layer, expert);
    if (r < 0) return -1;
    if (c->last_used >= 0) {
        if (!is_held(c, c->last_used)) c->held[c->n_held++] = c->last_used;
        c->last_used = -1;
    }
    return r;
}

void orc_ecache_release(orc_ecache *c) { c->n_held = 0; }

void orc_ecache_clear(orc_ecache *c)
{
    /* ecache.c:522-540 (the generator and the generation are kept) */
    for (int i = 0; i < c->n_slots; i++) {
        drop(c, i);
        c->slot[i].hits = 0;
        c->slot[i].last = 0;
    }
    c->clock = c->hits = c->misses = c->bytes_read = 0;
    c->evictions = c->prefetched = c->spec_issued = 0;
    c->pf_n = c->pf_issued = 0;
    c->last_used = -1;
    c->n_held = 0;
}

orc_ecache *orc_ecache_create(size_t budget_bytes, size_t rec_bytes, int policy, int n_layer, int n_expert)
{
    orc_ecache *c = (orc_ecache *)malloc(sizeof *c);
    if (!c) return NULL;
    if (orc_ecache_init(c, budget_bytes, rec_bytes, policy, n_layer, n_expert) != 0) {
        free(c);
        return NULL;
    }
    return c;
}

void orc_ecache_destroy(orc_ecache *c)
{
    if (!c) return;
    orc_ecache_free(c);
    free(c);
}

void orc_ecache_counters(const orc_ecache *c, uint64_t out[7])
{
    out[0] = c->hits;
    out[1] = c->misses;
    out[2] = c->bytes_read;
    out[3] = c->evictions;
    out[4] = c->prefetched;
    out[5] = c->spec_issued;
    out[6] = (uint64_t)c->n_slots;
}
