// qmag_ecache.hip -- a bounded cache of expert records in HBM: the role of
// qma_ecache (src/ecache.h:95-123, src/ecache.c) for models whose experts do
// not all fit on the device.  Host code only.
//
// The slots are one device allocation, n_slots = budget / rec_bytes (at
// least 4), each rec_bytes rounded up to 64 KiB.  A record is one expert's
// gate, up and down slabs back to back, as the reference's fetch callback
// lays them out (nn.c:1564-1595).  A read runs the caller's fetch callback
// into pinned host staging (one buffer per reader thread, one for the
// calling thread) and then copies the record into its slot on the cache's
// own copy stream.  The policy -- slot claims, LFRU/LRU victims drawn with
// the reference's sampler, pins for in-flight, hinted, held and last-used
// records, the demand-before-speculative read queue, and the counters -- is
// the reference's, decision for decision.
//
// Ordering on the device.  Every public call first records an event on the
// library stream; a copy into a slot waits on that event, so it lands only
// after every kernel queued before the call that freed the slot (a record
// handed out stays valid for work queued before the next get, or, held,
// before the release).  get() returns once the record's copy has completed,
// so kernels queued afterwards read the new bytes.
#include <string.h>

#include <condition_variable>
#include <deque>
#include <mutex>
#include <set>
#include <thread>
#include <unordered_map>
#include <vector>

#include "qmag_internal.h"

namespace {

enum { EC_EMPTY = 0, EC_READY, EC_INFLIGHT, EC_FAILED };
constexpr int PF_MAX = 64;        // most ids one hint takes, and most holds
constexpr int SAMPLE = 16;        // victims drawn per eviction
constexpr int QCAP = 256;         // queued reads
constexpr int MAXIO = 8;          // reader threads
constexpr size_t SLOT_ALIGN = 64 * 1024;

struct Slot {
    int32_t key = -1;
    uint8_t state = EC_EMPTY, fresh = 0;
    uint32_t hits = 0;
    uint64_t last = 0, pin = 0;
};
struct Job {
    int slot, layer, expert, prio;
};

int32_t key_of(int layer, int expert) { return (int32_t)(((uint32_t)layer << 16) | (uint32_t)expert); }

}  // namespace

struct qmag_ecache {
    std::vector<Slot> slot;
    int n_slots = 0;
    // the resident keys (key -> slot) and the empty slots in index order, so
    // that neither a lookup nor the first-empty-slot rule scans every slot
    // (an HBM budget holds over 100,000 records of 2 MB)
    std::unordered_map<int32_t, int> index;
    std::set<int> empty;
    size_t rec_bytes = 0, slot_bytes = 0;
    uint64_t clock = 0, hits = 0, misses = 0, bytes_read = 0, evictions = 0, prefetched = 0, spec_issued = 0;
    uint32_t rng = 0x9e3779b9u;
    int policy = 0;
    uint64_t pf_gen = 1;
    int pf_ids[PF_MAX] = {};
    int pf_layer = 0, pf_n = 0, pf_issued = 0;
    int held[PF_MAX] = {};
    int n_held = 0, last_used = -1;

    uint8_t *pool = nullptr;                 // device slots
    hipStream_t copy = nullptr;
    hipEvent_t use_ev = nullptr;             // library-stream work up to the last call
    uint8_t *sync_stage = nullptr;           // pinned staging for reads on the calling thread
    hipEvent_t sync_ev = nullptr;

    // reader threads
    std::mutex mu;
    std::condition_variable work, done;
    std::deque<Job> q;
    bool stop = false, io = false;
    int depth = 0;
    std::vector<std::thread> th;
    std::vector<uint8_t *> stage;            // pinned, one per reader
    std::vector<hipEvent_t> th_ev;
    qmag_fetch_fn fetch = nullptr;
    void *fetch_user = nullptr;
    const void *fits_user = nullptr;         // a GGUF file whose records fit rec_bytes
    int hip_error = 0;                       // first HIP failure seen by a reader
};

namespace {

using qmag::fail;

int lookup(const qmag_ecache *c, int32_t key)
{
    const auto it = c->index.find(key);
    return it == c->index.end() ? -1 : it->second;
}

bool is_held(const qmag_ecache *c, int i)
{
    for (int k = 0; k < c->n_held; k++)
        if (c->held[k] == i) return true;
    return false;
}

bool pinned(const qmag_ecache *c, int i)
{
    const Slot &s = c->slot[i];
    return s.state == EC_INFLIGHT || s.pin == c->pf_gen || i == c->last_used || is_held(c, i);
}

// ecache.c:280-306: first empty slot; else the best unpinned of SAMPLE draws
// of the LCG x <- 1664525 x + 1013904223, slot x mod n_slots (LFRU: fewest
// hits, then least recent; LRU: least recent); else the first unpinned
int victim(qmag_ecache *c)
{
    if (!c->empty.empty()) return *c->empty.begin();     // the lowest empty slot
    int best = -1;
    uint32_t bh = 0;
    uint64_t bl = 0;
    for (int s = 0; s < SAMPLE; s++) {
        c->rng = c->rng * 1664525u + 1013904223u;
        const int i = (int)(c->rng % (uint32_t)c->n_slots);
        if (pinned(c, i)) continue;
        const Slot &sl = c->slot[i];
        const bool better = c->policy == 1 ? (best < 0 || sl.last < bl)
                                           : (best < 0 || sl.hits < bh || (sl.hits == bh && sl.last < bl));
        if (better) {
            best = i;
            bh = sl.hits;
            bl = sl.last;
        }
    }
    if (best < 0)
        for (int i = 0; i < c->n_slots; i++)
            if (!pinned(c, i)) return i;
    return best;
}

void take(qmag_ecache *c, int vi, int32_t key)
{
    if (c->slot[vi].key >= 0) {
        c->evictions++;
        c->index.erase(c->slot[vi].key);
    }
    c->empty.erase(vi);
    c->index[key] = vi;
    c->slot[vi].key = key;
    c->slot[vi].state = EC_INFLIGHT;
}

// speculative read (ecache.c:308-323): immune through the next generation
void claim_spec(qmag_ecache *c, int vi, int32_t key)
{
    take(c, vi, key);
    Slot &s = c->slot[vi];
    s.fresh = 0;
    s.pin = c->pf_gen + 1;
    s.hits = 0;
    s.last = c->clock;
    c->spec_issued++;
    c->bytes_read += c->rec_bytes;
}

// demand read (ecache.c:325-340): a hinted (fresh) one is pinned to this
// generation and becomes a hit only on its second get
void claim(qmag_ecache *c, int vi, int32_t key, bool fresh)
{
    take(c, vi, key);
    Slot &s = c->slot[vi];
    s.fresh = fresh;
    s.pin = fresh ? c->pf_gen : 0;
    s.hits = 1;
    s.last = c->clock;
    c->misses++;
    c->bytes_read += c->rec_bytes;
}

void drop(qmag_ecache *c, int vi)
{
    Slot &s = c->slot[vi];
    if (s.key >= 0) c->index.erase(s.key);
    c->empty.insert(vi);
    s.key = -1;
    s.state = EC_EMPTY;
    s.fresh = 0;
    s.pin = 0;
}

// the read queue (ecache.c:113-138): demand reads after the demand reads
// already queued, ahead of every speculative one
bool push(qmag_ecache *c, int slot, int layer, int expert, int prio)
{
    if ((int)c->q.size() >= QCAP) return false;
    auto it = c->q.end();
    if (prio) {
        it = c->q.begin();
        while (it != c->q.end() && it->prio) ++it;
    }
    c->q.insert(it, Job{slot, layer, expert, prio});
    c->work.notify_one();
    return true;
}

// ecache.c:352-376 (under the lock)
void issue_next(qmag_ecache *c)
{
    if (!c->io) return;
    while (c->pf_issued < c->pf_n) {
        const int eid = c->pf_ids[c->pf_issued++];
        const int32_t key = key_of(c->pf_layer, eid);
        const int si = lookup(c, key);
        if (si >= 0) {
            c->slot[si].pin = c->pf_gen;
            continue;
        }
        const int vi = victim(c);
        if (vi < 0) {
            c->pf_issued--;
            return;
        }
        claim(c, vi, key, true);
        c->prefetched++;
        if (!push(c, vi, c->pf_layer, eid, 1)) {
            c->prefetched--;
            c->misses--;
            c->bytes_read -= c->rec_bytes;
            drop(c, vi);
            c->pf_issued--;
        }
        return;
    }
}

// queue the copy of a staged record into slot si behind the library-stream
// work recorded in use_ev (under the lock), then wait for it (outside)
bool copy_in(qmag_ecache *c, std::unique_lock<std::mutex> &lk, int si, const uint8_t *stage, hipEvent_t ev)
{
    hipError_t e = hipStreamWaitEvent(c->copy, c->use_ev, 0);
    if (e == hipSuccess)
        e = hipMemcpyAsync(c->pool + (size_t)si * c->slot_bytes, stage, c->rec_bytes, hipMemcpyHostToDevice,
                           c->copy);
    if (e == hipSuccess) e = hipEventRecord(ev, c->copy);
    if (e != hipSuccess) return false;
    lk.unlock();
    e = hipEventSynchronize(ev);
    lk.lock();
    return e == hipSuccess;
}

void reader(qmag_ecache *c, int t)
{
    (void)hipSetDevice(qmag::ctx().dev);               // the current device is per thread
    std::unique_lock<std::mutex> lk(c->mu);
    for (;;) {
        c->work.wait(lk, [&] { return c->stop || !c->q.empty(); });
        if (c->q.empty()) return;                      // stop, and nothing left
        const Job j = c->q.front();
        c->q.pop_front();
        lk.unlock();
        const int rc = c->fetch(c->fetch_user, j.layer, j.expert, c->stage[t]);
        lk.lock();
        bool ok = rc == 0;
        if (ok && !copy_in(c, lk, j.slot, c->stage[t], c->th_ev[t])) {
            ok = false;
            c->hip_error = 1;
        }
        c->slot[j.slot].state = ok ? EC_READY : EC_FAILED;
        c->done.notify_all();
    }
}

// The fetch callback fills rec_bytes of staging and cannot be told the size.
// The library's own GGUF callback writes the record of the layer asked for,
// and down types vary per layer: check once per file that its largest
// record fits (under the lock).
bool fetch_fits(qmag_ecache *c, qmag_fetch_fn fetch, void *user)
{
    if (fetch != qmag_gguf_fetch_expert || !user || user == c->fits_user) return true;
    size_t rec = 0;
    if (qmag_gguf_expert_record_bytes((const qmag_gguf *)user, &rec) != QMAG_OK) return false;
    if (rec > c->rec_bytes) {
        fail(QMAG_ERR_ARG, "ecache: records of %zu bytes, the file's largest has %zu", c->rec_bytes, rec);
        return false;
    }
    c->fits_user = user;
    return true;
}

// the calling-thread part of every public call: order later copies behind
// the library-stream work queued so far
void mark_use(qmag_ecache *c)
{
    (void)hipEventRecord(c->use_ev, qmag::ctx().stream);
}

const uint8_t *get_locked(qmag_ecache *c, std::unique_lock<std::mutex> &lk, int layer, int expert,
                          qmag_fetch_fn fetch, void *user)
{
    // ecache.c:414-498
    const int32_t key = key_of(layer, expert);
    c->clock++;
    if (c->last_used >= 0 && c->slot[c->last_used].state == EC_READY) c->last_used = -1;
    while (c->n_slots > 0) {
        const int si = lookup(c, key);
        if (si < 0) break;
        {
            // Wait for the read in flight.  While this call waits the slot can
            // change hands (the read fails and another call drops it, or it
            // lands and is evicted and claimed for another record): then the
            // key is looked up again instead of the slot's new record being
            // returned under this key.
            c->done.wait(lk, [&] { return c->slot[si].key != key || c->slot[si].state != EC_INFLIGHT; });
            if (c->slot[si].key != key) continue;
            if (c->slot[si].state != EC_READY) {
                drop(c, si);
                issue_next(c);
                return nullptr;
            }
            Slot &s = c->slot[si];
            if (s.fresh) s.fresh = 0;          // counted as a miss when issued
            else {
                c->hits++;
                s.hits++;
            }
            s.last = c->clock;
            c->last_used = si;
            issue_next(c);
            return c->pool + (size_t)si * c->slot_bytes;
        }
    }
    if (c->n_slots == 0) {
        c->misses++;
        c->bytes_read += c->rec_bytes;
        return nullptr;
    }
    // not resident, not hinted: read it here, through a slot
    if (!fetch_fits(c, fetch, user)) return nullptr;
    const int vi = victim(c);
    if (vi < 0) return nullptr;
    claim(c, vi, key, false);
    // one synchronous read at a time uses the calling-thread staging buffer
    c->done.wait(lk, [&] { return c->sync_ev != nullptr; });
    hipEvent_t ev = c->sync_ev;
    c->sync_ev = nullptr;
    lk.unlock();
    const int rc = fetch ? fetch(user, layer, expert, c->sync_stage) : -1;
    lk.lock();
    bool ok = rc == 0 && copy_in(c, lk, vi, c->sync_stage, ev);
    c->sync_ev = ev;
    c->done.notify_all();
    if (!ok) {
        drop(c, vi);
        return nullptr;
    }
    c->slot[vi].state = EC_READY;
    c->last_used = vi;
    issue_next(c);
    return c->pool + (size_t)vi * c->slot_bytes;
}

void stop_io(qmag_ecache *c)
{
    {
        std::lock_guard<std::mutex> g(c->mu);
        if (!c->io) return;
        c->stop = true;
        c->work.notify_all();
    }
    for (auto &t : c->th) t.join();
    c->th.clear();
    for (uint8_t *p : c->stage) (void)hipHostFree(p);
    for (hipEvent_t e : c->th_ev) (void)hipEventDestroy(e);
    c->stage.clear();
    c->th_ev.clear();
    std::lock_guard<std::mutex> g(c->mu);
    c->io = false;
    c->stop = false;
}

}  // namespace

using namespace qmag;

extern "C" {

int qmag_ecache_init(qmag_ecache **out, size_t budget_bytes, size_t rec_bytes, int policy)
{
    int st = require_ready();
    if (st) return st;
    if (!out) return fail(QMAG_ERR_ARG, "ecache: null handle");
    *out = nullptr;
    qmag_ecache *c = new qmag_ecache();
    c->rec_bytes = rec_bytes;
    c->policy = policy;
    // ecache.c:194-229: no slots when the budget holds no record
    if (rec_bytes && budget_bytes >= rec_bytes) {
        c->n_slots = (int)(budget_bytes / rec_bytes);
        if (c->n_slots < 4) c->n_slots = 4;
    }
    c->slot.assign((size_t)c->n_slots, Slot{});
    for (int i = 0; i < c->n_slots; i++) c->empty.insert(c->empty.end(), i);
    c->slot_bytes = (rec_bytes + SLOT_ALIGN - 1) / SLOT_ALIGN * SLOT_ALIGN;
    hipError_t e = hipSuccess;
    if (c->n_slots > 0) {
        e = hipMalloc(&c->pool, c->slot_bytes * (size_t)c->n_slots);
        if (e == hipSuccess) e = hipHostMalloc((void **)&c->sync_stage, rec_bytes, hipHostMallocDefault);
    }
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&c->copy, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&c->use_ev, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&c->sync_ev, hipEventDisableTiming);
    if (e != hipSuccess) {
        qmag_ecache_free(c);
        return hip_fail(e, "ecache init", __FILE__, __LINE__);
    }
    *out = c;
    return QMAG_OK;
}

void qmag_ecache_free(qmag_ecache *c)
{
    if (!c) return;
    stop_io(c);
    if (c->copy) (void)hipStreamSynchronize(c->copy);
    if (c->pool) {
        (void)hipStreamSynchronize(ctx().stream);        // kernels may still read slots
        (void)hipFree(c->pool);
    }
    if (c->sync_stage) (void)hipHostFree(c->sync_stage);
    if (c->sync_ev) (void)hipEventDestroy(c->sync_ev);
    if (c->use_ev) (void)hipEventDestroy(c->use_ev);
    if (c->copy) (void)hipStreamDestroy(c->copy);
    delete c;
}

void qmag_ecache_clear(qmag_ecache *c)
{
    // ecache.c:522-540, after the reads already queued or in flight have
    // landed: a reader still holding a job would otherwise copy its record
    // into a slot that may since hold another key
    if (!c) return;
    std::unique_lock<std::mutex> lk(c->mu);
    mark_use(c);
    c->done.wait(lk, [&] {
        if (!c->q.empty()) return false;
        for (const Slot &s : c->slot)
            if (s.state == EC_INFLIGHT) return false;
        return true;
    });
    c->index.clear();
    c->empty.clear();
    for (int i = 0; i < c->n_slots; i++) c->empty.insert(c->empty.end(), i);
    for (Slot &s : c->slot) {
        s.key = -1;
        s.state = EC_EMPTY;
        s.fresh = 0;
        s.pin = 0;
        s.hits = 0;
        s.last = 0;
    }
    c->clock = c->hits = c->misses = c->bytes_read = 0;
    c->evictions = c->prefetched = c->spec_issued = 0;
    c->pf_n = c->pf_issued = 0;
    c->last_used = -1;
    c->n_held = 0;
}

int qmag_ecache_io_start(qmag_ecache *c, qmag_fetch_fn fetch, void *user, int nthreads, int depth)
{
    // ecache.c:140-148: nothing to do without threads or slots; depth clamped
    // to [1, n_slots / 4]
    if (!c) return fail(QMAG_ERR_ARG, "ecache: null handle");
    if (c->io || nthreads <= 0 || c->n_slots <= 0 || !fetch) return QMAG_OK;
    if (nthreads > MAXIO) nthreads = MAXIO;
    if (depth < 1) depth = 1;
    if (depth > c->n_slots / 4) depth = c->n_slots / 4;
    if (depth < 1) return QMAG_OK;
    {
        std::lock_guard<std::mutex> g(c->mu);
        if (!fetch_fits(c, fetch, user)) return QMAG_ERR_ARG;
    }
    for (int t = 0; t < nthreads; t++) {
        uint8_t *p = nullptr;
        hipEvent_t ev = nullptr;
        if (hipHostMalloc((void **)&p, c->rec_bytes, hipHostMallocDefault) != hipSuccess) break;
        if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
            (void)hipHostFree(p);
            break;
        }
        c->stage.push_back(p);
        c->th_ev.push_back(ev);
    }
    if (c->stage.empty()) return fail(QMAG_ERR_HIP, "ecache: no pinned staging for the readers");
    std::lock_guard<std::mutex> g(c->mu);
    c->fetch = fetch;
    c->fetch_user = user;
    c->depth = depth;
    c->io = true;
    for (size_t t = 0; t < c->stage.size(); t++) c->th.emplace_back(reader, c, (int)t);
    return QMAG_OK;
}

void qmag_ecache_io_stop(qmag_ecache *c)
{
    if (c) stop_io(c);
}

void qmag_ecache_hint(qmag_ecache *c, int layer, const int *ids, int n)
{
    // ecache.c:399-412
    if (!c || !ids) return;
    std::lock_guard<std::mutex> g(c->mu);
    if (!c->io || c->n_slots <= 0 || n <= 0) return;
    mark_use(c);
    c->pf_gen++;
    c->pf_layer = layer;
    c->pf_n = n > PF_MAX ? PF_MAX : n;
    if (c->pf_n > c->n_slots / 4) c->pf_n = c->n_slots / 4;
    for (int i = 0; i < c->pf_n; i++) c->pf_ids[i] = ids[i];
    c->pf_issued = 0;
    for (int d = 0; d < c->depth; d++) issue_next(c);
}

void qmag_ecache_prefetch(qmag_ecache *c, int layer, const int *ids, int n)
{
    // ecache.c:378-397
    if (!c || !ids) return;
    std::lock_guard<std::mutex> g(c->mu);
    if (!c->io || c->n_slots <= 0 || n <= 0) return;
    mark_use(c);
    for (int i = 0; i < n; i++) {
        if (ids[i] < 0) continue;
        const int32_t key = key_of(layer, ids[i]);
        if (lookup(c, key) >= 0) continue;
        const int vi = victim(c);
        if (vi < 0) break;
        claim_spec(c, vi, key);
        if (!push(c, vi, layer, ids[i], 0)) {
            c->spec_issued--;
            c->bytes_read -= c->rec_bytes;
            drop(c, vi);
            break;
        }
    }
}

const uint8_t *qmag_ecache_get(qmag_ecache *c, int layer, int expert, qmag_fetch_fn fetch, void *user)
{
    if (!c) return nullptr;
    std::unique_lock<std::mutex> lk(c->mu);
    mark_use(c);
    return get_locked(c, lk, layer, expert, fetch, user);
}

const uint8_t *qmag_ecache_hold(qmag_ecache *c, int layer, int expert, qmag_fetch_fn fetch, void *user)
{
    // ecache.c:500-514
    if (!c) return nullptr;
    std::unique_lock<std::mutex> lk(c->mu);
    if (c->n_slots <= 0 || c->n_held >= PF_MAX) return nullptr;
    mark_use(c);
    const uint8_t *r = get_locked(c, lk, layer, expert, fetch, user);
    if (!r) return nullptr;
    if (c->last_used >= 0) {
        if (!is_held(c, c->last_used)) c->held[c->n_held++] = c->last_used;
        c->last_used = -1;
    }
    return r;
}

void qmag_ecache_release(qmag_ecache *c)
{
    if (!c) return;
    std::lock_guard<std::mutex> g(c->mu);
    mark_use(c);
    c->n_held = 0;
}

int qmag_ecache_drain(qmag_ecache *c)
{
    if (!c) return fail(QMAG_ERR_ARG, "ecache: null handle");
    std::unique_lock<std::mutex> lk(c->mu);
    c->done.wait(lk, [&] {
        if (!c->q.empty()) return false;
        for (const Slot &s : c->slot)
            if (s.state == EC_INFLIGHT) return false;
        return true;
    });
    if (c->hip_error) return fail(QMAG_ERR_HIP, "ecache: a record copy failed");
    return QMAG_OK;
}

int qmag_ecache_stats(const qmag_ecache *c, qmag_ecache_counters *out)
{
    if (!c || !out) return fail(QMAG_ERR_ARG, "ecache: null argument");
    qmag_ecache *m = const_cast<qmag_ecache *>(c);
    std::lock_guard<std::mutex> g(m->mu);
    out->hits = c->hits;
    out->misses = c->misses;
    out->bytes_read = c->bytes_read;
    out->evictions = c->evictions;
    out->prefetched = c->prefetched;
    out->spec_issued = c->spec_issued;
    out->n_slots = c->n_slots;
    out->rec_bytes = c->rec_bytes;
    out->slot_bytes = c->slot_bytes;
    return QMAG_OK;
}

int qmag_ecache_slot_of(const qmag_ecache *c, int layer, int expert)
{
    if (!c) return -1;
    qmag_ecache *m = const_cast<qmag_ecache *>(c);
    std::lock_guard<std::mutex> g(m->mu);
    return lookup(c, key_of(layer, expert));
}

const uint8_t *qmag_ecache_slot_ptr(const qmag_ecache *c, int slot)
{
    if (!c || slot < 0 || slot >= c->n_slots) return nullptr;
    return c->pool + (size_t)slot * c->slot_bytes;
}

}  // extern "C"
