// qmag_gguf.hip -- GGUF v3 weights into HBM residency: the loader role of
// src/gguf.c (qma_load, gguf.c:104-345) for the tensors of the MoE FFN path.
// Host code only.
//
// The file is mapped read-only and indexed: header, metadata (the keys this
// path reads, with the architecture prefix stripped as gguf.c:146-153 does),
// the tensor table (name, dims, type, offset) and the data section, which
// starts at the next multiple of general.alignment (default 32) after the
// table (gguf.c:254-262).  Every read is bounds-checked; a tensor whose bytes
// fall outside the file, whose first dimension is not a whole number of
// blocks, or whose type is not F32 / Q4_K / Q6_K fails the open, as
// gguf.c:264-283 does.  Expert tensors are 3-D with the expert index slowest
// (gguf.c:268-271), so each uploads as one contiguous copy, expert-major
// slabs unchanged: the layout the kernels read.
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <string>
#include <unordered_map>
#include <vector>

#include "qmag_internal.h"

struct GgufTensor {
    std::string name;
    int type;
    int64_t ne[3];
    uint64_t off;       // relative to the data section
    size_t nbytes;
};

struct qmag_gguf {
    int fd = -1;
    const uint8_t *map = nullptr;
    size_t size = 0;
    const uint8_t *data = nullptr;
    std::vector<GgufTensor> tensors;
    std::unordered_map<std::string, size_t> by_name;
    std::unordered_map<std::string, uint64_t> meta_u;   // unsigned / integer metadata, prefix stripped
};

namespace {

enum {
    GV_U8 = 0, GV_I8, GV_U16, GV_I16, GV_U32, GV_I32, GV_F32, GV_BOOL, GV_STR, GV_ARR, GV_U64, GV_I64, GV_F64
};
enum { T_F32 = 0, T_Q4K = 12, T_Q6K = 14 };

constexpr size_t QK_K_ELEMS = 256;
using qmag::fail;
#define err fail

struct Reader {
    const uint8_t *p, *end;
    bool bad = false;
    bool take(void *dst, size_t n)
    {
        if (bad || (size_t)(end - p) < n) {
            bad = true;
            return false;
        }
        memcpy(dst, p, n);
        p += n;
        return true;
    }
    uint64_t u64()
    {
        uint64_t v = 0;
        take(&v, 8);
        return v;
    }
    uint32_t u32()
    {
        uint32_t v = 0;
        take(&v, 4);
        return v;
    }
    std::string str()
    {
        const uint64_t n = u64();
        if (bad || (uint64_t)(end - p) < n) {
            bad = true;
            return std::string();
        }
        std::string s((const char *)p, (size_t)n);
        p += n;
        return s;
    }
    // skip one value of type t (arrays recursively, bounded depth)
    void skip(uint32_t t, int depth = 0)
    {
        static const int width[] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
        if (t <= GV_F64 && width[t]) {
            if ((size_t)(end - p) < (size_t)width[t]) bad = true;
            else p += width[t];
        } else if (t == GV_STR) {
            str();
        } else if (t == GV_ARR && depth < 4) {
            const uint32_t at = u32();
            const uint64_t n = u64();
            if (at <= GV_F64 && width[at] && !bad) {        // fixed-width elements: one bounds check
                if ((uint64_t)(end - p) / width[at] < n) bad = true;
                else p += n * width[at];
            } else {
                for (uint64_t i = 0; i < n && !bad; i++) skip(at, depth + 1);
            }
        } else {
            bad = true;
        }
    }
    // an integer of any integer type, or false (value skipped) otherwise
    bool uint_val(uint32_t t, uint64_t *out)
    {
        switch (t) {
        case GV_U8: { uint8_t v = 0; take(&v, 1); *out = v; return !bad; }
        case GV_U16: { uint16_t v = 0; take(&v, 2); *out = v; return !bad; }
        case GV_U32: { uint32_t v = 0; take(&v, 4); *out = v; return !bad; }
        case GV_U64: { take(out, 8); return !bad; }
        case GV_I32: { int32_t v = 0; take(&v, 4); *out = (uint64_t)(int64_t)v; return !bad; }
        case GV_I64: { int64_t v = 0; take(&v, 8); *out = (uint64_t)v; return !bad; }
        default: skip(t); return false;
        }
    }
};

// the architecture prefix of the metadata keys (gguf.c:150-153)
std::string strip_arch(const std::string &k)
{
    static const char *pre[] = {"qwen35moe.", "qwen35."};
    for (const char *p : pre)
        if (k.compare(0, strlen(p), p) == 0) return k.substr(strlen(p));
    return k;
}

const GgufTensor *find(const qmag_gguf *g, const std::string &name)
{
    auto it = g->by_name.find(name);
    return it == g->by_name.end() ? nullptr : &g->tensors[it->second];
}

int upload(const qmag_gguf *g, const GgufTensor *t, void **dptr)
{
    *dptr = nullptr;
    int st = qmag_malloc(dptr, t->nbytes);
    if (st) return st;
    st = qmag_h2d(*dptr, g->data + t->off, t->nbytes);
    if (st) {
        qmag_free(*dptr);
        *dptr = nullptr;
    }
    return st;
}

}  // namespace

extern "C" {

int qmag_gguf_open(const char *path, qmag_gguf **out)
{
    if (!path || !out) return err(QMAG_ERR_ARG, "gguf: null argument");
    *out = nullptr;
    auto *g = new qmag_gguf();
    auto fail_open = [&](int code) {
        qmag_gguf_close(g);
        return code;
    };
    g->fd = open(path, O_RDONLY);
    if (g->fd < 0) return fail_open(err(QMAG_ERR_ARG, "gguf: cannot open %s: %s", path, strerror(errno)));
    struct stat st;
    if (fstat(g->fd, &st) != 0 || st.st_size < 24) return fail_open(err(QMAG_ERR_ARG, "gguf: %s is too short", path));
    g->size = (size_t)st.st_size;
    void *m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) return fail_open(err(QMAG_ERR_ARG, "gguf: mmap of %s failed", path));
    g->map = (const uint8_t *)m;

    Reader r{g->map, g->map + g->size};
    char magic[4];
    r.take(magic, 4);
    if (memcmp(magic, "GGUF", 4) != 0) return fail_open(err(QMAG_ERR_ARG, "gguf: %s is not a GGUF file", path));
    const uint32_t version = r.u32();
    if (version < 2) return fail_open(err(QMAG_ERR_ARG, "gguf: version %u not supported", version));
    const uint64_t n_tensors = r.u64(), n_kv = r.u64();
    if (r.bad || n_tensors > (1u << 24) || n_kv > (1u << 24))
        return fail_open(err(QMAG_ERR_ARG, "gguf: corrupt header"));

    uint64_t alignment = 32;                                   // GGUF_DEFAULT_ALIGNMENT
    for (uint64_t i = 0; i < n_kv && !r.bad; i++) {
        const std::string key = strip_arch(r.str());
        const uint32_t t = r.u32();
        if (r.bad) break;
        uint64_t v = 0;
        if (t == GV_F32 || t == GV_F64 || t == GV_BOOL || t == GV_STR || t == GV_ARR) {
            r.skip(t);
        } else if (r.uint_val(t, &v)) {
            g->meta_u[key] = v;
            if (key == "general.alignment") alignment = v;
        }
    }
    if (r.bad) return fail_open(err(QMAG_ERR_ARG, "gguf: corrupt metadata"));
    if (alignment == 0 || alignment > 65536 || (alignment & (alignment - 1)))
        return fail_open(err(QMAG_ERR_ARG, "gguf: bad alignment %llu", (unsigned long long)alignment));

    // an entry takes at least 32 bytes of the file (name length, dims count,
    // one dim, type, offset): a corrupt count reserves no more than that allows
    g->tensors.reserve((size_t)std::min<uint64_t>(n_tensors, (uint64_t)(r.end - r.p) / 32));
    for (uint64_t i = 0; i < n_tensors && !r.bad; i++) {
        GgufTensor t;
        t.name = r.str();
        const uint32_t nd = r.u32();
        if (nd == 0 || nd > 4) {
            r.bad = true;
            break;
        }
        int64_t dims[4] = {1, 1, 1, 1};
        for (uint32_t d = 0; d < nd; d++) dims[d] = (int64_t)r.u64();
        t.type = (int)r.u32();
        t.off = r.u64();
        if (dims[3] != 1) return fail_open(err(QMAG_ERR_ARG, "gguf: tensor %s has 4 dimensions", t.name.c_str()));
        for (int d = 0; d < 3; d++) {
            if (dims[d] <= 0 || dims[d] > ((int64_t)1 << 40))
                return fail_open(err(QMAG_ERR_ARG, "gguf: tensor %s has a bad dimension", t.name.c_str()));
            t.ne[d] = dims[d];
        }
        g->tensors.push_back(t);
    }
    if (r.bad) return fail_open(err(QMAG_ERR_ARG, "gguf: corrupt tensor info"));
    // the data section starts aligned after the tensor table (gguf.c:254-262)
    const size_t pos = (size_t)(r.p - g->map);
    const size_t data_off = (pos + alignment - 1) / alignment * alignment;
    if (data_off > g->size) return fail_open(err(QMAG_ERR_ARG, "gguf: truncated before the data section"));
    g->data = g->map + data_off;
    const size_t data_size = g->size - data_off;
    for (size_t i = 0; i < g->tensors.size(); i++) {
        GgufTensor &t = g->tensors[i];
        size_t bs, blk;
        switch (t.type) {                                      // gguf.c:264-283
        case T_F32: bs = 4; blk = 1; break;
        case T_Q4K: bs = 144; blk = QK_K_ELEMS; break;
        case T_Q6K: bs = 210; blk = QK_K_ELEMS; break;
        default: return fail_open(err(QMAG_ERR_ARG, "gguf: tensor %s: unsupported type %d", t.name.c_str(), t.type));
        }
        if (t.ne[0] % (int64_t)blk != 0)
            return fail_open(err(QMAG_ERR_ARG, "gguf: tensor %s: ne0 not block multiple", t.name.c_str()));
        // (each dimension is below 2^40, so the product can overflow: a
        // wrapped size would pass the range check below with shapes that
        // name more bytes than are uploaded)
        size_t nb = 0;
        if (__builtin_mul_overflow((size_t)(t.ne[0] / (int64_t)blk), bs, &nb) ||
            __builtin_mul_overflow(nb, (size_t)t.ne[1], &nb) || __builtin_mul_overflow(nb, (size_t)t.ne[2], &nb))
            return fail_open(err(QMAG_ERR_ARG, "gguf: tensor %s is too large", t.name.c_str()));
        t.nbytes = nb;
        if (t.off > data_size || t.nbytes > data_size - t.off)
            return fail_open(err(QMAG_ERR_ARG, "gguf: tensor %s out of file range", t.name.c_str()));
        if (!g->by_name.emplace(t.name, i).second)
            return fail_open(err(QMAG_ERR_ARG, "gguf: duplicate tensor %s", t.name.c_str()));
    }
    *out = g;
    return QMAG_OK;
}

void qmag_gguf_close(qmag_gguf *g)
{
    if (!g) return;
    if (g->map) munmap((void *)g->map, g->size);
    if (g->fd >= 0) close(g->fd);
    delete g;
}

int qmag_gguf_meta_u64(const qmag_gguf *g, const char *key, uint64_t *val)
{
    if (!g || !key || !val) return err(QMAG_ERR_ARG, "gguf: null argument");
    auto it = g->meta_u.find(strip_arch(key));
    if (it == g->meta_u.end()) return err(QMAG_ERR_ARG, "gguf: no integer metadata %s", key);
    *val = it->second;
    return QMAG_OK;
}

int qmag_gguf_tensor(const qmag_gguf *g, const char *name, int *type, int64_t ne[3], const void **data,
                     size_t *nbytes)
{
    if (!g || !name) return err(QMAG_ERR_ARG, "gguf: null argument");
    const GgufTensor *t = find(g, name);
    if (!t) return err(QMAG_ERR_ARG, "gguf: missing tensor: %s", name);
    if (type) *type = t->type;
    if (ne)
        for (int d = 0; d < 3; d++) ne[d] = t->ne[d];
    if (data) *data = g->data + t->off;
    if (nbytes) *nbytes = t->nbytes;
    return QMAG_OK;
}

int qmag_gguf_upload_tensor(const qmag_gguf *g, const char *name, void **dptr, int *type, int64_t ne[3])
{
    if (!g || !name || !dptr) return err(QMAG_ERR_ARG, "gguf: null argument");
    const GgufTensor *t = find(g, name);
    if (!t) return err(QMAG_ERR_ARG, "gguf: missing tensor: %s", name);
    if (type) *type = t->type;
    if (ne)
        for (int d = 0; d < 3; d++) ne[d] = t->ne[d];
    return upload(g, t, dptr);
}

int qmag_gguf_upload_moe_layer(const qmag_gguf *g, int il, qmag_moe_layer *L)
{
    if (!g || !L || il < 0) return err(QMAG_ERR_ARG, "gguf: bad argument");
    memset(L, 0, sizeof(*L));
    // the per-layer MoE FFN tensors (gguf.c:318-326)
    static const char *names[] = {"ffn_gate_inp", "ffn_gate_exps", "ffn_up_exps", "ffn_down_exps",
                                  "ffn_gate_inp_shexp", "ffn_gate_shexp", "ffn_up_shexp", "ffn_down_shexp"};
    const GgufTensor *t[8];
    for (int i = 0; i < 8; i++) {
        const std::string nm = "blk." + std::to_string(il) + "." + names[i] + ".weight";
        t[i] = find(g, nm);
        if (!t[i]) return err(QMAG_ERR_ARG, "gguf: missing tensor: %s", nm.c_str());
    }
    const int64_t N = t[1]->ne[0], F = t[1]->ne[1], E = t[1]->ne[2];
    auto shape = [&](int i, int ty0, int ty1, int64_t a, int64_t b, int64_t c) {
        const GgufTensor &x = *t[i];
        return (x.type == ty0 || x.type == ty1) && x.ne[0] == a && x.ne[1] == b && x.ne[2] == c;
    };
    // types: f32 router and shared gate; Q4_K gate/up (the kernels' operand);
    // Q4_K or Q6_K down (varies per layer, qma.h:206, 212)
    if (!shape(0, T_F32, T_F32, N, E, 1) || !shape(1, T_Q4K, T_Q4K, N, F, E) || !shape(2, T_Q4K, T_Q4K, N, F, E) ||
        !shape(3, T_Q4K, T_Q6K, F, N, E) || !shape(4, T_F32, T_F32, N, 1, 1) ||
        !shape(5, T_Q4K, T_Q4K, N, F, 1) || !shape(6, T_Q4K, T_Q4K, N, F, 1) || !shape(7, T_Q4K, T_Q6K, F, N, 1))
        return err(QMAG_ERR_ARG,
                   "gguf: layer %d MoE tensors have unexpected types or shapes (gate_exps %lld x %lld x %lld); "
                   "the expert and shared hidden sizes must be equal",
                   il, (long long)N, (long long)F, (long long)E);
    uint64_t used = 8;                                         // N_EXPERT_USED, qma.h:58
    auto it = g->meta_u.find("expert_used_count");
    if (it != g->meta_u.end()) used = it->second;
    if (used < 1 || (int64_t)used > E || E > 256 || N > 8192 || F > 8192)
        return err(QMAG_ERR_ARG, "gguf: layer %d: %llu of %lld experts per token not supported", il,
                   (unsigned long long)used, (long long)E);
    L->n_embd = (int)N;
    L->n_ff = (int)F;
    L->n_expert = (int)E;
    L->n_used = (int)used;
    L->t_down_exps = t[3]->type;
    L->t_down_shexp = t[7]->type;
    void *p[8] = {};
    for (int i = 0; i < 8; i++) {
        const int st = upload(g, t[i], &p[i]);
        if (st) {
            for (int k = 0; k < i; k++) qmag_free(p[k]);
            memset(L, 0, sizeof(*L));
            return st;
        }
    }
    L->gate_inp = (const float *)p[0];
    L->gate_exps = p[1];
    L->up_exps = p[2];
    L->down_exps = p[3];
    L->gate_inp_shexp = (const float *)p[4];
    L->gate_shexp = p[5];
    L->up_shexp = p[6];
    L->down_shexp = p[7];
    L->router_bias = nullptr;                                  // the reference has none
    return QMAG_OK;
}

// One expert's record from the mapping: its gate, up and down slabs back to
// back (the layout expert_fetch, nn.c:1564-1595, preads into the cache).
static int expert_slabs(const qmag_gguf *g, int layer, int expert, const GgufTensor *t[3])
{
    static const char *names[] = {"ffn_gate_exps", "ffn_up_exps", "ffn_down_exps"};
    for (int i = 0; i < 3; i++) {
        const std::string nm = "blk." + std::to_string(layer) + "." + names[i] + ".weight";
        t[i] = find(g, nm);
        if (!t[i] || t[i]->ne[2] <= 0) return -1;
    }
    if (expert < 0 || expert >= t[0]->ne[2] || t[1]->ne[2] != t[0]->ne[2] || t[2]->ne[2] != t[0]->ne[2]) return -1;
    return 0;
}

int qmag_gguf_fetch_expert(void *user, int layer, int expert, uint8_t *dst)
{
    const qmag_gguf *g = (const qmag_gguf *)user;
    const GgufTensor *t[3];
    if (!g || !dst || layer < 0 || expert_slabs(g, layer, expert, t)) return -1;
    for (int i = 0; i < 3; i++) {
        const size_t slab = t[i]->nbytes / (size_t)t[i]->ne[2];
        memcpy(dst, g->data + t[i]->off + (size_t)expert * slab, slab);
        dst += slab;
    }
    return 0;
}

int qmag_gguf_expert_record_bytes(const qmag_gguf *g, size_t *rec)
{
    // The largest layer's record (nn.c:1601-1605): down types vary per
    // layer.  Every blk.N.ffn_{gate,up,down}_exps tensor of the table counts,
    // wherever its layer lies (a gap in the layer numbers does not end the
    // scan), and a layer with only part of the triple fails the query: the
    // fetch callback copies whatever the table holds, so the bound must cover
    // every layer it can be asked for.
    if (!g || !rec) return err(QMAG_ERR_ARG, "gguf: bad argument");
    static const char *const kinds[] = {".ffn_gate_exps.weight", ".ffn_up_exps.weight", ".ffn_down_exps.weight"};
    std::unordered_map<long, int> seen;          // layer -> bit mask of the kinds present
    for (const GgufTensor &t : g->tensors) {
        if (t.name.compare(0, 4, "blk.") != 0) continue;
        const size_t dot = t.name.find('.', 4);
        if (dot == std::string::npos || dot == 4 || dot > 13) continue;
        long il = 0;
        bool digits = true;
        for (size_t i = 4; i < dot; i++) {
            if (t.name[i] < '0' || t.name[i] > '9') digits = false;
            else il = il * 10 + (t.name[i] - '0');
        }
        if (!digits) continue;
        for (int k = 0; k < 3; k++)
            if (t.name.compare(dot, std::string::npos, kinds[k]) == 0) seen[il] |= 1 << k;
    }
    size_t best = 0;
    for (const auto &kv : seen) {
        if (kv.second != 7 || kv.first > INT32_MAX)
            return err(QMAG_ERR_ARG, "gguf: layer %ld has an incomplete expert tensor triple (gate/up/down mask %d)",
                       kv.first, kv.second);
        const GgufTensor *t[3];
        if (expert_slabs(g, (int)kv.first, 0, t))
            return err(QMAG_ERR_ARG, "gguf: layer %ld expert tensors disagree on the expert count", kv.first);
        size_t r = 0;
        for (int i = 0; i < 3; i++) r += t[i]->nbytes / (size_t)t[i]->ne[2];
        if (r > best) best = r;
    }
    if (!best) return err(QMAG_ERR_ARG, "gguf: no expert tensors");
    *rec = best;
    return QMAG_OK;
}

int qmag_gguf_free_moe_layer(qmag_moe_layer *L)
{
    if (!L) return err(QMAG_ERR_ARG, "gguf: null layer");
    const void *p[] = {L->gate_inp, L->gate_exps, L->up_exps, L->down_exps, L->gate_inp_shexp, L->gate_shexp,
                       L->up_shexp, L->down_shexp};
    int st = QMAG_OK;
    for (const void *q : p)
        if (q) {
            const int s = qmag_free((void *)q);
            if (s && !st) st = s;
        }
    memset(L, 0, sizeof(*L));
    return st;
}

}  // extern "C"
