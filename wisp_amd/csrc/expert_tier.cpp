/*
 * expert_tier.cpp — VRAM tier of the expert cache (host side, C++).
 *
 * Restates the reference's tier policy (csrc/core/wisp_engine.c:1138-1296,
 * wisp_expert_fetch; csrc/core/lru_cache.c:26-229) for the case the MI355X
 * build targets: every expert blob already sits in pinned host memory (the
 * RAM tier holds all of them), and a fixed number of VRAM slots caches the
 * hot ones.
 *
 *   first touch of an expert (the reference's SSD miss, :1205-1295): it
 *       takes a VRAM slot only if one is free, else it is served through
 *       the scratch ring; its RAM-tier hit count starts at 0
 *   VRAM hit (:1140-1148): move to the MRU end
 *   RAM hit (:1150-1203): hits++; below promote_hits (WISP_PROMOTE_HITS = 3,
 *       csrc/core/wisp_engine.h:219) it is served through the scratch ring,
 *       else it is promoted into a VRAM slot, evicting the LRU tail
 *   scratch ring (:1113-1132, sized top_k + 2 at :2122-2131): round-robin
 *       device buffers, one H2D copy, no cache insertion
 *
 * Differences, on purpose:
 *   - keys are the dense (layer, expert) space, so the LRU is an intrusive
 *     list over a flat node array (O(1) without hashing);
 *   - VRAM slots are one slab allocated up front (the reference allocates
 *     and frees device memory per promotion, mem_pool.c:138-181);
 *   - an evicted expert needs no copy back: the pinned RAM tier keeps
 *     every blob (the reference copies the victim to RAM, :1084-1094);
 *   - experts resolved for the layer being assembled are never evicted by
 *     a later lookup of the same layer (in the reference such an eviction
 *     frees a pointer the layer is about to use);
 *   - copies are asynchronous on a side stream (the reference synchronises
 *     after every copy, :1181-1187), ordered by events: compute waits for
 *     the copies it needs, a copy into a slot waits for the kernels that
 *     last read it.
 *   - one owner thread; no locks (the reference's locks leave races, e.g.
 *     lru_get returns a node after unlocking, lru_cache.c:133-138).
 */
#include <stdlib.h>
#include <string.h>

#include <new>
#include <string>
#include <thread>
#include <vector>

#include "../../include/wisp_amd.h"

#define WISP_TIER_MAX_PAIRS 256   /* n_tokens * top_k of one decode layer (4 x 64) */
#define WISP_TIER_MAX_EXPERTS 1024 /* experts per layer: the decode kernels' limit */

namespace {

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

struct Node {
    int slot = -1;       /* VRAM slot, -1 when not resident */
    int ram = -1;        /* RAM slot (bounded RAM tier), -1 when not in RAM */
    uint32_t hits = 0;   /* RAM-tier hits (promotion counter) */
    bool touched = false;   /* unbounded RAM tier: seen once, so in RAM for good */
    int prev = -1, next = -1;     /* VRAM recency list, MRU at head */
    int rprev = -1, rnext = -1;   /* RAM recency list (bounded tier) */
    uint64_t epoch = 0;           /* layer assembly that last resolved it */
    uint64_t ram_epoch = 0;       /* layer assembly whose copies use its RAM slot */
};

/* What one lookup asks the executor to do besides the path. */
struct Action {
    int slot = -1;          /* VRAM slot or scratch index                   */
    int victim = -1;        /* node evicted from VRAM by a promotion         */
    int ram = -1;           /* RAM slot holding the expert (bounded tier)    */
    bool read_file = false; /* SSD miss: the file must be read into `ram`    */
    int victim_ram = -1;    /* RAM slot the VRAM victim is copied back into  */
};

struct Policy {
    int L, E, n_slots, n_scratch, promote_hits;
    int n_ram;               /* RAM slots; < 0: every expert is in RAM (pinned) */
    std::vector<Node> nodes;
    std::vector<int> free_slots, free_ram;
    int head = -1, tail = -1;
    int rhead = -1, rtail = -1, ram_count = 0;
    int scratch_pos = 0;
    uint64_t epoch = 1;
    uint64_t stats[WISP_TIER_N_STATS] = {0};

    Policy(int l, int e, int s, int sc, int ph, int nr = -1)
        : L(l), E(e), n_slots(s), n_scratch(sc), promote_hits(ph), n_ram(nr), nodes((size_t)l * e) {
        for (int i = s - 1; i >= 0; i--) free_slots.push_back(i);
        for (int i = nr - 1; i >= 0; i--) free_ram.push_back(i);
    }
    bool bounded() const { return n_ram >= 0; }
    bool in_ram(int k) const { return bounded() ? nodes[k].ram >= 0 : nodes[k].touched; }
    void unlink(int k) {
        Node& n = nodes[k];
        if (n.prev >= 0) nodes[n.prev].next = n.next; else head = n.next;
        if (n.next >= 0) nodes[n.next].prev = n.prev; else tail = n.prev;
        n.prev = n.next = -1;
    }
    void push_front(int k) {
        Node& n = nodes[k];
        n.prev = -1;
        n.next = head;
        if (head >= 0) nodes[head].prev = k;
        head = k;
        if (tail < 0) tail = k;
    }
    void ram_unlink(int k) {
        Node& n = nodes[k];
        if (n.rprev >= 0) nodes[n.rprev].rnext = n.rnext; else rhead = n.rnext;
        if (n.rnext >= 0) nodes[n.rnext].rprev = n.rprev; else rtail = n.rprev;
        n.rprev = n.rnext = -1;
    }
    void ram_push_front(int k) {
        Node& n = nodes[k];
        n.rprev = -1;
        n.rnext = rhead;
        if (rhead >= 0) nodes[rhead].rprev = k;
        rhead = k;
        if (rtail < 0) rtail = k;
    }
    /* The reference's ram_put_evicting (csrc/core/wisp_engine.c:1053-1068):
     * while one more blob would overflow the RAM tier, drop the LRU entry
     * (its hit count goes with it), then insert k or refresh its recency.
     * Entries whose RAM slot a copy of the layer being assembled uses are
     * skipped (the copy may still be pending; the reference has no such
     * case because it copies synchronously). Returns true when k took a new
     * RAM slot (its bytes must be written there). */
    bool ram_put(int k) {
        while (ram_count + 1 > n_ram) {
            int v = rtail;
            while (v >= 0 && nodes[v].ram_epoch == epoch) v = nodes[v].rprev;
            if (v < 0) break;
            ram_unlink(v);
            free_ram.push_back(nodes[v].ram);
            nodes[v].ram = -1;
            nodes[v].hits = 0;
            ram_count--;
            stats[WISP_TIER_RAM_EVICTIONS]++;
        }
        Node& n = nodes[k];
        if (n.ram >= 0) {
            ram_unlink(k);
            ram_push_front(k);
            return false;
        }
        if (free_ram.empty()) return false;   /* not reachable: n_ram > scratch slots */
        n.ram = free_ram.back();
        free_ram.pop_back();
        n.hits = 0;
        ram_push_front(k);
        ram_count++;
        return true;
    }
    int next_scratch() {
        const int s = scratch_pos;
        scratch_pos = (scratch_pos + 1) % n_scratch;
        stats[WISP_TIER_SCRATCH_SERVES]++;
        return s;
    }
    /* least recently used resident expert not pinned by this layer */
    int victim() const {
        for (int k = tail; k >= 0; k = nodes[k].prev)
            if (nodes[k].epoch != epoch) return k;
        return -1;
    }
    int lookup(int layer, int expert, Action& a) {
        const int k = layer * E + expert;
        Node& n = nodes[k];
        a = Action();
        stats[WISP_TIER_LOOKUPS]++;
        n.epoch = epoch;
        if (n.slot >= 0) {
            stats[WISP_TIER_VRAM_HITS]++;
            unlink(k);
            push_front(k);
            a.slot = n.slot;
            a.ram = n.ram;
            return WISP_TIER_VRAM_HIT;
        }
        if (in_ram(k)) {
            stats[WISP_TIER_RAM_HITS]++;
            if (bounded()) {
                ram_unlink(k);
                ram_push_front(k);
                n.ram_epoch = epoch;   /* a copy of this layer reads its RAM slot */
            }
            a.ram = n.ram;
            n.hits++;
            if (n.hits < (uint32_t)promote_hits) {
                a.slot = next_scratch();
                return WISP_TIER_RAM_SCRATCH;
            }
            int s = -1;
            if (!free_slots.empty()) {
                s = free_slots.back();
                free_slots.pop_back();
            } else {
                const int v = victim();
                if (v < 0) {   /* every slot holds an expert of this layer */
                    a.slot = next_scratch();
                    return WISP_TIER_RAM_SCRATCH;
                }
                unlink(v);
                s = nodes[v].slot;
                nodes[v].slot = -1;
                a.victim = v;
                stats[WISP_TIER_EVICTIONS]++;
                /* the victim goes back to the RAM tier (:1084-1094); while
                 * its copy is pending it stays there for this layer */
                if (bounded() && ram_put(v)) {
                    a.victim_ram = nodes[v].ram;
                    nodes[v].ram_epoch = epoch;
                }
            }
            n.slot = s;
            push_front(k);
            stats[WISP_TIER_PROMOTIONS]++;
            a.slot = s;
            return WISP_TIER_RAM_PROMOTE;
        }
        /* SSD miss (first touch, or back after a RAM eviction): into the
         * RAM tier with a hit count of 0 (:1205-1241), then a VRAM slot
         * only if one is free (:1250-1258), else the scratch ring */
        n.touched = true;
        n.hits = 0;
        stats[WISP_TIER_FIRST_TOUCH]++;
        if (bounded()) {
            ram_put(k);
            n.ram_epoch = epoch;
            a.ram = n.ram;
            a.read_file = true;
        }
        if (!free_slots.empty()) {
            const int s = free_slots.back();
            free_slots.pop_back();
            n.slot = s;
            push_front(k);
            a.slot = s;
            return WISP_TIER_COLD_VRAM;
        }
        a.slot = next_scratch();
        return WISP_TIER_COLD_SCRATCH;
    }
};

}  // namespace

struct WispTierPolicy {
    Policy p;
    WispTierPolicy(int l, int e, int s, int sc, int ph, int nr = -1) : p(l, e, s, sc, ph, nr) {}
};

extern "C" WispTierPolicy* wisp_tier_policy_create(int n_layers, int n_experts, int n_slots,
                                                   int scratch_slots, int promote_hits) {
    if (n_layers < 1 || n_experts < 1 || n_slots < 0 || scratch_slots < 1 || promote_hits < 1 ||
        (long)n_layers * n_experts > (1L << 30))
        return nullptr;
    return new (std::nothrow) WispTierPolicy(n_layers, n_experts, n_slots, scratch_slots,
                                             promote_hits);
}

extern "C" WispTierPolicy* wisp_tier_policy_create_ram(int n_layers, int n_experts, int n_ram_slots,
                                                       int n_slots, int scratch_slots,
                                                       int promote_hits) {
    if (n_layers < 1 || n_experts < 1 || n_slots < 0 || scratch_slots < 1 || promote_hits < 1 ||
        n_ram_slots <= scratch_slots || (long)n_layers * n_experts > (1L << 30))
        return nullptr;
    return new (std::nothrow) WispTierPolicy(n_layers, n_experts, n_slots, scratch_slots,
                                             promote_hits, n_ram_slots);
}

extern "C" void wisp_tier_policy_destroy(WispTierPolicy* t) { delete t; }

extern "C" void wisp_tier_policy_begin_layer(WispTierPolicy* t) {
    if (t) t->p.epoch++;
}

extern "C" int wisp_tier_policy_lookup(WispTierPolicy* t, int layer, int expert, int* slot,
                                       int* victim_layer, int* victim_expert) {
    if (!t || !slot || layer < 0 || layer >= t->p.L || expert < 0 || expert >= t->p.E) return -1;
    Action a;
    const int path = t->p.lookup(layer, expert, a);
    *slot = a.slot;
    const int v = a.victim;
    if (victim_layer) *victim_layer = v >= 0 ? v / t->p.E : -1;
    if (victim_expert) *victim_expert = v >= 0 ? v % t->p.E : -1;
    return path;
}

extern "C" void wisp_tier_policy_stats(const WispTierPolicy* t, uint64_t* out) {
    if (!t || !out) return;
    for (int i = 0; i < WISP_TIER_N_STATS; i++) out[i] = t->p.stats[i];
}

/* ======================================================================= */
/* executor                                                                 */
/* ======================================================================= */

struct WispExpertTier {
    Policy pol;
    size_t blob_bytes = 0, stride = 0;
    std::vector<const void*> host;     /* [L * E] pinned host blob pointers */
    /* bounded RAM tier over expert files (wisp_tier_create_ssd) */
    std::string model_path;
    uint8_t* h_ram = nullptr;          /* pinned slab, n_ram * ram_stride     */
    size_t ram_stride = 0;
    std::vector<hipEvent_t> ram_ev;    /* last copy that read or wrote a RAM slot */
    std::vector<char> ram_ev_set;
    uint64_t stats_ssd_bytes = 0, stats_d2h_bytes = 0;
    uint8_t* d_slots = nullptr;        /* n_slots * stride                  */
    uint8_t* d_scratch = nullptr;      /* n_scratch * stride                */
    void** h_table = nullptr;          /* pinned [L][E] device blob pointers */
    void** d_table = nullptr;          /* device copy                       */
    hipStream_t copy = nullptr;
    hipEvent_t copies_done = nullptr;
    std::vector<hipEvent_t> slot_ev, scratch_ev;   /* last reader of a slot */
    std::vector<char> slot_ev_set, scratch_ev_set;
    std::vector<int> used_slots, used_scratch;     /* this layer             */
    /* per layer: the last copy of that layer's pinned rows (table, routing)
     * on `compute`; the host waits for it before rewriting the rows */
    std::vector<hipEvent_t> row_ev;
    std::vector<char> row_ev_set;
    bool pending_copies = false;
    uint64_t stats_h2d_bytes = 0;
    /* pinned staging for the routing arrays of wisp_tier_moe_decode_layer:
     * [n_layers][3][WISP_TIER_MAX_PAIRS] (hits-only ids, copied-only ids,
     * weights), one row per layer so a pending copy is never overwritten
     * before the next use of the same layer */
    int* h_route = nullptr;
    int* d_route = nullptr;

    WispExpertTier(int l, int e, int s, int sc, int ph, int nr = -1) : pol(l, e, s, sc, ph, nr) {}
    bool ssd() const { return pol.bounded(); }
    const void* blob_src(int key) const {
        return ssd() ? (const void*)(h_ram + (size_t)pol.nodes[key].ram * ram_stride) : host[key];
    }
};

static void tier_free(WispExpertTier* t) {
    if (!t) return;
    if (t->copy) (void)hipStreamSynchronize(t->copy);
    for (hipEvent_t ev : t->slot_ev) if (ev) (void)hipEventDestroy(ev);
    for (hipEvent_t ev : t->scratch_ev) if (ev) (void)hipEventDestroy(ev);
    for (hipEvent_t ev : t->row_ev) if (ev) (void)hipEventDestroy(ev);
    for (hipEvent_t ev : t->ram_ev) if (ev) (void)hipEventDestroy(ev);
    if (t->h_ram) (void)hipHostFree(t->h_ram);
    if (t->copies_done) (void)hipEventDestroy(t->copies_done);
    if (t->copy) (void)hipStreamDestroy(t->copy);
    if (t->d_slots) (void)hipFree(t->d_slots);
    if (t->d_scratch) (void)hipFree(t->d_scratch);
    if (t->d_table) (void)hipFree(t->d_table);
    if (t->h_table) (void)hipHostFree(t->h_table);
    if (t->h_route) (void)hipHostFree(t->h_route);
    if (t->d_route) (void)hipFree(t->d_route);
    delete t;
}

/* Device slots, tables, stream and events of a tier whose policy and
 * blob size are set. */
static hipError_t tier_init_device(WispExpertTier* t, int n_layers, int n_slots,
                                   int scratch_slots) {
    const size_t n = (size_t)n_layers * t->pol.E;
    hipError_t e = hipSuccess;
    /* blob at slot + 8: the 120-byte header then leaves every section
     * 16-byte aligned (what the fused kernels need) */
    t->stride = align_up(t->blob_bytes + 8, 4096);
    if (n_slots > 0) e = hipMalloc((void**)&t->d_slots, t->stride * n_slots);
    if (e == hipSuccess) e = hipMalloc((void**)&t->d_scratch, t->stride * scratch_slots);
    if (e == hipSuccess) e = hipHostMalloc((void**)&t->h_table, n * sizeof(void*), 0);
    if (e == hipSuccess) e = hipMalloc((void**)&t->d_table, n * sizeof(void*));
    if (e == hipSuccess)
        e = hipHostMalloc((void**)&t->h_route,
                          (size_t)n_layers * 3 * WISP_TIER_MAX_PAIRS * sizeof(int), 0);
    if (e == hipSuccess)
        e = hipMalloc((void**)&t->d_route, (size_t)n_layers * 3 * WISP_TIER_MAX_PAIRS * sizeof(int));
    if (e == hipSuccess) e = hipStreamCreate(&t->copy);   /* default priority */
    if (e == hipSuccess) e = hipEventCreateWithFlags(&t->copies_done, hipEventDisableTiming);
    t->slot_ev.assign(n_slots, nullptr);
    t->scratch_ev.assign(scratch_slots, nullptr);
    t->slot_ev_set.assign(n_slots, 0);
    t->scratch_ev_set.assign(scratch_slots, 0);
    for (int i = 0; i < n_slots && e == hipSuccess; i++)
        e = hipEventCreateWithFlags(&t->slot_ev[i], hipEventDisableTiming);
    for (int i = 0; i < scratch_slots && e == hipSuccess; i++)
        e = hipEventCreateWithFlags(&t->scratch_ev[i], hipEventDisableTiming);
    t->row_ev.assign(n_layers, nullptr);
    t->row_ev_set.assign(n_layers, 0);
    for (int i = 0; i < n_layers && e == hipSuccess; i++)
        e = hipEventCreateWithFlags(&t->row_ev[i], hipEventDisableTiming);
    if (e == hipSuccess) {
        memset(t->h_table, 0, n * sizeof(void*));
        e = hipMemset(t->d_table, 0, n * sizeof(void*));
    }
    return e;
}

static bool tier_args_ok(int n_layers, int n_experts, size_t blob_bytes, int n_slots,
                         int scratch_slots, int promote_hits) {
    return n_layers >= 1 && n_experts >= 1 && blob_bytes > 0 && n_slots >= 0 &&
           scratch_slots >= 1 && promote_hits >= 1 && n_experts <= WISP_TIER_MAX_EXPERTS &&
           (long)n_layers * n_experts <= (1L << 24);
}

extern "C" WispExpertTier* wisp_tier_create(int n_layers, int n_experts, size_t blob_bytes,
                                            const void* const* host_blobs, int n_slots,
                                            int scratch_slots, int promote_hits,
                                            hipError_t* err) {
    hipError_t e = hipErrorInvalidValue;
    WispExpertTier* t = nullptr;
    if (host_blobs &&
        tier_args_ok(n_layers, n_experts, blob_bytes, n_slots, scratch_slots, promote_hits)) {
        t = new (std::nothrow) WispExpertTier(n_layers, n_experts, n_slots, scratch_slots,
                                              promote_hits);
        e = t ? hipSuccess : hipErrorOutOfMemory;
    }
    if (t) {
        const size_t n = (size_t)n_layers * n_experts;
        t->blob_bytes = blob_bytes;
        t->host.assign(host_blobs, host_blobs + n);
        for (size_t i = 0; i < n && e == hipSuccess; i++)
            if (!t->host[i]) e = hipErrorInvalidValue;
        if (e == hipSuccess) e = tier_init_device(t, n_layers, n_slots, scratch_slots);
        if (e != hipSuccess) {
            tier_free(t);
            t = nullptr;
        }
    }
    if (err) *err = e;
    return t;
}

extern "C" WispExpertTier* wisp_tier_create_ssd(int n_layers, int n_experts, size_t blob_bytes,
                                                const char* model_path, int n_ram_slots,
                                                int n_slots, int scratch_slots, int promote_hits,
                                                hipError_t* err) {
    hipError_t e = hipErrorInvalidValue;
    WispExpertTier* t = nullptr;
    if (model_path && n_ram_slots > scratch_slots &&
        tier_args_ok(n_layers, n_experts, blob_bytes, n_slots, scratch_slots, promote_hits)) {
        t = new (std::nothrow) WispExpertTier(n_layers, n_experts, n_slots, scratch_slots,
                                              promote_hits, n_ram_slots);
        e = t ? hipSuccess : hipErrorOutOfMemory;
    }
    if (t) {
        t->blob_bytes = blob_bytes;
        t->model_path = model_path;
        t->ram_stride = align_up(blob_bytes, 4096);
        e = hipHostMalloc((void**)&t->h_ram, t->ram_stride * (size_t)n_ram_slots, 0);
        t->ram_ev.assign(n_ram_slots, nullptr);
        t->ram_ev_set.assign(n_ram_slots, 0);
        for (int i = 0; i < n_ram_slots && e == hipSuccess; i++)
            e = hipEventCreateWithFlags(&t->ram_ev[i], hipEventDisableTiming);
        if (e == hipSuccess) e = tier_init_device(t, n_layers, n_slots, scratch_slots);
        if (e != hipSuccess) {
            tier_free(t);
            t = nullptr;
        }
    }
    if (err) *err = e;
    return t;
}

extern "C" void wisp_tier_destroy(WispExpertTier* t) { tier_free(t); }

extern "C" void** wisp_tier_device_table(WispExpertTier* t, int layer) {
    if (!t || layer < 0 || layer >= t->pol.L) return nullptr;
    return t->d_table + (size_t)layer * t->pol.E;
}

/* Reads the expert file of (layer, expert) into RAM slot `ram` (the
 * caller has waited for the slot's last copy). */
static hipError_t tier_read_file(WispExpertTier* t, int layer, int expert, int ram) {
    const int64_t got = wisp_expert_file_read(t->model_path.c_str(), (uint32_t)layer,
                                              (uint32_t)expert, t->h_ram + (size_t)ram * t->ram_stride,
                                              t->ram_stride);
    return got == (int64_t)t->blob_bytes ? hipSuccess : hipErrorFileNotFound;
}

extern "C" hipError_t wisp_tier_fetch_layer(WispExpertTier* t, int layer,
                                            const int* expert_ids, int n, int* out_path,
                                            hipStream_t compute) {
    if (!t || layer < 0 || layer >= t->pol.L || n < 0 || (n > 0 && !expert_ids))
        return hipErrorInvalidValue;
    Policy& P = t->pol;
    hipError_t e = hipSuccess;
    /* every expert of the layer may ride the scratch ring at once: it must
     * not wrap within one layer */
    int n_valid = 0;
    for (int i = 0; i < n; i++) n_valid += expert_ids[i] >= 0 && expert_ids[i] < P.E;
    if (n_valid > P.n_scratch) return hipErrorInvalidValue;
    /* the previous copies of this layer's pinned rows must have run */
    if (t->row_ev_set[layer]) {
        e = hipEventSynchronize(t->row_ev[layer]);
        if (e != hipSuccess) return e;
    }
    P.epoch++;
    t->used_slots.clear();
    t->used_scratch.clear();
    t->pending_copies = false;
    /* 1. policy: paths, slots and the RAM-tier work */
    struct Item {
        int id, path;
        Action a;
    };
    std::vector<Item> items;
    for (int i = 0; i < n; i++) {
        const int id = expert_ids[i];
        if (id < 0 || id >= P.E) {
            if (out_path) out_path[i] = -1;
            continue;
        }
        Item it;
        it.id = id;
        it.path = P.lookup(layer, id, it.a);
        if (out_path) out_path[i] = it.path;
        items.push_back(it);
    }
    /* 2. expert files of the SSD misses into their RAM slots, in parallel;
     * each slot's earlier copies must have run first */
    std::vector<int> reads;
    for (int i = 0; i < (int)items.size(); i++)
        if (items[i].a.read_file) reads.push_back(i);
    for (int i : reads) {
        const int r = items[i].a.ram;
        if (e == hipSuccess && t->ram_ev_set[r]) e = hipEventSynchronize(t->ram_ev[r]);
    }
    if (e == hipSuccess && !reads.empty()) {
        std::vector<hipError_t> res(reads.size(), hipSuccess);
        std::vector<std::thread> pool;
        for (size_t q = 1; q < reads.size(); q++)
            pool.emplace_back([&, q]() {
                res[q] = tier_read_file(t, layer, items[reads[q]].id, items[reads[q]].a.ram);
            });
        res[0] = tier_read_file(t, layer, items[reads[0]].id, items[reads[0]].a.ram);
        for (auto& th : pool) th.join();
        for (hipError_t r : res)
            if (r != hipSuccess) e = r;
        if (e == hipSuccess) t->stats_ssd_bytes += reads.size() * t->blob_bytes;
    }
    /* 3. copies on the tier's stream, in lookup order */
    for (const Item& it : items) {
        if (e != hipSuccess) break;
        const int slot = it.a.slot;
        const bool scratch =
            it.path == WISP_TIER_RAM_SCRATCH || it.path == WISP_TIER_COLD_SCRATCH;
        uint8_t* base = scratch ? t->d_scratch + (size_t)slot * t->stride
                                : t->d_slots + (size_t)slot * t->stride;
        if (it.path != WISP_TIER_VRAM_HIT) {
            if (it.a.victim_ram >= 0) {
                /* the evicted expert's bytes go back to RAM before the slot
                 * is overwritten (same stream) */
                e = hipMemcpyAsync(t->h_ram + (size_t)it.a.victim_ram * t->ram_stride, base + 8,
                                   t->blob_bytes, hipMemcpyDeviceToHost, t->copy);
                if (e == hipSuccess) e = hipEventRecord(t->ram_ev[it.a.victim_ram], t->copy);
                t->ram_ev_set[it.a.victim_ram] = 1;
                if (e == hipSuccess) t->stats_d2h_bytes += t->blob_bytes;
            }
            /* the slot's previous readers must be done before it is overwritten */
            char& set = scratch ? t->scratch_ev_set[slot] : t->slot_ev_set[slot];
            hipEvent_t ev = scratch ? t->scratch_ev[slot] : t->slot_ev[slot];
            if (e == hipSuccess && set) e = hipStreamWaitEvent(t->copy, ev, 0);
            if (e == hipSuccess)
                e = hipMemcpyAsync(base + 8, t->blob_src(layer * P.E + it.id), t->blob_bytes,
                                   hipMemcpyHostToDevice, t->copy);
            if (e == hipSuccess && t->ssd()) {
                e = hipEventRecord(t->ram_ev[it.a.ram], t->copy);
                t->ram_ev_set[it.a.ram] = 1;
            }
            if (e == hipSuccess) t->stats_h2d_bytes += t->blob_bytes;
            t->pending_copies = true;
        }
        (scratch ? t->used_scratch : t->used_slots).push_back(slot);
        t->h_table[(size_t)layer * P.E + it.id] = base + 8;
    }
    if (e == hipSuccess && t->pending_copies) e = hipEventRecord(t->copies_done, t->copy);
    /* the layer's table row, ordered before the kernels that read it */
    if (e == hipSuccess)
        e = hipMemcpyAsync(t->d_table + (size_t)layer * P.E, t->h_table + (size_t)layer * P.E,
                           (size_t)P.E * sizeof(void*), hipMemcpyHostToDevice, compute);
    if (e == hipSuccess) e = hipEventRecord(t->row_ev[layer], compute);
    if (e == hipSuccess) t->row_ev_set[layer] = 1;
    return e;
}

extern "C" hipError_t wisp_tier_wait_copies(WispExpertTier* t, hipStream_t compute) {
    if (!t) return hipErrorInvalidValue;
    if (!t->pending_copies) return hipSuccess;
    return hipStreamWaitEvent(compute, t->copies_done, 0);
}

extern "C" hipError_t wisp_tier_release_layer(WispExpertTier* t, hipStream_t compute) {
    if (!t) return hipErrorInvalidValue;
    hipError_t e = hipSuccess;
    for (int s : t->used_slots) {
        if (e == hipSuccess) e = hipEventRecord(t->slot_ev[s], compute);
        t->slot_ev_set[s] = 1;
    }
    for (int s : t->used_scratch) {
        if (e == hipSuccess) e = hipEventRecord(t->scratch_ev[s], compute);
        t->scratch_ev_set[s] = 1;
    }
    t->used_slots.clear();
    t->used_scratch.clear();
    return e;
}

extern "C" void wisp_tier_stats(const WispExpertTier* t, uint64_t* out) {
    if (!t || !out) return;
    for (int i = 0; i < WISP_TIER_N_STATS; i++) out[i] = t->pol.stats[i];
    out[WISP_TIER_H2D_BYTES] = t->stats_h2d_bytes;
    out[WISP_TIER_SSD_BYTES] = t->stats_ssd_bytes;
    out[WISP_TIER_D2H_BYTES] = t->stats_d2h_bytes;
}

/* One MoE decode layer served by the tier (routing known on the host). */
extern "C" hipError_t wisp_tier_moe_decode_layer(WispExpertTier* t, int layer,
                                                 const void* d_shared_blob,
                                                 const WispExpertLayout* L, const void* d_x,
                                                 int x_dtype, int n_tokens, const int* h_topk_idx,
                                                 const float* h_topk_w, int top_k,
                                                 void* d_workspace, size_t workspace_bytes,
                                                 float* d_out_f32, wisp_half* d_out_f16,
                                                 hipStream_t compute) {
    if (!t || layer < 0 || layer >= t->pol.L || n_tokens < 1 || top_k < 1 || !h_topk_idx ||
        !h_topk_w || n_tokens > WISP_TIER_MAX_PAIRS || top_k > WISP_TIER_MAX_PAIRS ||
        n_tokens * top_k > WISP_TIER_MAX_PAIRS || !d_out_f32)   /* no int overflow */
        return hipErrorInvalidValue;
    const int np = n_tokens * top_k;
    const int E = t->pol.E;
    /* unique ids of the layer, first appearance order */
    int ids[WISP_TIER_MAX_PAIRS], paths[WISP_TIER_MAX_PAIRS], n = 0;
    for (int i = 0; i < np; i++) {
        const int id = h_topk_idx[i];
        if (id < 0 || id >= E) continue;
        bool dup = false;
        for (int q = 0; q < n; q++) dup |= ids[q] == id;
        if (!dup) ids[n++] = id;
    }
    hipError_t e = wisp_tier_fetch_layer(t, layer, ids, n, paths, compute);
    if (e != hipSuccess) return e;
    /* split the selection: experts resident now vs. experts being copied */
    int* row = t->h_route + (size_t)layer * 3 * WISP_TIER_MAX_PAIRS;
    int* hit = row;
    int* cp = row + WISP_TIER_MAX_PAIRS;
    float* w = (float*)(row + 2 * WISP_TIER_MAX_PAIRS);
    int n_hit = 0, n_cp = 0;
    for (int i = 0; i < np; i++) {
        const int id = h_topk_idx[i];
        int path = -1;
        for (int q = 0; q < n; q++)
            if (ids[q] == id) path = paths[q];
        const bool ready = path == WISP_TIER_VRAM_HIT;
        hit[i] = (path >= 0 && ready) ? id : -1;
        cp[i] = (path >= 0 && !ready) ? id : -1;
        n_hit += hit[i] >= 0;
        n_cp += cp[i] >= 0;
        w[i] = h_topk_w[i];
    }
    int* d_row = t->d_route + (size_t)layer * 3 * WISP_TIER_MAX_PAIRS;
    e = hipMemcpyAsync(d_row, row, 3 * WISP_TIER_MAX_PAIRS * sizeof(int), hipMemcpyHostToDevice,
                       compute);
    if (e == hipSuccess) e = hipEventRecord(t->row_ev[layer], compute);
    if (e != hipSuccess) return e;
    const void* const* table = (const void* const*)wisp_tier_device_table(t, layer);
    const float* d_w = (const float*)(d_row + 2 * WISP_TIER_MAX_PAIRS);
    const bool first = n_hit > 0 || d_shared_blob || n_cp == 0;
    if (first) {
        /* resident experts (and the shared one) while the copies run; with
         * nothing routed at all this pass writes the zero output */
        e = wisp_gpu_moe_decode_int4(table, d_shared_blob, L, d_x, x_dtype, n_tokens, d_row, d_w,
                                     top_k, E, d_workspace, workspace_bytes, 0, d_out_f32,
                                     n_cp ? nullptr : d_out_f16, compute);
        if (e != hipSuccess) return e;
    }
    if (n_cp) {
        e = wisp_tier_wait_copies(t, compute);
        if (e == hipSuccess)
            e = wisp_gpu_moe_decode_int4(table, nullptr, L, d_x, x_dtype, n_tokens,
                                         d_row + WISP_TIER_MAX_PAIRS, d_w, top_k, E, d_workspace,
                                         workspace_bytes, first ? 1 : 0, d_out_f32, d_out_f16,
                                         compute);
        if (e != hipSuccess) return e;
    }
    return wisp_tier_release_layer(t, compute);
}
