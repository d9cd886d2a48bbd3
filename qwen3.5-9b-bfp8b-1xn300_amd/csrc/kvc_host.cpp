// kvc_host.cpp -- host side of libkvc: C ABI entry points, block allocator,
// sequence table, chained-hash prefix index, snapshot pool, kernel launches.
//
// Reference sites replaced (src/engine.cpp of the reference):
//   alloc of caches/state  :3835-3843      reset_state       :4164-4176
//   decode append+attn     :3521-3564      prefill append+attn :2885-2924
//   prefix reuse           :4058-4080      token commit      :4118, :4150-4151
// The reference reuses state only when its single cached token list is a
// strict prefix of the new prompt; this library generalises that to many
// sequences sharing 32-token blocks through a verified hash chain, and to
// hybrid models through recurrent-state snapshots at fixed boundaries.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <set>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "../../include/kvc.h"
#include "kvc_internal.h"

using namespace kvc;

// ---------------------------------------------------------------------------
// errors

namespace {
thread_local std::string g_err;

int set_err(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_err(hipError_t e, const char* what) {
    return set_err(KVC_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define KVC_HIP(call, what)                               \
    do {                                                  \
        hipError_t e_ = (call);                           \
        if (e_ != hipSuccess) return hip_err(e_, (what)); \
    } while (0)

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ULL;
constexpr uint64_t kHashRoot = 0x6B76635F726F6F74ULL;

uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

// Chained block hash: absorbs the parent hash, the block length and each token
// through the splitmix64 finaliser.  The weak variant (test hook) keeps 4 bits.
uint64_t block_hash(uint64_t parent, const int32_t* tok, int n, bool weak) {
    uint64_t h = mix64(parent ^ (kGolden * (uint64_t)(n + 1)));
    for (int i = 0; i < n; i++) h = mix64(h + (uint64_t)(uint32_t)tok[i] + kGolden * (uint64_t)(i + 1));
    return weak ? (h & 0xFULL) : h;
}
}  // namespace

// ---------------------------------------------------------------------------
// context

struct Seq {
    bool live = false;
    int32_t len = 0;      // committed tokens (g_pos)
    int32_t pending = 0;  // reserved, not yet committed
    bool tokens_known = true;
    std::vector<int32_t> blocks;   // block id per 32-token block
    std::vector<int32_t> tokens;   // committed token ids (when known)
    std::vector<int32_t> entries;  // prefix-index entry per full block, -1 = none
    // Block pinned on behalf of entries[i] when that entry indexes another
    // sequence's copy of the same tokens (two sequences filled the block
    // independently); -1 when the entry indexes this sequence's own block,
    // which the sequence already holds.  The pin keeps the entry live, so
    // entries[i] stays a valid parent for block i + 1.
    std::vector<int32_t> pins;
    bool state_dirty = false;      // recurrent state must be zeroed before its next use
};

struct Entry {
    bool live = false;
    uint64_t hash = 0;
    int32_t parent = -1;
    int32_t block = -1;
    int32_t n_children = 0;
    uint64_t tick = 0;
    std::vector<int32_t> tok;
};

struct Snapshot {
    bool live = false;
    bool pinned = false;  // explicit save: kept until kvc_snapshot_release
    bool keyed = false;   // reachable from the snapshot index
    int32_t boundary = 0;
    uint64_t hash = 0;
    uint64_t tick = 0;
    std::vector<int32_t> tokens;  // [0, boundary) when keyed
};

struct kvc_ctx {
    kvc_config cfg{};
    bool has_device = false;
    int64_t n_blocks = 0;
    int32_t max_blocks = 0;  // block-table width
    int32_t seg_blocks = 0;  // blocks per snapshot segment
    int64_t layer_kv_bytes = 0;
    int64_t state_bytes = 0;  // per sequence slot (padded)
    int64_t rec_bytes = 0, conv_bytes = 0;
    int64_t snap_bytes = 0;
    int64_t hbm_bytes = 0;

    uint8_t* d_pool = nullptr;
    int32_t* d_table = nullptr;
    uint8_t* d_state = nullptr;
    uint8_t* d_snap = nullptr;
    float* d_part = nullptr;
    int32_t* d_counters = nullptr;
    float* s_part = nullptr;        // this device's static decode workspace
    int32_t* s_counters = nullptr;  // (file-scope __device__ array, never freed)
    float* d_rope = nullptr;  // RoPE cos [max_seq_len][rope_dim/2], then sin likewise

    std::vector<int32_t> refcnt;
    std::vector<int32_t> free_blocks;
    std::vector<Seq> seqs;
    std::vector<int32_t> free_seqs;

    std::vector<Entry> entries;
    std::vector<int32_t> free_entries;
    std::unordered_map<uint64_t, int32_t> index;
    std::set<std::pair<uint64_t, int32_t>> leaves;  // (tick, entry) of leaf entries

    std::vector<Snapshot> snaps;
    std::unordered_map<uint64_t, int32_t> snap_index;

    uint64_t tick = 0;
    int64_t prefix_hits = 0;
    int64_t evictions = 0;

    std::vector<std::pair<int32_t, int32_t>> table_updates;  // (flat index, block)
    std::vector<std::pair<int32_t, int32_t>> cow_copies;     // (src, dst)
};

namespace {

bool seq_ok(kvc_ctx* c, int32_t s) {
    return s >= 0 && s < (int32_t)c->seqs.size() && c->seqs[s].live;
}

// ---- prefix index --------------------------------------------------------

void leaf_insert(kvc_ctx* c, int32_t e) { c->leaves.insert({c->entries[e].tick, e}); }
void leaf_erase(kvc_ctx* c, int32_t e) { c->leaves.erase({c->entries[e].tick, e}); }

void touch_entry(kvc_ctx* c, int32_t e) {
    Entry& en = c->entries[e];
    const bool leaf = en.n_children == 0;
    if (leaf) leaf_erase(c, e);
    en.tick = ++c->tick;
    if (leaf) leaf_insert(c, e);
}

void unref_block(kvc_ctx* c, int32_t b) {
    if (--c->refcnt[b] == 0) c->free_blocks.push_back(b);
}

void evict_entry(kvc_ctx* c, int32_t e) {
    Entry& en = c->entries[e];
    leaf_erase(c, e);
    c->index.erase(en.hash);
    if (en.parent >= 0) {
        Entry& p = c->entries[en.parent];
        if (--p.n_children == 0) leaf_insert(c, en.parent);
    }
    unref_block(c, en.block);
    en = Entry();
    c->free_entries.push_back(e);
    c->evictions++;
}

// Reclaim one block held only by the index (least recently used leaf).
bool evict_one(kvc_ctx* c) {
    for (auto it = c->leaves.begin(); it != c->leaves.end(); ++it) {
        const int32_t e = it->second;
        if (c->refcnt[c->entries[e].block] == 1) {
            evict_entry(c, e);
            return true;
        }
    }
    return false;
}

int32_t alloc_block(kvc_ctx* c) {
    if (c->free_blocks.empty() && !evict_one(c)) return -1;
    const int32_t b = c->free_blocks.back();
    c->free_blocks.pop_back();
    c->refcnt[b] = 1;
    return b;
}

int32_t new_entry(kvc_ctx* c) {
    if (!c->free_entries.empty()) {
        const int32_t e = c->free_entries.back();
        c->free_entries.pop_back();
        return e;
    }
    c->entries.emplace_back();
    return (int32_t)c->entries.size() - 1;
}

// Look up block i of a chain: hash hit + same parent entry + same tokens.
int32_t find_entry(kvc_ctx* c, uint64_t h, int32_t parent, const int32_t* tok) {
    auto it = c->index.find(h);
    if (it == c->index.end()) return -1;
    const Entry& en = c->entries[it->second];
    if (en.parent != parent) return -1;
    if (memcmp(en.tok.data(), tok, sizeof(int32_t) * c->cfg.block_tokens) != 0) return -1;
    return it->second;
}

// Keep the first k index entries of s, dropping the pins of the rest.
void drop_entries(kvc_ctx* c, Seq& s, size_t k) {
    while (s.entries.size() > k) {
        if (s.pins.back() >= 0) unref_block(c, s.pins.back());
        s.entries.pop_back();
        s.pins.pop_back();
    }
}

void push_entry(kvc_ctx* c, Seq& s, int32_t e, int32_t own_block) {
    int32_t pin = -1;
    if (e >= 0 && c->entries[e].block != own_block) {
        pin = c->entries[e].block;
        c->refcnt[pin]++;
    }
    s.entries.push_back(e);
    s.pins.push_back(pin);
}

// Register the full blocks of s that have no entry yet.
void register_blocks(kvc_ctx* c, Seq& s) {
    const int bt = c->cfg.block_tokens;
    const bool weak = c->cfg.flags & KVC_FLAG_WEAK_HASH;
    const int full = s.len / bt;
    drop_entries(c, s, (size_t)full);
    for (int i = (int)s.entries.size(); i < full; i++) {
        const int32_t parent = i == 0 ? -1 : s.entries[i - 1];
        if (i > 0 && parent < 0) {  // chain broken earlier (collision)
            push_entry(c, s, -1, -1);
            continue;
        }
        const uint64_t ph = i == 0 ? kHashRoot : c->entries[parent].hash;
        const int32_t* tok = s.tokens.data() + (size_t)i * bt;
        const uint64_t h = block_hash(ph, tok, bt, weak);
        auto it = c->index.find(h);
        if (it != c->index.end()) {
            const int32_t e = find_entry(c, h, parent, tok);
            if (e >= 0) touch_entry(c, e);
            push_entry(c, s, e, s.blocks[i]);  // -1 on a collision: not registered
            continue;
        }
        const int32_t e = new_entry(c);
        Entry& en = c->entries[e];
        en.live = true;
        en.hash = h;
        en.parent = parent;
        en.block = s.blocks[i];
        en.n_children = 0;
        en.tick = ++c->tick;
        en.tok.assign(tok, tok + bt);
        c->refcnt[en.block]++;
        c->index[h] = e;
        if (parent >= 0) {
            Entry& p = c->entries[parent];
            if (p.n_children++ == 0) leaf_erase(c, parent);
        }
        leaf_insert(c, e);
        push_entry(c, s, e, s.blocks[i]);
    }
}

uint64_t chain_hash(kvc_ctx* c, const int32_t* tok, int n_blocks) {
    const bool weak = c->cfg.flags & KVC_FLAG_WEAK_HASH;
    uint64_t h = kHashRoot;
    for (int i = 0; i < n_blocks; i++) h = block_hash(h, tok + (size_t)i * c->cfg.block_tokens, c->cfg.block_tokens, weak);
    return h;
}

// ---- device helpers --------------------------------------------------------

int flush_table(kvc_ctx* c, void* stream) {
    if (!c->has_device) {
        c->table_updates.clear();
        c->cow_copies.clear();
        return KVC_OK;
    }
    size_t i = 0;
    while (i < c->table_updates.size()) {
        TableUpdateArgs a{};
        a.table = c->d_table;
        a.n = 0;
        for (; i < c->table_updates.size() && a.n < kTableUpdatesPerLaunch; i++, a.n++) {
            a.index[a.n] = c->table_updates[i].first;
            a.block[a.n] = c->table_updates[i].second;
        }
        int e = launch_table_update(a, stream);
        if (e) return hip_err((hipError_t)e, "table update launch");
    }
    c->table_updates.clear();
    i = 0;
    while (i < c->cow_copies.size()) {
        BlockCopyArgs a{};
        a.pool_base = c->d_pool;
        a.layer_kv_bytes = c->layer_kv_bytes;
        a.n_layers = c->cfg.n_attn_layers;
        for (; i < c->cow_copies.size() && a.n < kMaxBatch; i++, a.n++) {
            a.src[a.n] = c->cow_copies[i].first;
            a.dst[a.n] = c->cow_copies[i].second;
        }
        int e = launch_block_copy(a, stream);
        if (e) return hip_err((hipError_t)e, "block copy launch");
    }
    c->cow_copies.clear();
    return KVC_OK;
}

void set_table(kvc_ctx* c, int32_t slot, int32_t idx, int32_t block) {
    c->table_updates.push_back({slot * c->max_blocks + idx, block});
}

void release_tail(kvc_ctx* c, int32_t slot, int32_t keep_blocks) {
    Seq& s = c->seqs[slot];
    while ((int32_t)s.blocks.size() > keep_blocks) {
        unref_block(c, s.blocks.back());
        s.blocks.pop_back();
    }
}

// A created or reset sequence's recurrent state reads as zero (reset_state()
// zero-fills it, src/engine.cpp:4164-4176).  The fill is deferred to the first
// operation that uses the state, on that operation's stream: the Gated-DeltaNet
// step, a snapshot save, kvc_state_ptrs.  A snapshot restore overwrites the
// whole state and clears the flag.
int clean_states(kvc_ctx* c, const int32_t* seqs, size_t n, void* stream) {
    if (!c->has_device || c->state_bytes == 0) return KVC_OK;
    ZeroStateArgs z{};
    z.state = c->d_state;
    z.state_bytes = c->state_bytes;
    for (size_t i = 0; i < n; i++) {
        Seq& s = c->seqs[seqs[i]];
        if (!s.state_dirty) continue;
        s.state_dirty = false;
        z.slot[z.n_slots++] = seqs[i];
        if (z.n_slots == kMaxBatch || i + 1 == n) {
            int e = launch_zero_state(z, stream);
            if (e) return hip_err((hipError_t)e, "state zero-fill launch");
            z.n_slots = 0;
        }
    }
    if (z.n_slots > 0) {
        int e = launch_zero_state(z, stream);
        if (e) return hip_err((hipError_t)e, "state zero-fill launch");
    }
    return KVC_OK;
}

int launch_snapshots(kvc_ctx* c, const std::vector<int32_t>& seq_slots,
                     const std::vector<int32_t>& snap_slots, const std::vector<int32_t>& first_blocks,
                     bool restore, bool do_state, bool do_kv, void* stream) {
    if (!c->has_device) return KVC_OK;
    if (do_state && !restore) {  // a save reads the state: it must hold its zeros
        int rc = clean_states(c, seq_slots.data(), seq_slots.size(), stream);
        if (rc) return rc;
    }
    if (do_state && restore)
        for (int32_t s : seq_slots) c->seqs[s].state_dirty = false;  // overwritten below
    for (size_t i0 = 0; i0 < seq_slots.size(); i0 += kMaxBatch) {
        SnapshotArgs a{};
        a.state_base = c->d_state;
        a.snap_base = c->d_snap;
        a.pool_base = c->d_pool;
        a.table = c->d_table;
        a.state_bytes = c->state_bytes;
        a.snap_bytes = c->snap_bytes;
        a.layer_kv_bytes = c->layer_kv_bytes;
        a.n_layers = c->cfg.n_attn_layers;
        a.seg_blocks = c->seg_blocks;
        a.table_stride = c->max_blocks;
        a.restore = restore;
        a.do_state = do_state;
        a.do_kv = do_kv;
        const size_t n = std::min((size_t)kMaxBatch, seq_slots.size() - i0);
        a.n_pairs = (int32_t)n;
        for (size_t k = 0; k < n; k++) {
            a.seq_slot[k] = seq_slots[i0 + k];
            a.snap_slot[k] = snap_slots[i0 + k];
            a.first_block[k] = first_blocks[i0 + k];
        }
        int e = launch_snapshot(a, stream);
        if (e) return hip_err((hipError_t)e, "snapshot launch");
    }
    return KVC_OK;
}

// Free or LRU-evictable snapshot slot, or -1.
int32_t alloc_snapshot(kvc_ctx* c) {
    int32_t victim = -1;
    for (int32_t i = 0; i < (int32_t)c->snaps.size(); i++) {
        if (!c->snaps[i].live) return i;
        if (!c->snaps[i].pinned && (victim < 0 || c->snaps[i].tick < c->snaps[victim].tick)) victim = i;
    }
    if (victim >= 0) {
        Snapshot& sn = c->snaps[victim];
        if (sn.keyed) {
            auto it = c->snap_index.find(sn.hash);
            if (it != c->snap_index.end() && it->second == victim) c->snap_index.erase(it);
        }
        sn = Snapshot();
    }
    return victim;
}

void key_snapshot(kvc_ctx* c, int32_t id, const std::vector<int32_t>& tokens, int32_t boundary) {
    Snapshot& sn = c->snaps[id];
    sn.keyed = true;
    sn.tokens.assign(tokens.begin(), tokens.begin() + boundary);
    sn.hash = chain_hash(c, sn.tokens.data(), boundary / c->cfg.block_tokens);
    auto it = c->snap_index.find(sn.hash);
    if (it != c->snap_index.end() && it->second != id) c->snaps[it->second].keyed = false;
    c->snap_index[sn.hash] = id;
}

// Snapshot keyed at `boundary` whose tokens equal tok[0, boundary), or -1.
int32_t find_snapshot(kvc_ctx* c, const int32_t* tok, int32_t boundary, uint64_t h) {
    auto it = c->snap_index.find(h);
    if (it == c->snap_index.end()) return -1;
    const Snapshot& sn = c->snaps[it->second];
    if (!sn.live || !sn.keyed || sn.boundary != boundary) return -1;
    if (memcmp(sn.tokens.data(), tok, sizeof(int32_t) * boundary) != 0) return -1;
    return it->second;
}

int check_layer(kvc_ctx* c, int32_t layer) {
    if (layer < 0 || layer >= c->cfg.n_attn_layers)
        return set_err(KVC_ERR_RANGE, "layer %d out of range [0, %d)", layer, c->cfg.n_attn_layers);
    return KVC_OK;
}

int check_device(kvc_ctx* c) {
    if (!c->has_device) return set_err(KVC_ERR_NO_DEVICE, "context was created host-only (device = -1)");
    return KVC_OK;
}

int check_seqs(kvc_ctx* c, const int32_t* seqs, int32_t n) {
    if (!seqs || n <= 0) return set_err(KVC_ERR_INVALID, "empty sequence list");
    for (int32_t i = 0; i < n; i++) {
        if (!seq_ok(c, seqs[i])) return set_err(KVC_ERR_INVALID, "sequence %d is not live", seqs[i]);
        for (int32_t j = 0; j < i; j++)
            if (seqs[j] == seqs[i]) return set_err(KVC_ERR_INVALID, "sequence %d listed twice", seqs[i]);
    }
    return KVC_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI

extern "C" {

int kvc_abi_version(void) { return KVC_ABI_VERSION; }

const char* kvc_last_error(void) { return g_err.c_str(); }

void kvc_config_default(kvc_config* cfg) {
    if (!cfg) return;
    memset(cfg, 0, sizeof *cfg);
    cfg->n_attn_layers = 8;
    cfg->n_ssm_layers = 24;
    cfg->n_q_heads = 16;
    cfg->n_kv_heads = 4;
    cfg->head_dim = 256;
    cfg->block_tokens = 32;
    cfg->snapshot_interval = 256;
    cfg->max_seqs = 64;
    cfg->max_seq_len = 65536;
    cfg->ssm_v_heads = 32;
    cfg->ssm_k_dim = 128;
    cfg->ssm_v_dim = 128;
    cfg->conv_rows = 3;
    cfg->conv_channels = 8192;
    cfg->pool_blocks = 0;
    cfg->pool_fraction = 0.5;
    cfg->snapshot_slots = 64;
    cfg->decode_chunk_blocks = 0;
    cfg->device = 0;
    cfg->flags = 0;
    cfg->alloc_seed = 0;
    cfg->rms_norm_eps = 1e-6f;
    cfg->rope_freq_base = 1.0e7f;
    cfg->rope_dim = 64;
    cfg->reserved = 0;
}

static void free_device(kvc_ctx* c) {
    if (!c->has_device) return;
    if (c->d_pool) (void)hipFree(c->d_pool);
    if (c->d_table) (void)hipFree(c->d_table);
    if (c->d_state) (void)hipFree(c->d_state);
    if (c->d_snap) (void)hipFree(c->d_snap);
    if (c->d_part) (void)hipFree(c->d_part);
    if (c->d_counters) (void)hipFree(c->d_counters);
    if (c->d_rope) (void)hipFree(c->d_rope);
}

static int dev_alloc(kvc_ctx* c, void** p, size_t bytes, const char* what) {
    if (bytes == 0) {
        *p = nullptr;
        return KVC_OK;
    }
    hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return set_err(KVC_ERR_NOMEM, "hipMalloc(%s, %zu bytes): %s", what, bytes, hipGetErrorString(e));
    }
    c->hbm_bytes += (int64_t)bytes;
    return KVC_OK;
}

// RoPE cos/sin tables for every position of a sequence, computed as the
// reference precomputes them (src/engine.cpp:2408-2419: fp32 freq = 1 /
// powf(base, 2p / rope_dim), theta = pos * freq, cosf / sinf) and uploaded
// once.
static int build_rope_table(kvc_ctx* c) {
    const int half = c->cfg.rope_dim / 2;
    const size_t n = (size_t)c->cfg.max_seq_len * half;
    std::vector<float> tab(2 * n);
    for (int pos = 0; pos < c->cfg.max_seq_len; pos++) {
        for (int p = 0; p < half; p++) {
            const float freq = 1.0f / powf(c->cfg.rope_freq_base, 2.0f * p / c->cfg.rope_dim);
            const float theta = pos * freq;
            tab[(size_t)pos * half + p] = cosf(theta);
            tab[n + (size_t)pos * half + p] = sinf(theta);
        }
    }
    int rc = dev_alloc(c, (void**)&c->d_rope, tab.size() * sizeof(float), "RoPE tables");
    if (rc) return rc;
    hipError_t e = hipMemcpy(c->d_rope, tab.data(), tab.size() * sizeof(float), hipMemcpyHostToDevice);
    return e == hipSuccess ? KVC_OK : hip_err(e, "RoPE table upload");
}

int kvc_create(const kvc_config* cfg, kvc_ctx** out) {
    if (!cfg || !out) return set_err(KVC_ERR_INVALID, "null config or output");
    *out = nullptr;
    const kvc_config& k = *cfg;
    if (k.n_q_heads != kQHeads || k.n_kv_heads != kKvHeads || k.head_dim != kHeadDim || k.block_tokens != kBlockTok)
        return set_err(KVC_ERR_UNSUPPORTED,
                       "kernels are built for q/kv heads %d/%d, head_dim %d, block %d (got %d/%d, %d, %d)",
                       kQHeads, kKvHeads, kHeadDim, kBlockTok, k.n_q_heads, k.n_kv_heads, k.head_dim,
                       k.block_tokens);
    if (k.n_attn_layers < 1 || k.n_ssm_layers < 0 || k.max_seqs < 1 || k.max_seq_len < 1)
        return set_err(KVC_ERR_INVALID, "layer/sequence counts must be positive");
    if (k.snapshot_interval < 0 || (k.snapshot_interval % k.block_tokens) != 0)
        return set_err(KVC_ERR_INVALID, "snapshot_interval must be a non-negative multiple of block_tokens");
    if (k.snapshot_slots < 0) return set_err(KVC_ERR_INVALID, "snapshot_slots must be >= 0");
    if ((k.flags & KVC_FLAG_DECODE_SPLIT_D) && (k.flags & KVC_FLAG_DECODE_NO_SPLIT_D))
        return set_err(KVC_ERR_INVALID, "KVC_FLAG_DECODE_SPLIT_D and KVC_FLAG_DECODE_NO_SPLIT_D exclude each other");
    if (k.n_ssm_layers > 0 &&
        (k.ssm_v_heads <= 0 || k.ssm_k_dim <= 0 || k.ssm_v_dim <= 0 || k.conv_rows <= 0 || k.conv_channels <= 0))
        return set_err(KVC_ERR_INVALID, "recurrent-state shape must be positive");
    if (k.rope_dim != 0 && (k.rope_dim < 8 || k.rope_dim > kHeadDim || (k.rope_dim & (k.rope_dim - 1)) != 0))
        return set_err(KVC_ERR_UNSUPPORTED, "rope_dim must be 0 or a power of two in [8, %d] (got %d)", kHeadDim,
                       k.rope_dim);
    if (!(k.rope_freq_base > 0.0f) || !std::isfinite(k.rope_freq_base) || !(k.rms_norm_eps >= 0.0f) ||
        !std::isfinite(k.rms_norm_eps))
        return set_err(KVC_ERR_INVALID, "rope_freq_base must be positive and rms_norm_eps non-negative");

    kvc_ctx* c = new (std::nothrow) kvc_ctx();
    if (!c) return set_err(KVC_ERR_NOMEM, "host allocation failed");
    c->cfg = k;
    c->max_blocks = (k.max_seq_len + kBlockTok - 1) / kBlockTok;
    c->seg_blocks = k.snapshot_interval / kBlockTok;
    if (k.n_ssm_layers > 0) {
        c->rec_bytes = (int64_t)k.ssm_v_heads * k.ssm_v_dim * k.ssm_k_dim * 4;
        c->conv_bytes = (int64_t)k.conv_rows * k.conv_channels * 4;
    }
    c->state_bytes = ((int64_t)k.n_ssm_layers * (c->rec_bytes + c->conv_bytes) + 255) / 256 * 256;
    const int64_t seg_bytes = (int64_t)k.n_attn_layers * 2 * c->seg_blocks * (int64_t)kBlockBytes;
    c->snap_bytes = c->state_bytes + seg_bytes;
    const int n_snap = k.snapshot_interval > 0 ? k.snapshot_slots : 0;

    c->has_device = k.device >= 0;
    int rc = KVC_OK;
    if (c->has_device) {
        int ndev = 0;
        hipError_t e = hipGetDeviceCount(&ndev);
        if (e != hipSuccess || k.device >= ndev) {
            (void)hipGetLastError();
            delete c;
            return set_err(KVC_ERR_NO_DEVICE, "HIP device %d not available (%d devices)", k.device, ndev);
        }
        e = hipSetDevice(k.device);
        if (e != hipSuccess) {
            delete c;
            return hip_err(e, "hipSetDevice");
        }
        const size_t table_bytes = (size_t)k.max_seqs * c->max_blocks * 4;
        const size_t part_bytes = kPartBytes;
        const size_t ctr_bytes = kCounterBytes;
        if ((rc = dev_alloc(c, (void**)&c->d_table, table_bytes, "block table")) ||
            (rc = dev_alloc(c, (void**)&c->d_state, (size_t)c->state_bytes * k.max_seqs, "state pool")) ||
            (rc = dev_alloc(c, (void**)&c->d_snap, (size_t)c->snap_bytes * n_snap, "snapshot pool")) ||
            (rc = dev_alloc(c, (void**)&c->d_part, part_bytes, "split-K workspace")) ||
            (rc = dev_alloc(c, (void**)&c->d_counters, ctr_bytes, "arrival counters"))) {
            free_device(c);
            delete c;
            return rc;
        }
        int64_t nb = k.pool_blocks;
        if (nb <= 0) {
            size_t free_b = 0, total_b = 0;
            if ((e = hipMemGetInfo(&free_b, &total_b)) != hipSuccess) {
                free_device(c);
                delete c;
                return hip_err(e, "hipMemGetInfo");
            }
            const double frac = k.pool_fraction > 0 && k.pool_fraction <= 0.95 ? k.pool_fraction : 0.5;
            nb = (int64_t)((double)free_b * frac) / ((int64_t)k.n_attn_layers * 2 * (int64_t)kBlockBytes);
        }
        if (nb < 1 || nb > INT32_MAX) {
            free_device(c);
            delete c;
            return set_err(KVC_ERR_NOMEM, "block pool of %lld blocks is not usable", (long long)nb);
        }
        c->n_blocks = nb;
        c->layer_kv_bytes = nb * (int64_t)kBlockBytes;
        if ((rc = dev_alloc(c, (void**)&c->d_pool, (size_t)c->layer_kv_bytes * 2 * k.n_attn_layers, "K/V pools"))) {
            free_device(c);
            delete c;
            return rc;
        }
        // one-time zeroing at creation (never inside captured work)
        if ((e = hipMemset(c->d_table, 0, table_bytes)) != hipSuccess ||
            (e = hipMemset(c->d_counters, 0, ctr_bytes)) != hipSuccess ||
            (c->state_bytes && (e = hipMemset(c->d_state, 0, (size_t)c->state_bytes * k.max_seqs)) != hipSuccess) ||
            (e = hipDeviceSynchronize()) != hipSuccess) {
            free_device(c);
            delete c;
            return hip_err(e, "initialising device tables");
        }
        if (k.rope_dim > 0 && (rc = build_rope_table(c))) {
            free_device(c);
            delete c;
            return rc;
        }
        // the static decode workspace of kvc_decode_attn_static: its device
        // address on this GPU, looked up once per device
        if ((e = (hipError_t)static_scratch(k.device, &c->s_part, &c->s_counters)) != hipSuccess) {
            free_device(c);
            delete c;
            return hip_err(e, "static decode workspace");
        }
    } else {
        if (k.pool_blocks <= 0 || k.pool_blocks > INT32_MAX) {
            delete c;
            return set_err(KVC_ERR_INVALID, "host-only context needs pool_blocks > 0");
        }
        c->n_blocks = k.pool_blocks;
        c->layer_kv_bytes = c->n_blocks * (int64_t)kBlockBytes;
    }

    c->refcnt.assign(c->n_blocks, 0);
    c->free_blocks.resize(c->n_blocks);
    // free list is popped from the back: block 0 is handed out first
    for (int64_t i = 0; i < c->n_blocks; i++) c->free_blocks[i] = (int32_t)(c->n_blocks - 1 - i);
    if (k.alloc_seed) {  // seeded Fisher-Yates permutation of the free list
        uint64_t st = k.alloc_seed;
        for (int64_t i = c->n_blocks - 1; i > 0; i--) {
            st += kGolden;
            const uint64_t r = mix64(st) % (uint64_t)(i + 1);
            std::swap(c->free_blocks[i], c->free_blocks[r]);
        }
    }
    c->seqs.resize(k.max_seqs);
    for (int32_t i = k.max_seqs - 1; i >= 0; i--) c->free_seqs.push_back(i);
    c->snaps.resize(n_snap);
    *out = c;
    return KVC_OK;
}

int kvc_destroy(kvc_ctx* c) {
    if (!c) return KVC_OK;
    if (c->has_device) (void)hipDeviceSynchronize();
    free_device(c);
    delete c;
    return KVC_OK;
}

int kvc_get_stats(kvc_ctx* c, kvc_stats* s) {
    if (!c || !s) return set_err(KVC_ERR_INVALID, "null argument");
    memset(s, 0, sizeof *s);
    s->pool_blocks = c->n_blocks;
    s->free_blocks = (int64_t)c->free_blocks.size();
    for (const Entry& e : c->entries)
        if (e.live) {
            s->indexed_blocks++;
            if (c->refcnt[e.block] == 1) s->cached_blocks++;
        }
    for (const Snapshot& sn : c->snaps) s->snapshots += sn.live;
    s->snapshot_slots = (int64_t)c->snaps.size();
    s->hbm_bytes = c->hbm_bytes;
    s->block_bytes = (int64_t)kBlockBytes;
    s->prefix_hits = c->prefix_hits;
    s->evictions = c->evictions;
    return KVC_OK;
}

// ---- sequences -------------------------------------------------------------

int kvc_seq_create(kvc_ctx* c, int32_t* seq) {
    if (!c || !seq) return set_err(KVC_ERR_INVALID, "null argument");
    if (c->free_seqs.empty()) return set_err(KVC_ERR_NOMEM, "all %d sequence slots in use", c->cfg.max_seqs);
    const int32_t s = c->free_seqs.back();
    c->free_seqs.pop_back();
    c->seqs[s] = Seq();
    c->seqs[s].live = true;
    c->seqs[s].state_dirty = c->cfg.n_ssm_layers > 0;  // the slot may hold an earlier sequence's state
    *seq = s;
    return KVC_OK;
}

int kvc_seq_reset(kvc_ctx* c, int32_t seq) {
    if (!c) return set_err(KVC_ERR_INVALID, "null context");
    if (!seq_ok(c, seq)) return set_err(KVC_ERR_INVALID, "sequence %d is not live", seq);
    release_tail(c, seq, 0);
    Seq& s = c->seqs[seq];
    s.len = s.pending = 0;
    s.tokens.clear();
    drop_entries(c, s, 0);
    s.tokens_known = true;
    s.state_dirty = c->cfg.n_ssm_layers > 0;
    return KVC_OK;
}

int kvc_seq_release(kvc_ctx* c, int32_t seq) {
    int rc = kvc_seq_reset(c, seq);
    if (rc) return rc;
    c->seqs[seq].live = false;
    c->free_seqs.push_back(seq);
    return KVC_OK;
}

int kvc_seq_len(kvc_ctx* c, int32_t seq, int32_t* len) {
    if (!c || !len) return set_err(KVC_ERR_INVALID, "null argument");
    if (!seq_ok(c, seq)) return set_err(KVC_ERR_INVALID, "sequence %d is not live", seq);
    *len = c->seqs[seq].len;
    return KVC_OK;
}

int kvc_seq_truncate(kvc_ctx* c, int32_t seq, int32_t len) {
    if (!c) return set_err(KVC_ERR_INVALID, "null context");
    if (!seq_ok(c, seq)) return set_err(KVC_ERR_INVALID, "sequence %d is not live", seq);
    Seq& s = c->seqs[seq];
    if (s.pending) return set_err(KVC_ERR_STATE, "sequence %d has %d uncommitted tokens", seq, s.pending);
    if (len < 0 || len > s.len) return set_err(KVC_ERR_RANGE, "truncate to %d outside [0, %d]", len, s.len);
    release_tail(c, seq, (len + kBlockTok - 1) / kBlockTok);
    drop_entries(c, s, (size_t)(len / kBlockTok));
    if (c->cfg.n_ssm_layers > 0 && len < s.len) {
        // The recurrent state cannot be rolled back: it still holds the
        // dropped tokens.  K/V and state committed from here on are no longer
        // a function of the token ids, so they must not be keyed by them:
        // the sequence stops feeding the prefix index and the boundary
        // snapshots until a reset or a snapshot restore.  The blocks it
        // indexed before the truncation stay valid.
        s.tokens_known = false;
        s.tokens.clear();
    }
    s.len = len;
    if (s.tokens_known) s.tokens.resize(len);
    return KVC_OK;
}

int kvc_seq_reserve(kvc_ctx* c, const int32_t* seqs, int32_t n_seqs, int32_t n_tok, void* stream) {
    if (!c) return set_err(KVC_ERR_INVALID, "null context");
    int rc = check_seqs(c, seqs, n_seqs);
    if (rc) return rc;
    if (n_tok <= 0) return set_err(KVC_ERR_INVALID, "n_tok must be positive");
    for (int32_t i = 0; i < n_seqs; i++) {
        const Seq& s = c->seqs[seqs[i]];
        if (s.pending) return set_err(KVC_ERR_STATE, "sequence %d already has %d reserved tokens", seqs[i], s.pending);
        if ((int64_t)s.len + n_tok > c->cfg.max_seq_len)
            return set_err(KVC_ERR_RANGE, "sequence %d: %d + %d tokens exceeds max_seq_len %d", seqs[i], s.len,
                           n_tok, c->cfg.max_seq_len);
    }
    // allocate everything first so a failure leaves no partial reservation
    struct Grant { int32_t seq, idx, block, cow_src; };
    std::vector<Grant> grants;
    bool fail = false;
    for (int32_t i = 0; i < n_seqs && !fail; i++) {
        const Seq& s = c->seqs[seqs[i]];
        if (s.len % kBlockTok) {
            const int32_t idx = s.len / kBlockTok;
            const int32_t b = s.blocks[idx];
            if (c->refcnt[b] > 1) {  // shared partial block: copy before writing
                const int32_t nb = alloc_block(c);
                if (nb < 0) { fail = true; break; }
                grants.push_back({seqs[i], idx, nb, b});
            }
        }
        const int32_t need = (s.len + n_tok + kBlockTok - 1) / kBlockTok;
        for (int32_t idx = (int32_t)s.blocks.size(); idx < need; idx++) {
            const int32_t nb = alloc_block(c);
            if (nb < 0) { fail = true; break; }
            grants.push_back({seqs[i], idx, nb, -1});
        }
    }
    if (fail) {
        for (const Grant& g : grants) unref_block(c, g.block);
        return set_err(KVC_ERR_NOMEM, "block pool exhausted (%lld blocks per layer)", (long long)c->n_blocks);
    }
    for (const Grant& g : grants) {
        Seq& s = c->seqs[g.seq];
        if (g.cow_src >= 0) {
            c->cow_copies.push_back({g.cow_src, g.block});
            unref_block(c, g.cow_src);
            s.blocks[g.idx] = g.block;
            drop_entries(c, s, (size_t)g.idx);
        } else {
            s.blocks.push_back(g.block);
        }
        set_table(c, g.seq, g.idx, g.block);
    }
    for (int32_t i = 0; i < n_seqs; i++) c->seqs[seqs[i]].pending = n_tok;
    return flush_table(c, stream);
}

int kvc_seq_commit(kvc_ctx* c, const int32_t* seqs, int32_t n_seqs, int32_t n_tok, const int32_t* tokens,
                   void* stream) {
    if (!c) return set_err(KVC_ERR_INVALID, "null context");
    int rc = check_seqs(c, seqs, n_seqs);
    if (rc) return rc;
    for (int32_t i = 0; i < n_seqs; i++)
        if (c->seqs[seqs[i]].pending != n_tok)
            return set_err(KVC_ERR_STATE, "sequence %d: commit of %d tokens but %d reserved", seqs[i], n_tok,
                           c->seqs[seqs[i]].pending);
    std::vector<int32_t> snap_seq, snap_slot, snap_first;
    const int iv = c->cfg.snapshot_interval;
    for (int32_t i = 0; i < n_seqs; i++) {
        Seq& s = c->seqs[seqs[i]];
        s.len += n_tok;
        s.pending = 0;
        if (!tokens) {
            s.tokens_known = false;
            continue;
        }
        if (!s.tokens_known) continue;
        const int32_t* t = tokens + (size_t)i * n_tok;
        s.tokens.insert(s.tokens.end(), t, t + n_tok);
        register_blocks(c, s);
        // automatic snapshot when landing on a boundary (hybrid models only)
        if (c->cfg.n_ssm_layers > 0 && iv > 0 && !c->snaps.empty() && s.len % iv == 0) {
            const uint64_t h = chain_hash(c, s.tokens.data(), s.len / kBlockTok);
            const int32_t have = find_snapshot(c, s.tokens.data(), s.len, h);
            if (have >= 0) {
                c->snaps[have].tick = ++c->tick;
                continue;
            }
            const int32_t id = alloc_snapshot(c);
            if (id < 0) continue;
            Snapshot& sn = c->snaps[id];
            sn.live = true;
            sn.pinned = false;
            sn.boundary = s.len;
            sn.tick = ++c->tick;
            key_snapshot(c, id, s.tokens, s.len);
            snap_seq.push_back(seqs[i]);
            snap_slot.push_back(id);
            snap_first.push_back((s.len - iv) / kBlockTok);
        }
    }
    if (!snap_seq.empty()) return launch_snapshots(c, snap_seq, snap_slot, snap_first, false, true, true, stream);
    return KVC_OK;
}

// ---- prefix match ----------------------------------------------------------

int kvc_prefix_match(kvc_ctx* c, int32_t seq, const int32_t* tokens, int32_t n, int32_t* reuse_len, void* stream) {
    if (!c || !reuse_len) return set_err(KVC_ERR_INVALID, "null argument");
    *reuse_len = 0;
    if (!seq_ok(c, seq)) return set_err(KVC_ERR_INVALID, "sequence %d is not live", seq);
    Seq& s = c->seqs[seq];
    if (s.len || s.pending) return set_err(KVC_ERR_STATE, "prefix match needs an empty sequence");
    if (n < 0 || (n > 0 && !tokens)) return set_err(KVC_ERR_INVALID, "bad token list");
    if (n > c->cfg.max_seq_len) return set_err(KVC_ERR_RANGE, "prompt of %d tokens exceeds max_seq_len", n);
    const int bt = kBlockTok;
    const bool weak = c->cfg.flags & KVC_FLAG_WEAK_HASH;
    const int n_full = n > 0 ? (n - 1) / bt : 0;  // never reuse the whole prompt
    std::vector<uint64_t> hashes(n_full);
    std::vector<int32_t> res;  // resident entries, chain-verified
    uint64_t h = kHashRoot;
    int32_t parent = -1;
    bool chain = true;
    for (int i = 0; i < n_full; i++) {
        h = block_hash(h, tokens + (size_t)i * bt, bt, weak);
        hashes[i] = h;
        if (chain) {
            const int32_t e = find_entry(c, h, parent, tokens + (size_t)i * bt);
            if (e < 0) chain = false;
            else {
                res.push_back(e);
                parent = e;
            }
        }
    }
    const int n_res = (int)res.size();
    const bool hybrid = c->cfg.n_ssm_layers > 0;
    const int iv = c->cfg.snapshot_interval;
    const int segb = c->seg_blocks;
    int reuse_blocks = n_res;
    int32_t snap_at = -1;           // snapshot providing the recurrent state
    std::vector<int32_t> seg_snap;  // per segment: snapshot holding its K/V, or -1
    if (hybrid) {
        // resume only where a state snapshot exists, and only if every
        // segment before it is resident or held by a snapshot of its own
        reuse_blocks = 0;
        if (iv > 0) {
            const int n_seg = n_full / segb;
            std::vector<int32_t> found(n_seg, -1);
            for (int k = 0; k < n_seg; k++)
                found[k] = find_snapshot(c, tokens, (k + 1) * iv, hashes[(size_t)(k + 1) * segb - 1]);
            for (int k = n_seg; k >= 1; k--) {
                if (found[k - 1] < 0) continue;
                bool ok = true;
                for (int j = 0; j < k && ok; j++)
                    if ((j + 1) * segb > n_res && found[j] < 0) ok = false;
                if (!ok) continue;
                snap_at = found[k - 1];
                reuse_blocks = k * segb;
                seg_snap.assign(found.begin(), found.begin() + k);
                break;
            }
        }
    }
    if (reuse_blocks == 0) return KVC_OK;

    // resident blocks are mapped (zero copy); a segment with any block not
    // resident is rebuilt in fresh blocks from its snapshot's K/V copy
    std::vector<int32_t> rs_seq, rs_snap, rs_first;
    int mapped = 0;  // leading blocks mapped from the index
    for (int i = 0; i < reuse_blocks; i++) {
        const bool resident = hybrid ? (i / segb + 1) * segb <= n_res : true;
        if (resident) {
            const int32_t b = c->entries[res[i]].block;
            c->refcnt[b]++;
            s.blocks.push_back(b);
            if (mapped == i) mapped++;
            continue;
        }
        const int32_t b = alloc_block(c);
        if (b < 0) {
            release_tail(c, seq, 0);
            return set_err(KVC_ERR_NOMEM, "block pool exhausted while restoring a prefix");
        }
        s.blocks.push_back(b);
        if (i % segb == 0) {
            rs_seq.push_back(seq);
            rs_snap.push_back(seg_snap[i / segb]);
            rs_first.push_back(i);
        }
    }
    for (int i = 0; i < reuse_blocks; i++) set_table(c, seq, i, s.blocks[i]);
    s.len = reuse_blocks * bt;
    s.tokens.assign(tokens, tokens + s.len);
    s.tokens_known = true;
    drop_entries(c, s, 0);
    for (int i = 0; i < mapped; i++) {
        push_entry(c, s, res[i], s.blocks[i]);  // its own block: no pin
        touch_entry(c, res[i]);
    }
    int rc = flush_table(c, stream);
    if (rc) return rc;
    if (!rs_seq.empty() && (rc = launch_snapshots(c, rs_seq, rs_snap, rs_first, true, false, true, stream))) return rc;
    if (snap_at >= 0) {
        c->snaps[snap_at].tick = ++c->tick;
        if ((rc = launch_snapshots(c, {seq}, {snap_at}, {0}, true, true, false, stream))) return rc;
    }
    register_blocks(c, s);  // restored blocks re-enter the index
    c->prefix_hits += s.len;
    *reuse_len = s.len;
    return KVC_OK;
}

// ---- device ops ------------------------------------------------------------

int kvc_append(kvc_ctx* c, int32_t layer, const int32_t* seqs, int32_t n_seqs, int32_t n_tok, const void* k,
               const void* v, void* stream) {
    if (!c) return set_err(KVC_ERR_INVALID, "null context");
    int rc;
    if ((rc = check_device(c)) || (rc = check_layer(c, layer)) || (rc = check_seqs(c, seqs, n_seqs))) return rc;
    if (!k || !v || n_tok <= 0) return set_err(KVC_ERR_INVALID, "append needs k, v and n_tok > 0");
    for (int32_t i = 0; i < n_seqs; i++)
        if (c->seqs[seqs[i]].pending < n_tok)
            return set_err(KVC_ERR_STATE, "sequence %d: append of %d tokens but %d reserved", seqs[i], n_tok,
                           c->seqs[seqs[i]].pending);
    if ((int64_t)std::min(kMaxBatch, n_seqs) * n_tok > INT32_MAX) return set_err(KVC_ERR_RANGE, "append too large");
    const size_t row = (size_t)kKvHeads * kHeadDim;
    for (int32_t i0 = 0; i0 < n_seqs; i0 += kMaxBatch) {
        const int32_t n = std::min(kMaxBatch, n_seqs - i0);
        AppendArgs a{};
        a.kpool = reinterpret_cast<uint16_t*>(c->d_pool + (int64_t)(layer * 2) * c->layer_kv_bytes);
        a.vpool = reinterpret_cast<uint16_t*>(c->d_pool + (int64_t)(layer * 2 + 1) * c->layer_kv_bytes);
        a.table = c->d_table;
        a.k = static_cast<const uint16_t*>(k) + (size_t)i0 * n_tok * row;
        a.v = static_cast<const uint16_t*>(v) + (size_t)i0 * n_tok * row;
        a.table_stride = c->max_blocks;
        a.n_seqs = n;
        a.n_tok = n_tok;
        for (int32_t j = 0; j < n; j++) {
            const Seq& s = c->seqs[seqs[i0 + j]];
            a.slot[j] = seqs[i0 + j];
            a.pos0[j] = s.len + s.pending - n_tok;
        }
        int e = launch_append(a, stream);
        if (e) return hip_err((hipError_t)e, "append launch");
    }
    return KVC_OK;
}

int kvc_qkv_append(kvc_ctx* c, int32_t layer, const int32_t* seqs, int32_t n_seqs, int32_t n_tok, const void* qkv,
                   int32_t in_dtype, const void* q_norm, const void* k_norm, void* q_out, void* gate_out,
                   void* stream) {
    if (!c) return set_err(KVC_ERR_INVALID, "null context");
    int rc;
    if ((rc = check_device(c)) || (rc = check_layer(c, layer)) || (rc = check_seqs(c, seqs, n_seqs))) return rc;
    if (!qkv || !q_norm || !k_norm || n_tok <= 0)
        return set_err(KVC_ERR_INVALID, "qkv append needs qkv, q_norm, k_norm and n_tok > 0");
    if (in_dtype != KVC_DTYPE_F32 && in_dtype != KVC_DTYPE_BF16) return set_err(KVC_ERR_INVALID, "bad in_dtype");
    for (int32_t i = 0; i < n_seqs; i++)
        if (c->seqs[seqs[i]].pending < n_tok)
            return set_err(KVC_ERR_STATE, "sequence %d: append of %d tokens but %d reserved", seqs[i], n_tok,
                           c->seqs[seqs[i]].pending);
    if ((int64_t)std::min(kMaxBatch, n_seqs) * n_tok > INT32_MAX)
        return set_err(KVC_ERR_RANGE, "qkv append too large");
    const size_t esz = in_dtype == KVC_DTYPE_BF16 ? 2 : 4;
    const size_t qrow = (size_t)kQHeads * kHeadDim;
    for (int32_t i0 = 0; i0 < n_seqs; i0 += kMaxBatch) {
        const int32_t n = std::min(kMaxBatch, n_seqs - i0);
        QkvArgs a{};
        a.qkv = static_cast<const uint8_t*>(qkv) + (size_t)i0 * n_tok * kQkvRow * esz;
        a.q_norm = static_cast<const float*>(q_norm);
        a.k_norm = static_cast<const float*>(k_norm);
        a.rope = c->d_rope;
        a.kpool = reinterpret_cast<uint16_t*>(c->d_pool + (int64_t)(layer * 2) * c->layer_kv_bytes);
        a.vpool = reinterpret_cast<uint16_t*>(c->d_pool + (int64_t)(layer * 2 + 1) * c->layer_kv_bytes);
        a.table = c->d_table;
        a.q_out = q_out ? static_cast<uint16_t*>(q_out) + (size_t)i0 * n_tok * qrow : nullptr;
        a.gate_out = gate_out ? static_cast<uint16_t*>(gate_out) + (size_t)i0 * n_tok * qrow : nullptr;
        a.eps = c->cfg.rms_norm_eps;
        a.in_bf16 = in_dtype == KVC_DTYPE_BF16;
        a.rope_half = c->cfg.rope_dim / 2;
        a.rope_rows = c->cfg.max_seq_len;
        a.table_stride = c->max_blocks;
        a.n_seqs = n;
        a.n_tok = n_tok;
        for (int32_t j = 0; j < n; j++) {
            const Seq& s = c->seqs[seqs[i0 + j]];
            a.slot[j] = seqs[i0 + j];
            a.pos0[j] = s.len + s.pending - n_tok;
        }
        int e = launch_qkv_append(a, stream);
        if (e) return hip_err((hipError_t)e, "qkv append launch");
    }
    return KVC_OK;
}

// Decode launches with fewer work items than this split each chunk's output
// dims over 2 workgroups (one per CU of the 256 is the aim).
constexpr int64_t kDsplitBelowItems = 256;

static int32_t auto_chunk_blocks(kvc_ctx* c, int64_t total_blocks) {
    if (c->cfg.decode_chunk_blocks > 0) return c->cfg.decode_chunk_blocks;
    // About 16 items per CU on 256 CUs (kAutoItems): three decode workgroups
    // are resident per CU, and many short items balance the ragged sequences'
    // chunks better than a few long ones (config d: 598-602 us per layer at
    // 3072-6144 items against 627 at 1024).  Chunks of at least 4 blocks keep
    // the split-K partial traffic and the final combine small.
    int64_t cb = (total_blocks * kKvHeads + kAutoItems - 1) / kAutoItems;
    return (int32_t)std::max<int64_t>(4, cb);
}

// Argument block of the decode launch over seqs[i0, i0 + n): work split and
// pointers.  The split-K partials and arrival counters live in `part` /
// `counters`; a launch needing more than `max_items` items is refused
// (KVC_ERR_RANGE).  No allocation.
// The producer inputs of kvc_decode_step (qkv == nullptr: plain decode).
struct DecodeProducer {
    const void* qkv = nullptr;
    int32_t in_dtype = KVC_DTYPE_BF16;
    const void* q_norm = nullptr;
    const void* k_norm = nullptr;
};

static int build_decode_args(kvc_ctx* c, int32_t layer, const int32_t* seqs, int32_t i0, int32_t n, const void* q,
                             const void* k_new, const void* v_new, const void* gate, const DecodeProducer& prod,
                             void* out, int32_t out_dtype, float scale, float* part, uint32_t part_bytes,
                             int32_t* counters, int64_t max_items, const char* workspace, DecodeArgs& a) {
    const size_t qrow = (size_t)kQHeads * kHeadDim, kvrow = (size_t)kKvHeads * kHeadDim;
    const size_t osz = out_dtype == KVC_DTYPE_BF16 ? 2 : 4;
    memset(&a, 0, sizeof a);
    int64_t total_blocks = 0;
    for (int32_t j = 0; j < n; j++) {
        const Seq& s = c->seqs[seqs[i0 + j]];
        const int32_t L = s.len + s.pending;
        if (L <= 0) return set_err(KVC_ERR_STATE, "sequence %d has no keys to attend", seqs[i0 + j]);
        if ((k_new || prod.qkv) && s.pending < 1)
            return set_err(KVC_ERR_STATE, "sequence %d: fused append needs a reserved token", seqs[i0 + j]);
        a.slot[j] = seqs[i0 + j];
        a.kv_len[j] = L;
        total_blocks += (L + kBlockTok - 1) / kBlockTok;
    }
    int32_t cb = auto_chunk_blocks(c, total_blocks);
    const bool auto_cb = c->cfg.decode_chunk_blocks <= 0;
    const bool force_split = c->cfg.flags & KVC_FLAG_DECODE_SPLIT_D;
    const int64_t max_chunks = force_split ? kMaxChunks / kMaxDParts : kMaxChunks;
    int64_t total_chunks;
    for (;;) {
        total_chunks = 0;
        for (int32_t j = 0; j < n; j++) {
            a.chunk_begin[j] = (int32_t)total_chunks;
            const int32_t nb = (a.kv_len[j] + kBlockTok - 1) / kBlockTok;
            total_chunks += (nb + cb - 1) / cb;
        }
        // an automatic chunk also grows until the launch has at most
        // kAutoItems items (each sequence's last, partial chunk adds one per
        // kv head, and a forced output-dim split doubles them), the same in
        // either workspace; a chunk size the caller set is kept and checked
        // below
        const int64_t auto_items = total_chunks * kKvHeads * (force_split ? kMaxDParts : 1);
        if (total_chunks <= max_chunks && (!auto_cb || auto_items <= kAutoItems)) break;
        cb *= 2;
    }
    int32_t d_parts = 1;
    if (force_split ||
        (!(c->cfg.flags & KVC_FLAG_DECODE_NO_SPLIT_D) && total_chunks * kKvHeads < kDsplitBelowItems))
        d_parts = 2;
    const int64_t items = total_chunks * kKvHeads * d_parts;
    if (items > max_items)
        return set_err(KVC_ERR_RANGE,
                       "decode of sequences %d..%d needs %lld split-K items; the %s holds %lld (use a larger "
                       "decode_chunk_blocks or fewer sequences per call)",
                       seqs[i0], seqs[i0 + n - 1], (long long)items, workspace, (long long)max_items);
    a.chunk_begin[n] = (int32_t)total_chunks;
    a.kpool = reinterpret_cast<const uint16_t*>(c->d_pool + (int64_t)(layer * 2) * c->layer_kv_bytes);
    a.vpool = reinterpret_cast<const uint16_t*>(c->d_pool + (int64_t)(layer * 2 + 1) * c->layer_kv_bytes);
    a.table = c->d_table;
    if (prod.qkv) {
        a.qkv_f32 = prod.in_dtype == KVC_DTYPE_F32;
        a.qkv = static_cast<const uint8_t*>(prod.qkv) + (size_t)i0 * kQkvRow * (a.qkv_f32 ? 4 : 2);
        a.q_norm = static_cast<const float*>(prod.q_norm);
        a.k_norm = static_cast<const float*>(prod.k_norm);
        a.rope = c->d_rope;
        a.eps = c->cfg.rms_norm_eps;
        a.rope_half = c->cfg.rope_dim / 2;
        a.rope_rows = c->cfg.max_seq_len;
    }
    a.q = q ? static_cast<const uint16_t*>(q) + (size_t)i0 * qrow : nullptr;
    a.k_new = k_new ? static_cast<const uint16_t*>(k_new) + (size_t)i0 * kvrow : nullptr;
    a.v_new = v_new ? static_cast<const uint16_t*>(v_new) + (size_t)i0 * kvrow : nullptr;
    a.gate = gate ? static_cast<const uint16_t*>(gate) + (size_t)i0 * qrow : nullptr;
    a.out = static_cast<uint8_t*>(out) + (size_t)i0 * qrow * osz;
    a.part = part;
    a.part_bytes = part_bytes;
    a.counters = counters;
    a.scale_log2 = scale * 1.4426950408889634f;
    a.out_bf16 = out_dtype == KVC_DTYPE_BF16;
    a.table_stride = c->max_blocks;
    a.n_seqs = n;
    a.chunk_blocks = cb;
    a.total_chunks = (int32_t)total_chunks;
    a.d_parts = d_parts;
    a.gate_ref = !(c->cfg.flags & KVC_FLAG_EXACT_MATH);
    a.n_items = (int32_t)items;
    a.per_xcd = (a.n_items + 7) / 8;
    return KVC_OK;
}

// Decode over all seqs, 64 per launch; every launch is validated before the
// first one is made.  Launches of one call run in stream order and share the
// workspace.
static int decode_impl(kvc_ctx* c, int32_t layer, const int32_t* seqs, int32_t n_seqs, const void* q,
                       const void* k_new, const void* v_new, const void* gate, const DecodeProducer& prod,
                       void* out, int32_t out_dtype, float scale, void* stream, float* part, uint32_t part_bytes,
                       int32_t* counters, int64_t max_items, const char* workspace) {
    if (!c) return set_err(KVC_ERR_INVALID, "null context");
    int rc;
    if ((rc = check_device(c)) || (rc = check_layer(c, layer)) || (rc = check_seqs(c, seqs, n_seqs))) return rc;
    if (prod.qkv) {
        if (!prod.q_norm || !prod.k_norm) return set_err(KVC_ERR_INVALID, "decode step needs q_norm and k_norm");
        if (prod.in_dtype != KVC_DTYPE_F32 && prod.in_dtype != KVC_DTYPE_BF16)
            return set_err(KVC_ERR_INVALID, "bad in_dtype");
    } else if (!q) {
        return set_err(KVC_ERR_INVALID, "decode needs q and out");
    }
    if (!out) return set_err(KVC_ERR_INVALID, "decode needs q and out");
    if ((k_new == nullptr) != (v_new == nullptr)) return set_err(KVC_ERR_INVALID, "k_new and v_new go together");
    if (out_dtype != KVC_DTYPE_F32 && out_dtype != KVC_DTYPE_BF16) return set_err(KVC_ERR_INVALID, "bad out_dtype");
    if (!std::isfinite(scale)) return set_err(KVC_ERR_INVALID, "scale must be finite");
    if (!part || !counters) return set_err(KVC_ERR_STATE, "no %s", workspace);
    DecodeArgs a;
    for (int pass = 0; pass < 2; pass++) {
        for (int32_t i0 = 0; i0 < n_seqs; i0 += kMaxBatch) {
            const int32_t n = std::min(kMaxBatch, n_seqs - i0);
            if ((rc = build_decode_args(c, layer, seqs, i0, n, q, k_new, v_new, gate, prod, out, out_dtype, scale,
                                        part, part_bytes, counters, max_items, workspace, a)))
                return rc;
            if (pass == 1) {
                int e = launch_decode(a, stream);
                if (e) return hip_err((hipError_t)e, "decode launch");
            }
        }
    }
    return KVC_OK;
}

int kvc_decode_attn(kvc_ctx* c, int32_t layer, const int32_t* seqs, int32_t n_seqs, const void* q, const void* k_new,
                    const void* v_new, const void* gate, void* out, int32_t out_dtype, float scale, void* stream) {
    return decode_impl(c, layer, seqs, n_seqs, q, k_new, v_new, gate, DecodeProducer{}, out, out_dtype, scale,
                       stream, c ? c->d_part : nullptr, (uint32_t)kPartBytes, c ? c->d_counters : nullptr,
                       (int64_t)kMaxChunks * kKvHeads, "context's split-K workspace");
}

int kvc_decode_step(kvc_ctx* c, int32_t layer, const int32_t* seqs, int32_t n_seqs, const void* qkv,
                    int32_t in_dtype, const void* q_norm, const void* k_norm, void* out, int32_t out_dtype,
                    float scale, void* stream) {
    if (!qkv) return set_err(KVC_ERR_INVALID, "decode step needs qkv");
    DecodeProducer prod;
    prod.qkv = qkv;
    prod.in_dtype = in_dtype;
    prod.q_norm = q_norm;
    prod.k_norm = k_norm;
    return decode_impl(c, layer, seqs, n_seqs, nullptr, nullptr, nullptr, nullptr, prod, out, out_dtype, scale,
                       stream, c ? c->d_part : nullptr, (uint32_t)kPartBytes, c ? c->d_counters : nullptr,
                       (int64_t)kMaxChunks * kKvHeads, "context's split-K workspace");
}

int kvc_decode_attn_static(kvc_ctx* c, int32_t layer, const int32_t* seqs, int32_t n_seqs, const void* q,
                           const void* k_new, const void* v_new, const void* gate, void* out, int32_t out_dtype,
                           float scale, void* stream) {
    return decode_impl(c, layer, seqs, n_seqs, q, k_new, v_new, gate, DecodeProducer{}, out, out_dtype, scale,
                       stream, c ? c->s_part : nullptr, (uint32_t)kStaticPartBytes, c ? c->s_counters : nullptr,
                       kStaticItems, "static decode workspace");
}

// Prefill launches over all seqs, 64 per launch (arguments checked by the
// caller).  With qkv (the prefill step), q and gate come from the projection
// rows instead of q / gate.
static int prefill_launches(kvc_ctx* c, int32_t layer, const int32_t* seqs, int32_t n_seqs, int32_t n_q,
                            const void* q, const void* gate, const void* qkv, int32_t in_dtype, const void* q_norm,
                            void* out, int32_t out_dtype, float scale, void* stream) {
    const size_t qrow = (size_t)n_q * kQHeads * kHeadDim;
    const size_t osz = out_dtype == KVC_DTYPE_BF16 ? 2 : 4;
    const size_t isz = in_dtype == KVC_DTYPE_F32 ? 4 : 2;
    for (int32_t i0 = 0; i0 < n_seqs; i0 += kMaxBatch) {
        const int32_t n = std::min(kMaxBatch, n_seqs - i0);
        PrefillArgs a{};
        for (int32_t j = 0; j < n; j++) {
            const Seq& s = c->seqs[seqs[i0 + j]];
            a.slot[j] = seqs[i0 + j];
            a.q_pos0[j] = s.len + s.pending - n_q;
        }
        a.kpool = reinterpret_cast<const uint16_t*>(c->d_pool + (int64_t)(layer * 2) * c->layer_kv_bytes);
        a.vpool = reinterpret_cast<const uint16_t*>(c->d_pool + (int64_t)(layer * 2 + 1) * c->layer_kv_bytes);
        a.table = c->d_table;
        if (qkv) {
            a.qkv = static_cast<const uint8_t*>(qkv) + (size_t)i0 * n_q * kQkvRow * isz;
            a.qkv_f32 = in_dtype == KVC_DTYPE_F32;
            a.q_norm = static_cast<const float*>(q_norm);
            a.rope = c->d_rope;
            a.eps = c->cfg.rms_norm_eps;
            a.rope_half = c->cfg.rope_dim / 2;
            a.rope_rows = c->cfg.max_seq_len;
        } else {
            a.q = static_cast<const uint16_t*>(q) + (size_t)i0 * qrow;
            a.gate = gate ? static_cast<const uint16_t*>(gate) + (size_t)i0 * qrow : nullptr;
        }
        a.out = static_cast<uint8_t*>(out) + (size_t)i0 * qrow * osz;
        a.scale_log2 = scale * 1.4426950408889634f;
        a.out_bf16 = out_dtype == KVC_DTYPE_BF16;
        a.table_stride = c->max_blocks;
        a.n_seqs = n;
        a.n_q = n_q;
        a.gate_ref = !(c->cfg.flags & KVC_FLAG_EXACT_MATH);
        a.n_groups = n * kKvHeads;
        for (int32_t j = 0; j < n; j++) a.seq_order[j] = j;
        std::stable_sort(a.seq_order, a.seq_order + n,
                         [&](int32_t x, int32_t y) { return a.q_pos0[x] > a.q_pos0[y]; });
        int e = launch_prefill(a, stream);
        if (e) return hip_err((hipError_t)e, "prefill launch");
    }
    return KVC_OK;
}

static int check_prefill(kvc_ctx* c, int32_t layer, const int32_t* seqs, int32_t n_seqs, int32_t n_q, void* out,
                         int32_t out_dtype, float scale) {
    int rc;
    if ((rc = check_device(c)) || (rc = check_layer(c, layer)) || (rc = check_seqs(c, seqs, n_seqs))) return rc;
    if (!out || n_q <= 0) return set_err(KVC_ERR_INVALID, "prefill needs q, out and n_q > 0");
    if (out_dtype != KVC_DTYPE_F32 && out_dtype != KVC_DTYPE_BF16) return set_err(KVC_ERR_INVALID, "bad out_dtype");
    if (!std::isfinite(scale)) return set_err(KVC_ERR_INVALID, "scale must be finite");
    for (int32_t i = 0; i < n_seqs; i++)
        if (c->seqs[seqs[i]].pending < n_q)
            return set_err(KVC_ERR_STATE, "sequence %d: prefill of %d rows but %d reserved", seqs[i], n_q,
                           c->seqs[seqs[i]].pending);
    return KVC_OK;
}

int kvc_prefill_attn(kvc_ctx* c, int32_t layer, const int32_t* seqs, int32_t n_seqs, int32_t n_q, const void* q,
                     const void* gate, void* out, int32_t out_dtype, float scale, void* stream) {
    if (!c) return set_err(KVC_ERR_INVALID, "null context");
    if (!q) return set_err(KVC_ERR_INVALID, "prefill needs q, out and n_q > 0");
    int rc;
    if ((rc = check_prefill(c, layer, seqs, n_seqs, n_q, out, out_dtype, scale))) return rc;
    return prefill_launches(c, layer, seqs, n_seqs, n_q, q, gate, nullptr, KVC_DTYPE_BF16, nullptr, out, out_dtype,
                            scale, stream);
}

int kvc_prefill_step(kvc_ctx* c, int32_t layer, const int32_t* seqs, int32_t n_seqs, int32_t n_q, const void* qkv,
                     int32_t in_dtype, const void* q_norm, const void* k_norm, void* out, int32_t out_dtype,
                     float scale, void* stream) {
    if (!c) return set_err(KVC_ERR_INVALID, "null context");
    if (!qkv || !q_norm || !k_norm) return set_err(KVC_ERR_INVALID, "prefill step needs qkv, q_norm and k_norm");
    if (in_dtype != KVC_DTYPE_F32 && in_dtype != KVC_DTYPE_BF16) return set_err(KVC_ERR_INVALID, "bad in_dtype");
    int rc;
    if ((rc = check_prefill(c, layer, seqs, n_seqs, n_q, out, out_dtype, scale))) return rc;
    // the K/V side of the producer (kvc_qkv_append with no q / gate output),
    // then the attention with q and gate built from the rows
    if ((rc = kvc_qkv_append(c, layer, seqs, n_seqs, n_q, qkv, in_dtype, q_norm, k_norm, nullptr, nullptr, stream)))
        return rc;
    return prefill_launches(c, layer, seqs, n_seqs, n_q, nullptr, nullptr, qkv, in_dtype, q_norm, out, out_dtype,
                            scale, stream);
}

int kvc_gather(kvc_ctx* c, int32_t layer, const int32_t* seqs, int32_t n_seqs, int32_t tok0, const int32_t* n_tok,
               void* k_out, void* v_out, void* stream) {
    if (!c) return set_err(KVC_ERR_INVALID, "null context");
    int rc;
    if ((rc = check_device(c)) || (rc = check_layer(c, layer)) || (rc = check_seqs(c, seqs, n_seqs))) return rc;
    if (!n_tok || !k_out || !v_out || tok0 < 0) return set_err(KVC_ERR_INVALID, "gather needs n_tok and outputs");
    int64_t batch_items = 0;  // work items of the current launch (one per 32 output tokens)
    for (int32_t i = 0; i < n_seqs; i++) {
        const Seq& s = c->seqs[seqs[i]];
        const int32_t nt = n_tok[i];
        if (nt < 0 || (int64_t)tok0 + nt > s.len + s.pending)
            return set_err(KVC_ERR_RANGE, "sequence %d: gather [%d, %d) beyond length %d", seqs[i], tok0, tok0 + nt,
                           s.len + s.pending);
        if (i % kMaxBatch == 0) batch_items = 0;
        batch_items += (nt + kBlockTok - 1) / kBlockTok;
        if (batch_items * kGatherWgsPerItem * 256 > (int64_t)UINT32_MAX)
            return set_err(KVC_ERR_RANGE, "gather too large");
    }
    const size_t row = (size_t)kKvHeads * kHeadDim;
    int64_t out_off = 0;
    for (int32_t i0 = 0; i0 < n_seqs; i0 += kMaxBatch) {
        const int32_t n = std::min(kMaxBatch, n_seqs - i0);
        GatherArgs a{};
        int64_t tot = 0, items = 0;
        for (int32_t j = 0; j < n; j++) {
            const int32_t nt = n_tok[i0 + j];
            a.slot[j] = seqs[i0 + j];
            a.out_begin[j] = (int32_t)tot;
            a.item_begin[j] = (int32_t)items;
            tot += nt;
            items += (nt + kBlockTok - 1) / kBlockTok;
        }
        a.out_begin[n] = (int32_t)tot;
        a.item_begin[n] = (int32_t)items;
        a.n_items = (int32_t)items;
        a.kpool = reinterpret_cast<const uint16_t*>(c->d_pool + (int64_t)(layer * 2) * c->layer_kv_bytes);
        a.vpool = reinterpret_cast<const uint16_t*>(c->d_pool + (int64_t)(layer * 2 + 1) * c->layer_kv_bytes);
        a.table = c->d_table;
        a.k_out = static_cast<uint16_t*>(k_out) + (size_t)out_off * row;
        a.v_out = static_cast<uint16_t*>(v_out) + (size_t)out_off * row;
        a.table_stride = c->max_blocks;
        a.n_seqs = n;
        a.tok0 = tok0;
        a.total_tok = (int32_t)tot;
        if (tot > 0) {
            int e = launch_gather(a, stream);
            if (e) return hip_err((hipError_t)e, "gather launch");
        }
        out_off += tot;
    }
    return KVC_OK;
}

int kvc_kv_checksum(kvc_ctx* c, int32_t layer, const int32_t* seqs, int32_t n_seqs, uint64_t* out, void* stream) {
    if (!c) return set_err(KVC_ERR_INVALID, "null context");
    int rc;
    if ((rc = check_device(c)) || (rc = check_layer(c, layer)) || (rc = check_seqs(c, seqs, n_seqs))) return rc;
    if (!out) return set_err(KVC_ERR_INVALID, "checksum needs an output array");
    int64_t batch_units = 0;  // units of the current launch
    for (int32_t i = 0; i < n_seqs; i++) {
        const Seq& s = c->seqs[seqs[i]];
        if (i % kMaxBatch == 0) batch_units = 0;
        batch_units += (int64_t)((s.len + s.pending + kBlockTok - 1) / kBlockTok) * 2 * kKvHeads;
        if (batch_units > INT32_MAX) return set_err(KVC_ERR_RANGE, "checksum too large");
    }
    int64_t out_off = 0;
    for (int32_t i0 = 0; i0 < n_seqs; i0 += kMaxBatch) {
        const int32_t n = std::min(kMaxBatch, n_seqs - i0);
        ChecksumArgs a{};
        int64_t units = 0;
        for (int32_t j = 0; j < n; j++) {
            const Seq& s = c->seqs[seqs[i0 + j]];
            const int32_t L = s.len + s.pending;
            a.slot[j] = seqs[i0 + j];
            a.kv_len[j] = L;
            a.unit_begin[j] = (int32_t)units;
            units += (int64_t)((L + kBlockTok - 1) / kBlockTok) * 2 * kKvHeads;
        }
        a.unit_begin[n] = (int32_t)units;
        a.kpool = reinterpret_cast<const uint16_t*>(c->d_pool + (int64_t)(layer * 2) * c->layer_kv_bytes);
        a.vpool = reinterpret_cast<const uint16_t*>(c->d_pool + (int64_t)(layer * 2 + 1) * c->layer_kv_bytes);
        a.table = c->d_table;
        a.out = out + out_off;
        a.table_stride = c->max_blocks;
        a.n_seqs = n;
        a.n_units = (int32_t)units;
        if (units > 0) {
            int e = launch_checksum(a, stream);
            if (e) return hip_err((hipError_t)e, "checksum launch");
        }
        out_off += units;
    }
    return KVC_OK;
}

// ---- state + snapshots -------------------------------------------------------

int kvc_state_ptrs(kvc_ctx* c, int32_t seq, int32_t ssm_layer, void** rec, void** conv) {
    if (!c) return set_err(KVC_ERR_INVALID, "null context");
    int rc;
    if ((rc = check_device(c))) return rc;
    if (!seq_ok(c, seq)) return set_err(KVC_ERR_INVALID, "sequence %d is not live", seq);
    if (ssm_layer < 0 || ssm_layer >= c->cfg.n_ssm_layers)
        return set_err(KVC_ERR_RANGE, "ssm layer %d out of range [0, %d)", ssm_layer, c->cfg.n_ssm_layers);
    if (c->seqs[seq].state_dirty) {  // hand out zeros, finished
        if ((rc = clean_states(c, &seq, 1, nullptr))) return rc;
        hipError_t e = hipStreamSynchronize(nullptr);
        if (e != hipSuccess) return hip_err(e, "state zero-fill");
    }
    uint8_t* base = c->d_state + (int64_t)seq * c->state_bytes + (int64_t)ssm_layer * (c->rec_bytes + c->conv_bytes);
    if (rec) *rec = base;
    if (conv) *conv = base + c->rec_bytes;
    return KVC_OK;
}

int kvc_deltanet_step(kvc_ctx* c, int32_t ssm_layer, const int32_t* seqs, int32_t n_seqs, int32_t n_tok,
                      const void* proj, int32_t in_dtype, const void* conv_w, const void* dt_bias, const void* a,
                      const void* norm_w, void* out, int32_t out_dtype, void* stream) {
    if (!c) return set_err(KVC_ERR_INVALID, "null context");
    int rc;
    if ((rc = check_device(c)) || (rc = check_seqs(c, seqs, n_seqs))) return rc;
    const kvc_config& k = c->cfg;
    if (ssm_layer < 0 || ssm_layer >= k.n_ssm_layers)
        return set_err(KVC_ERR_RANGE, "ssm_layer %d out of range [0, %d)", ssm_layer, k.n_ssm_layers);
    if (k.ssm_v_heads != kSsmVHeads || k.ssm_k_dim != kSsmDk || k.ssm_v_dim != kSsmDv ||
        k.conv_rows != kSsmConvRows || k.conv_channels != kSsmC)
        return set_err(KVC_ERR_UNSUPPORTED,
                       "the DeltaNet step is built for %d v-heads, %dx%d heads, %d conv rows, %d channels",
                       kSsmVHeads, kSsmDv, kSsmDk, kSsmConvRows, kSsmC);
    if (!proj || !conv_w || !dt_bias || !a || !norm_w || !out || n_tok <= 0)
        return set_err(KVC_ERR_INVALID, "deltanet step needs proj, weights, out and n_tok > 0");
    if ((in_dtype != KVC_DTYPE_F32 && in_dtype != KVC_DTYPE_BF16) ||
        (out_dtype != KVC_DTYPE_F32 && out_dtype != KVC_DTYPE_BF16))
        return set_err(KVC_ERR_INVALID, "bad in_dtype / out_dtype");
    const size_t isz = in_dtype == KVC_DTYPE_BF16 ? 2 : 4, osz = out_dtype == KVC_DTYPE_BF16 ? 2 : 4;
    // the chunk kernel addresses one seq's rows with 32-bit buffer offsets
    if ((size_t)n_tok * kSsmProj * isz >= ((size_t)1 << 31))
        return set_err(KVC_ERR_RANGE, "n_tok %d: one seq's projection rows exceed 2 GiB", n_tok);
    if ((rc = clean_states(c, seqs, (size_t)n_seqs, stream))) return rc;
    for (int32_t i0 = 0; i0 < n_seqs; i0 += kMaxBatch) {
        const int32_t n = std::min(kMaxBatch, n_seqs - i0);
        DeltaNetArgs d{};
        d.proj = static_cast<const uint8_t*>(proj) + (size_t)i0 * n_tok * kSsmProj * isz;
        d.conv_w = static_cast<const float*>(conv_w);
        d.dt_bias = static_cast<const float*>(dt_bias);
        d.a = static_cast<const float*>(a);
        d.norm_w = static_cast<const float*>(norm_w);
        d.out = static_cast<uint8_t*>(out) + (size_t)i0 * n_tok * kSsmVHeads * kSsmDv * osz;
        d.state = c->d_state;
        d.state_bytes = c->state_bytes;
        d.layer_off = (int64_t)ssm_layer * (c->rec_bytes + c->conv_bytes);
        d.rec_bytes = c->rec_bytes;
        d.eps = k.rms_norm_eps;
        d.out_scale = 1.0f / 11.3137f;  // src/engine.cpp:3251
        d.in_bf16 = in_dtype == KVC_DTYPE_BF16;
        d.out_bf16 = out_dtype == KVC_DTYPE_BF16;
        d.n_seqs = n;
        d.n_tok = n_tok;
        d.ref_math = !(k.flags & KVC_FLAG_EXACT_MATH);
        for (int32_t j = 0; j < n; j++) d.slot[j] = seqs[i0 + j];
        int e = launch_deltanet(d, stream);
        if (e) return hip_err((hipError_t)e, "deltanet launch");
    }
    return KVC_OK;
}

int kvc_snapshot_save(kvc_ctx* c, const int32_t* seqs, int32_t n_seqs, int32_t* snap_ids, void* stream) {
    if (!c || !snap_ids) return set_err(KVC_ERR_INVALID, "null argument");
    int rc;
    if ((rc = check_device(c)) || (rc = check_seqs(c, seqs, n_seqs))) return rc;
    const int iv = c->cfg.snapshot_interval;
    if (iv <= 0 || c->snaps.empty()) return set_err(KVC_ERR_UNSUPPORTED, "snapshots are disabled");
    for (int32_t i = 0; i < n_seqs; i++) {
        const Seq& s = c->seqs[seqs[i]];
        if (s.pending) return set_err(KVC_ERR_STATE, "sequence %d has uncommitted tokens", seqs[i]);
        if (s.len <= 0 || s.len % iv)
            return set_err(KVC_ERR_STATE, "sequence %d length %d is not a positive multiple of %d", seqs[i], s.len, iv);
    }
    // Count the slots first (free, or held by an unpinned snapshot that may
    // be evicted), so that a save that cannot fit fails with no side effect.
    int32_t avail = 0;
    for (const Snapshot& sn : c->snaps) avail += !sn.live || !sn.pinned;
    if (avail < n_seqs)
        return set_err(KVC_ERR_NOMEM, "snapshot pool full: %d slots available, %d needed", avail, n_seqs);
    std::vector<int32_t> ss, sl, fb;
    for (int32_t i = 0; i < n_seqs; i++) {
        const int32_t id = alloc_snapshot(c);  // cannot fail: counted above
        const Seq& s = c->seqs[seqs[i]];
        Snapshot& sn = c->snaps[id];
        sn.live = true;
        sn.pinned = true;
        sn.boundary = s.len;
        sn.tick = ++c->tick;
        if (s.tokens_known) key_snapshot(c, id, s.tokens, s.len);
        ss.push_back(seqs[i]);
        sl.push_back(id);
        fb.push_back((s.len - iv) / kBlockTok);
        snap_ids[i] = id;
    }
    return launch_snapshots(c, ss, sl, fb, false, true, true, stream);
}

int kvc_snapshot_restore(kvc_ctx* c, const int32_t* seqs, const int32_t* snap_ids, int32_t n_seqs, void* stream) {
    if (!c || !snap_ids) return set_err(KVC_ERR_INVALID, "null argument");
    int rc;
    if ((rc = check_device(c)) || (rc = check_seqs(c, seqs, n_seqs))) return rc;
    const int iv = c->cfg.snapshot_interval;
    for (int32_t i = 0; i < n_seqs; i++) {
        const int32_t id = snap_ids[i];
        if (id < 0 || id >= (int32_t)c->snaps.size() || !c->snaps[id].live)
            return set_err(KVC_ERR_INVALID, "snapshot %d is not live", id);
        const Seq& s = c->seqs[seqs[i]];
        if (s.pending) return set_err(KVC_ERR_STATE, "sequence %d has uncommitted tokens", seqs[i]);
        if (s.len < c->snaps[id].boundary - iv)
            return set_err(KVC_ERR_STATE, "sequence %d holds %d tokens; snapshot at %d needs %d", seqs[i], s.len,
                           c->snaps[id].boundary, c->snaps[id].boundary - iv);
    }
    // allocate fresh segment blocks for every pair first
    std::vector<int32_t> granted;
    for (int32_t i = 0; i < n_seqs; i++)
        for (int b = 0; b < c->seg_blocks; b++) {
            const int32_t nb = alloc_block(c);
            if (nb < 0) {
                for (int32_t g : granted) unref_block(c, g);
                return set_err(KVC_ERR_NOMEM, "block pool exhausted during restore");
            }
            granted.push_back(nb);
        }
    std::vector<int32_t> ss, sl, fb;
    for (int32_t i = 0; i < n_seqs; i++) {
        Seq& s = c->seqs[seqs[i]];
        Snapshot& sn = c->snaps[snap_ids[i]];
        const int32_t keep = sn.boundary - iv;
        const bool same_prefix = s.tokens_known && sn.keyed && (int32_t)s.tokens.size() >= keep &&
                                 memcmp(s.tokens.data(), sn.tokens.data(), sizeof(int32_t) * keep) == 0;
        release_tail(c, seqs[i], keep / kBlockTok);
        for (int b = 0; b < c->seg_blocks; b++) {
            const int32_t nb = granted[(size_t)i * c->seg_blocks + b];
            s.blocks.push_back(nb);
            set_table(c, seqs[i], keep / kBlockTok + b, nb);
        }
        s.len = sn.boundary;
        drop_entries(c, s, (size_t)(keep / kBlockTok));
        if (same_prefix) {
            s.tokens = sn.tokens;
            s.tokens_known = true;
        } else {
            s.tokens.clear();
            drop_entries(c, s, 0);
            s.tokens_known = false;
        }
        sn.tick = ++c->tick;
        ss.push_back(seqs[i]);
        sl.push_back(snap_ids[i]);
        fb.push_back(keep / kBlockTok);
    }
    if ((rc = flush_table(c, stream))) return rc;
    if ((rc = launch_snapshots(c, ss, sl, fb, true, true, true, stream))) return rc;
    for (int32_t i = 0; i < n_seqs; i++) {
        Seq& s = c->seqs[seqs[i]];
        if (s.tokens_known) register_blocks(c, s);
    }
    return KVC_OK;
}

int kvc_snapshot_release(kvc_ctx* c, int32_t id) {
    if (!c) return set_err(KVC_ERR_INVALID, "null context");
    if (id < 0 || id >= (int32_t)c->snaps.size() || !c->snaps[id].live)
        return set_err(KVC_ERR_INVALID, "snapshot %d is not live", id);
    Snapshot& sn = c->snaps[id];
    if (sn.keyed) {
        auto it = c->snap_index.find(sn.hash);
        if (it != c->snap_index.end() && it->second == id) c->snap_index.erase(it);
    }
    sn = Snapshot();
    return KVC_OK;
}

// ---- synthetic data + sync ----------------------------------------------------

int kvc_pool_fill_normal(kvc_ctx* c, uint64_t seed, void* stream) {
    if (!c) return set_err(KVC_ERR_INVALID, "null context");
    int rc;
    if ((rc = check_device(c))) return rc;
    const int64_t n = c->layer_kv_bytes * 2 * c->cfg.n_attn_layers / 2;
    int e = launch_fill_normal(reinterpret_cast<uint16_t*>(c->d_pool), n, seed, 1.0f, stream);
    if (e) return hip_err((hipError_t)e, "fill launch");
    return KVC_OK;
}

int kvc_fill_normal_bf16(kvc_ctx* c, void* dst, int64_t n, uint64_t seed, float scale, void* stream) {
    if (!c || !dst || n < 0) return set_err(KVC_ERR_INVALID, "bad fill arguments");
    int rc;
    if ((rc = check_device(c))) return rc;
    if (n == 0) return KVC_OK;
    int e = launch_fill_normal(static_cast<uint16_t*>(dst), n, seed, scale, stream);
    if (e) return hip_err((hipError_t)e, "fill launch");
    return KVC_OK;
}

int kvc_sync(kvc_ctx* c, void* stream) {
    if (!c) return set_err(KVC_ERR_INVALID, "null context");
    if (!c->has_device) return KVC_OK;
    KVC_HIP(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
    return KVC_OK;
}

}  // extern "C"
