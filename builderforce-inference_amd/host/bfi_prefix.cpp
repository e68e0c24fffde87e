// bfi_prefix.cpp — the prefix cache of include/bfi_prefix.h: a byte-bounded LRU of sequence
// states keyed by token prefix (crates/bfi-runtime/src/engine/prefix.rs), the states kept in
// one device allocation per entry.
//
// Lookup is O(prompt length) on the host: one rolling hash over the prompt, probed against
// marks at every BFI_PC_BLOCK-token boundary of rewindable entries and at every entry's end,
// then a token-by-token check of the deepest candidates (a hash collision never restores the
// wrong state). The bytes of an entry are counted as the reference counts them: 4 per token,
// 4 per logit, the kept rows of every K/V tensor, whole tensors and recurrent tensors.
#include "../../include/bfi_prefix.h"

#include <hip/hip_runtime.h>

#include "../csrc/pc_copy.h"

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

namespace {

constexpr uint64_t BLOCK = BFI_PC_BLOCK;

// Rolling prefix hash: h(ids[..n+1]) = hstep(h(ids[..n]), ids[n]). Marks only select
// candidates; every candidate is confirmed by comparing tokens.
constexpr uint64_t HSEED = 0x243f6a8885a308d3ull;
inline uint64_t hstep(uint64_t h, uint32_t t) {
    uint64_t z = (h ^ ((uint64_t)t * 0x9e3779b97f4a7c15ull)) + 0x632be59bd9b4e019ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

uint64_t common_prefix(const uint32_t* a, uint64_t na, const uint32_t* b, uint64_t nb) {
    const uint64_t n = std::min(na, nb);
    uint64_t i = 0;
    while (i < n && a[i] == b[i]) i++;
    return i;
}

// One kept tensor: `bytes` at `off` in the entry's block; row_bytes > 0: `rows` kept rows.
struct Part {
    uint64_t off = 0, bytes = 0, row_bytes = 0, rows = 0;
    bool present = false;  // (a recurrent slot: the layer has state)
};

struct Entry {
    std::vector<uint32_t> tokens;
    std::vector<Part> kv, rec;
    Part logits;
    uint64_t n_logits = 0;
    void* block = nullptr;
    bool rewindable = true;
    uint64_t bytes = 0, last_used = 0;
    std::vector<uint64_t> marks;
};

}  // namespace

struct bfi_pc {
    int device = -1;
    uint64_t budget = 0, used = 0, next_id = 0, tick = 0, forwarded = 0;
    std::unordered_map<uint64_t, Entry> entries;
    std::unordered_map<uint64_t, std::vector<uint64_t>> marks;
    std::string err;
};

namespace {

int fail(const bfi_pc* pc, int code, const char* fmt, ...) {
    if (pc) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        const_cast<bfi_pc*>(pc)->err = buf;
    }
    return code;
}

int hip_fail(const bfi_pc* pc, hipError_t e, const char* what) {
    return fail(pc, BFI_SMP_EHIP, "%s: %s", what, hipGetErrorString(e));
}

void free_block(bfi_pc* pc, void* p) {
    if (!p) return;
    if (pc->device >= 0) (void)hipFree(p);
    else std::free(p);
}

// The copies of one insert or restore, run together: host memory by memcpy / memset; device
// memory in batched launches (pc_copy.hip) when every range is 16-byte aligned, else one
// hipMemcpyAsync / hipMemsetAsync per range.
struct Xfer {
    std::vector<bfi::PcRange> r;
    void add(void* dst, const void* src, uint64_t copy, uint64_t zero) {
        if (copy || zero) r.push_back(bfi::PcRange{src, dst, copy, zero});
    }
};

int run_xfer(bfi_pc* pc, const Xfer& x, hipStream_t s) {
    if (pc->device < 0) {
        for (const auto& r : x.r) {
            if (r.copy_bytes) std::memcpy(r.dst, r.src, r.copy_bytes);
            if (r.zero_bytes) std::memset((char*)r.dst + r.copy_bytes, 0, r.zero_bytes);
        }
        return BFI_SMP_OK;
    }
    bool aligned = true;
    for (const auto& r : x.r) aligned = aligned && bfi::pc_range_aligned(r);
    if (aligned) {
        for (size_t i = 0; i < x.r.size(); i += bfi::PC_MAX_RANGES) {
            const int n = (int)std::min(x.r.size() - i, (size_t)bfi::PC_MAX_RANGES);
            const hipError_t e = bfi::pc_copy_launch(x.r.data() + i, n, s);
            if (e != hipSuccess) return hip_fail(pc, e, "prefix cache copy launch");
        }
        return BFI_SMP_OK;
    }
    for (const auto& r : x.r) {
        hipError_t e = hipSuccess;
        if (r.copy_bytes) e = hipMemcpyAsync(r.dst, r.src, r.copy_bytes, hipMemcpyDeviceToDevice, s);
        if (e == hipSuccess && r.zero_bytes) e = hipMemsetAsync((char*)r.dst + r.copy_bytes, 0, r.zero_bytes, s);
        if (e != hipSuccess) return hip_fail(pc, e, "prefix cache copy");
    }
    return BFI_SMP_OK;
}

// prefix.rs:335-347 `remove`
void remove_entry(bfi_pc* pc, uint64_t id) {
    auto it = pc->entries.find(id);
    if (it == pc->entries.end()) return;
    Entry& e = it->second;
    pc->used -= e.bytes;
    for (uint64_t m : e.marks) {
        auto mt = pc->marks.find(m);
        if (mt == pc->marks.end()) continue;
        auto& list = mt->second;
        list.erase(std::remove(list.begin(), list.end(), id), list.end());
        if (list.empty()) pc->marks.erase(mt);
    }
    free_block(pc, e.block);
    pc->entries.erase(it);
}

// prefix.rs:324-333 `evict_lru`
bool evict_lru(bfi_pc* pc) {
    if (pc->entries.empty()) return false;
    uint64_t oldest = 0, when = UINT64_MAX;
    for (const auto& kv : pc->entries)
        if (kv.second.last_used < when) {
            when = kv.second.last_used;
            oldest = kv.first;
        }
    remove_entry(pc, oldest);
    return true;
}

// prefix.rs:310-322 `drop_superseded`: an identical sequence, or (both rewindable) a cached
// prefix of the new one.
void drop_superseded(bfi_pc* pc, const uint32_t* tokens, uint64_t n, bool rewindable) {
    std::vector<uint64_t> doomed;
    for (const auto& kv : pc->entries) {
        const Entry& e = kv.second;
        const bool same = e.tokens.size() == n && std::equal(e.tokens.begin(), e.tokens.end(), tokens);
        const bool covered = rewindable && e.rewindable && e.tokens.size() <= n &&
                             std::equal(e.tokens.begin(), e.tokens.end(), tokens);
        if (same || covered) doomed.push_back(kv.first);
    }
    for (uint64_t id : doomed) remove_entry(pc, id);
}

bool valid_tensor(const bfi_pc_tensor& t) { return t.data != nullptr || t.rows == 0; }

}  // namespace

extern "C" {

int bfi_pc_create(int device, uint64_t budget_bytes, bfi_pc** out) {
    if (!out) return BFI_SMP_EINVAL;
    *out = nullptr;
    if (device < -1) return BFI_SMP_EINVAL;
    if (device >= 0) {
        const hipError_t e = hipSetDevice(device);
        if (e != hipSuccess) return BFI_SMP_EHIP;
    }
    bfi_pc* pc = new (std::nothrow) bfi_pc;
    if (!pc) return BFI_SMP_ENOMEM;
    pc->device = device;
    pc->budget = budget_bytes;
    *out = pc;
    return BFI_SMP_OK;
}

void bfi_pc_destroy(bfi_pc* pc) {
    if (!pc) return;
    bfi_pc_clear(pc);
    delete pc;
}

const char* bfi_pc_last_error(const bfi_pc* pc) { return pc ? pc->err.c_str() : "null cache"; }

int bfi_pc_lookup(const bfi_pc* pc, const uint32_t* ids, uint64_t n_ids, bfi_pc_hit* hit, int* found) {
    if (!pc || !hit || !found || (n_ids && !ids)) return fail(pc, BFI_SMP_EINVAL, "bfi_pc_lookup: null argument");
    *found = 0;
    // deepest probe first: one pass over the prompt collects every (length, entry) its
    // prefix hashes name
    std::vector<std::pair<uint64_t, uint64_t>> probes;
    uint64_t h = HSEED;
    for (uint64_t i = 0; i < n_ids; i++) {
        h = hstep(h, ids[i]);
        auto mt = pc->marks.find(h);
        if (mt == pc->marks.end()) continue;
        for (uint64_t id : mt->second) probes.emplace_back(i + 1, id);
    }
    bool have = false;
    uint64_t best_m = 0, best_id = 0;
    for (auto it = probes.rbegin(); it != probes.rend(); ++it) {
        const uint64_t len = it->first, id = it->second;
        if (have && best_m >= len + BLOCK) break;  // nothing shallower can extend past the best
        auto et = pc->entries.find(id);
        if (et == pc->entries.end()) continue;
        const Entry& e = et->second;
        if (e.tokens.size() < len || !std::equal(e.tokens.begin(), e.tokens.begin() + len, ids)) continue;
        uint64_t matched;
        if (e.rewindable) matched = len + common_prefix(e.tokens.data() + len, e.tokens.size() - len, ids + len, n_ids - len);
        else if (len == e.tokens.size()) matched = len;
        else continue;  // a recurrent state cannot resume mid-entry
        if (!have || matched > best_m) {
            have = true;
            best_m = matched;
            best_id = id;
        }
    }
    // a share shorter than one block reaches no boundary mark: compare the first tokens of
    // every rewindable entry directly (equal shares found this way go to the oldest entry; the
    // reference leaves them to its hash map's iteration order)
    if (!have || best_m < BLOCK) {
        bool direct = false;
        for (const auto& kv : pc->entries) {
            const Entry& e = kv.second;
            if (!e.rewindable) continue;
            const uint64_t m = common_prefix(e.tokens.data(), e.tokens.size(), ids, n_ids);
            if (m > 0 && (!have || m > best_m || (direct && m == best_m && kv.first < best_id))) {
                have = true;
                direct = true;
                best_m = m;
                best_id = kv.first;
            }
        }
    }
    if (!have) return BFI_SMP_OK;
    const Entry& e = pc->entries.at(best_id);
    const uint64_t restore = best_m == e.tokens.size() ? best_m : std::min(best_m, n_ids ? n_ids - 1 : 0);
    if (restore == 0) return BFI_SMP_OK;
    *hit = bfi_pc_hit{best_id, best_m, restore};
    *found = 1;
    return BFI_SMP_OK;
}

int bfi_pc_restore(bfi_pc* pc, const bfi_pc_hit* hit, const bfi_pc_state* dst, uint64_t* n, int* logits_restored,
                   int* found, void* stream) {
    if (!pc || !hit || !dst || !n || !logits_restored || !found)
        return fail(pc, BFI_SMP_EINVAL, "bfi_pc_restore: null argument");
    *found = 0;
    *logits_restored = 0;
    pc->tick++;
    auto et = pc->entries.find(hit->id);
    if (et == pc->entries.end()) return BFI_SMP_OK;
    Entry& e = et->second;
    // the destination must hold what was inserted
    if (dst->n_kv != e.kv.size() || dst->n_rec != e.rec.size() || (dst->n_kv && !dst->kv) || (dst->n_rec && !dst->rec))
        return fail(pc, BFI_SMP_EINVAL, "bfi_pc_restore: %llu K/V and %llu recurrent tensors, the entry has %zu and %zu",
                    (unsigned long long)dst->n_kv, (unsigned long long)dst->n_rec, e.kv.size(), e.rec.size());
    for (size_t i = 0; i < e.kv.size(); i++) {
        const bfi_pc_tensor& t = dst->kv[i];
        const Part& p = e.kv[i];
        const bool ok = t.data && t.row_bytes == p.row_bytes && (p.row_bytes ? t.rows >= p.rows : t.rows == p.bytes);
        if (!ok) return fail(pc, BFI_SMP_EINVAL, "bfi_pc_restore: K/V tensor %zu does not match the entry's layout", i);
    }
    for (size_t i = 0; i < e.rec.size(); i++)
        if (e.rec[i].present && (!dst->rec[i].data || dst->rec[i].rows != e.rec[i].bytes))
            return fail(pc, BFI_SMP_EINVAL, "bfi_pc_restore: recurrent tensor %zu does not match the entry's", i);
    const bool with_logits = hit->restore == e.tokens.size();
    if (with_logits && e.n_logits && (!dst->logits || dst->n_logits != e.n_logits))
        return fail(pc, BFI_SMP_EINVAL, "bfi_pc_restore: %llu logits, the entry has %llu",
                    (unsigned long long)dst->n_logits, (unsigned long long)e.n_logits);
    e.last_used = pc->tick;
    char* blk = (char*)e.block;
    Xfer x;
    for (size_t i = 0; i < e.kv.size(); i++) {
        const bfi_pc_tensor& t = dst->kv[i];
        const Part& p = e.kv[i];
        x.add(t.data, blk + p.off, p.bytes, p.row_bytes ? t.rows * t.row_bytes - p.bytes : 0);
    }
    for (size_t i = 0; i < e.rec.size(); i++)
        if (e.rec[i].present) x.add(dst->rec[i].data, blk + e.rec[i].off, e.rec[i].bytes, 0);
    if (with_logits) x.add(dst->logits, blk + e.logits.off, e.logits.bytes, 0);
    const int rc = run_xfer(pc, x, (hipStream_t)stream);
    if (rc != BFI_SMP_OK) return rc;
    *logits_restored = with_logits ? 1 : 0;
    *n = hit->restore;
    *found = 1;
    return BFI_SMP_OK;
}

int bfi_pc_insert(bfi_pc* pc, const uint32_t* tokens, uint64_t n_tokens, const bfi_pc_state* st, void* stream) {
    if (!pc || !st || (n_tokens && !tokens)) return fail(pc, BFI_SMP_EINVAL, "bfi_pc_insert: null argument");
    if (n_tokens == 0 || st->n != n_tokens) return BFI_SMP_OK;  // (prefix.rs:234, 249)
    if ((st->n_kv && !st->kv) || (st->n_rec && !st->rec) || (st->n_logits && !st->logits))
        return fail(pc, BFI_SMP_EINVAL, "bfi_pc_insert: null tensor array");
    for (uint64_t i = 0; i < st->n_kv; i++)
        if (!valid_tensor(st->kv[i])) return fail(pc, BFI_SMP_EINVAL, "bfi_pc_insert: K/V tensor %llu has no data", (unsigned long long)i);
    // the entry's layout: kept rows of each K/V tensor, the recurrent tensors, the logits
    Entry e;
    uint64_t off = 0, data_bytes = 0;
    auto place = [&](uint64_t bytes) {
        const uint64_t o = off;
        off += (bytes + 255u) & ~(uint64_t)255u;
        data_bytes += bytes;
        return o;
    };
    e.kv.resize(st->n_kv);
    for (uint64_t i = 0; i < st->n_kv; i++) {
        const bfi_pc_tensor& t = st->kv[i];
        Part& p = e.kv[i];
        p.row_bytes = t.row_bytes;
        p.rows = t.row_bytes ? std::min(st->n, t.rows) : 0;
        p.bytes = t.row_bytes ? p.rows * t.row_bytes : t.rows;
        p.present = true;
        p.off = place(p.bytes);
    }
    e.rec.resize(st->n_rec);
    e.rewindable = true;
    for (uint64_t i = 0; i < st->n_rec; i++) {
        const bfi_pc_tensor& t = st->rec[i];
        Part& p = e.rec[i];
        p.present = t.data != nullptr;
        if (!p.present) continue;
        e.rewindable = false;  // (prefix.rs:270)
        p.bytes = t.row_bytes ? t.rows * t.row_bytes : t.rows;
        p.off = place(p.bytes);
    }
    e.n_logits = st->n_logits;
    e.logits.bytes = st->n_logits * sizeof(float);
    e.logits.off = place(e.logits.bytes);
    e.bytes = n_tokens * sizeof(uint32_t) + data_bytes;
    if (e.bytes > pc->budget) return BFI_SMP_OK;  // larger than the whole budget: not cached
    drop_superseded(pc, tokens, n_tokens, e.rewindable);
    while (pc->used + e.bytes > pc->budget)
        if (!evict_lru(pc)) break;
    // the copies
    if (off) {
        if (pc->device >= 0) {
            const hipError_t he = hipMalloc(&e.block, off);
            if (he != hipSuccess) {
                e.block = nullptr;
                return fail(pc, BFI_SMP_ENOMEM, "bfi_pc_insert: %llu bytes of device memory: %s", (unsigned long long)off,
                            hipGetErrorString(he));
            }
        } else {
            e.block = std::malloc(off);
            if (!e.block) return fail(pc, BFI_SMP_ENOMEM, "bfi_pc_insert: %llu bytes of host memory", (unsigned long long)off);
        }
    }
    char* blk = (char*)e.block;
    Xfer x;
    for (uint64_t i = 0; i < st->n_kv; i++) x.add(blk + e.kv[i].off, st->kv[i].data, e.kv[i].bytes, 0);
    for (uint64_t i = 0; i < st->n_rec; i++)
        if (e.rec[i].present) x.add(blk + e.rec[i].off, st->rec[i].data, e.rec[i].bytes, 0);
    x.add(blk + e.logits.off, st->logits, e.logits.bytes, 0);
    const int rc = run_xfer(pc, x, (hipStream_t)stream);
    if (rc != BFI_SMP_OK) {
        free_block(pc, e.block);
        return rc;
    }
    // marks: every BLOCK boundary (rewindable entries resume anywhere) and the end
    e.tokens.assign(tokens, tokens + n_tokens);
    uint64_t h = HSEED;
    for (uint64_t i = 0; i < n_tokens; i++) {
        h = hstep(h, tokens[i]);
        const uint64_t len = i + 1;
        if (len == n_tokens || (e.rewindable && len % BLOCK == 0)) e.marks.push_back(h);
    }
    pc->tick++;
    e.last_used = pc->tick;
    const uint64_t id = pc->next_id++;
    for (uint64_t m : e.marks) pc->marks[m].push_back(id);
    pc->used += e.bytes;
    pc->entries.emplace(id, std::move(e));
    return BFI_SMP_OK;
}

uint64_t bfi_pc_used_bytes(const bfi_pc* pc) { return pc ? pc->used : 0; }
uint64_t bfi_pc_len(const bfi_pc* pc) { return pc ? pc->entries.size() : 0; }
void bfi_pc_note_forward(bfi_pc* pc, uint64_t n) {
    if (pc) pc->forwarded += n;
}
uint64_t bfi_pc_forwarded(const bfi_pc* pc) { return pc ? pc->forwarded : 0; }

void bfi_pc_clear(bfi_pc* pc) {
    if (!pc) return;
    for (auto& kv : pc->entries) free_block(pc, kv.second.block);
    pc->entries.clear();
    pc->marks.clear();
    pc->used = 0;
}

}  // extern "C"
