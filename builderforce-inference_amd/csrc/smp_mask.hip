// Allow-mask producer of the decode-based constraint (include/bfi_mask.h).
//
// The reference re-decodes the whole generated text for every vocabulary id and rescans the
// concatenation (sample.rs:82-89: V scans of |so_far| + |piece| bytes per step). Here the
// checks of `token_allowed` (sample.rs:92-107) are byte automata: the host runs them once over
// `so_far`, and one GPU thread per id continues the resulting state over its piece, so a step
// reads each piece once (a 16-byte row per id: about 2.5 MB for a 152K vocabulary). Integer
// work, no MFMA.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/bfi_mask.h"
#include "../host/bfi_grammar.hpp"

namespace bfim {

constexpr int BLOCK = 256;

// u8::is_ascii_whitespace (sample.rs:144-206, 236-286): space, \t, \n, form feed, \r.
__host__ __device__ inline bool ascii_ws(uint32_t c) {
    return c == 0x20u || c == 0x09u || c == 0x0Au || c == 0x0Cu || c == 0x0Du;
}

// json_object_prefix_ok (sample.rs:236-286) as an automaton. LEAD: only whitespace so far;
// OBJ: inside the first object (depth >= 1, string and escape flags); AFTER: the object closed,
// whitespace since; DEAD: rejected. The string is accepted unless DEAD (inside OBJ the depth is
// positive, which the reference's final test accepts).
enum : uint8_t { J_LEAD = 0, J_OBJ = 1, J_AFTER = 2, J_DEAD = 3 };
struct JState {
    uint8_t phase;
    uint8_t in_string;
    uint8_t escape;
    int32_t depth;
};
__host__ __device__ inline void j_step(JState& s, uint32_t c) {
    switch (s.phase) {
        case J_LEAD:
            if (ascii_ws(c)) return;
            if (c == '{') {
                s.phase = J_OBJ;
                s.depth = 1;
                s.in_string = 0;
                s.escape = 0;
            } else {
                s.phase = J_DEAD;
            }
            return;
        case J_OBJ:
            if (s.in_string) {
                if (s.escape) s.escape = 0;
                else if (c == '\\') s.escape = 1;
                else if (c == '"') s.in_string = 0;
                return;
            }
            if (c == '"') {
                s.in_string = 1;
            } else if (c == '{' || c == '[') {
                s.depth++;
            } else if (c == '}' || c == ']') {
                if (--s.depth == 0) s.phase = J_AFTER;
            }
            return;
        case J_AFTER:
            if (!ascii_ws(c)) s.phase = J_DEAD;
            return;
        default:
            return;
    }
}

// The per-call tables: tool names, the named tool, the literal's tail (bytes past so_far).
struct Tables {
    int32_t n_names;
    int32_t req_len;   // Named(..) length, -1 when the choice is Required
    int32_t lit_len;   // bytes of the literal tail held in `bytes` (<= the longest piece)
    int32_t lit_rem;   // full length of the literal tail
    uint16_t name_off[BFI_MASK_MAX_TOOL_NAMES + 1];
    uint16_t req_off;
    uint16_t lit_off;
    uint8_t bytes[BFI_MASK_MAX_TABLE_BYTES];
};

// json_name_so_far (sample.rs:144-206) as an automaton. N_SEARCH: looking for `"name"` with
// k bytes of it matched (a mismatch restarts at 1 if the byte is a quote, else 0: the only
// quote of the pattern besides its last byte is its first); N_KEY: the key matched, skipping
// whitespace (z: none skipped yet); N_COLON: after ':', skipping whitespace; N_VALUE: inside the
// value string (esc); N_DONE: the value closed; N_INVALID. A key followed by something other
// than whitespace or ':' resumes the scan one byte after the key's start (sample.rs:160-163):
// of those bytes only the key's closing quote can begin a new match, and only when no
// whitespace followed it. The value's bytes (escapes kept, as the reference slices them) are
// matched against the names as they arrive: req_ok says the value is a prefix of the named
// tool, mask which of the listed names it is a prefix of.
enum : uint8_t { N_SEARCH = 0, N_KEY = 1, N_COLON = 2, N_VALUE = 3, N_DONE = 4, N_INVALID = 5 };
struct NState {
    uint8_t phase;
    uint8_t k;    // N_SEARCH: bytes of `"name"` matched
    uint8_t z;    // N_KEY: no whitespace after the key yet
    uint8_t esc;  // N_VALUE: the previous byte was an unescaped backslash
    uint8_t req_ok;
    int32_t vlen;
    uint64_t mask;
};

__host__ __device__ inline void n_search(NState& s, uint32_t c) {
    const uint8_t pat[6] = {'"', 'n', 'a', 'm', 'e', '"'};
    if (c == pat[s.k]) {
        if (++s.k == 6) {
            s.phase = N_KEY;
            s.z = 1;
        }
    } else {
        s.k = c == '"' ? 1 : 0;
    }
}

__host__ __device__ inline void n_value_byte(NState& s, uint32_t c, const Tables& t) {
    if (s.req_ok) {
        const int32_t rl = t.req_len < 0 ? 0 : t.req_len;
        s.req_ok = (s.vlen < rl && t.bytes[t.req_off + s.vlen] == (uint8_t)c) ? 1 : 0;
    }
    uint64_t m = s.mask;
    while (m) {
        const int j = __builtin_ctzll(m);
        m &= m - 1;
        const int32_t len = (int32_t)t.name_off[j + 1] - (int32_t)t.name_off[j];
        if (s.vlen >= len || t.bytes[t.name_off[j] + s.vlen] != (uint8_t)c) s.mask &= ~(1ull << j);
    }
    s.vlen++;
}

__host__ __device__ inline void n_step(NState& s, uint32_t c, const Tables& t) {
    switch (s.phase) {
        case N_SEARCH:
            n_search(s, c);
            return;
        case N_KEY:
            if (ascii_ws(c)) {
                s.z = 0;
            } else if (c == ':') {
                s.phase = N_COLON;
            } else {  // resume one byte after the key's start
                s.phase = N_SEARCH;
                s.k = s.z ? 1 : 0;
                n_search(s, c);
            }
            return;
        case N_COLON:
            if (ascii_ws(c)) return;
            if (c == '"') {
                s.phase = N_VALUE;
                s.esc = 0;
                s.vlen = 0;
                s.req_ok = 1;
                s.mask = t.n_names >= 64 ? ~0ull : ((1ull << t.n_names) - 1ull);
            } else {
                s.phase = N_INVALID;
            }
            return;
        case N_VALUE:
            if (s.esc) {
                s.esc = 0;
            } else if (c == '\\') {
                s.esc = 1;
            } else if (c == '"') {
                s.phase = N_DONE;
                return;
            }
            n_value_byte(s, c, t);
            return;
        default:
            return;
    }
}

// tool_call_prefix_ok's verdict on the name (sample.rs:117-135) at the end of the string.
__host__ __device__ inline bool n_accept(const NState& s, const Tables& t) {
    switch (s.phase) {
        case N_VALUE:  // Partial
            if (t.req_len >= 0) return s.req_ok;
            return t.n_names == 0 || s.mask != 0;
        case N_DONE: {  // Complete
            if (t.req_len >= 0) return s.req_ok && s.vlen == t.req_len;
            if (t.n_names == 0) return true;
            uint64_t m = s.mask;
            while (m) {
                const int j = __builtin_ctzll(m);
                m &= m - 1;
                if ((int32_t)t.name_off[j + 1] - (int32_t)t.name_off[j] == s.vlen) return true;
            }
            return false;
        }
        case N_INVALID:
            return false;
        default:  // Missing, or Partial("") right after the colon
            return true;
    }
}

enum : int32_t { M_ALL = 0, M_SCAN = 1, M_NONE = 2 };

struct MaskArgs {
    const uint8_t* bytes;
    const uint32_t* off;
    const uint4* rows;  // per id: up to 15 bytes of its piece, byte 15 its length (LONG: longer)
    uint32_t* mask;
    int64_t V;
    int32_t mode;
    int32_t json_on;  // json_object || tool choice constrains (sample.rs:94)
    int32_t tool_on;  // tool choice constrains (sample.rs:97)
    int32_t lit_on;   // grammar is a literal (sample.rs:103-105)
    int32_t lit_ok;   // so_far is a prefix of the literal
    JState j0;        // states after so_far
    NState n0;
    Tables t;
};

constexpr uint32_t LONG = 0xFFu;  // length byte of a piece longer than 15 bytes

// One thread per id; a wave's 64 verdicts become two mask words by ballot. A piece of at most
// 15 bytes comes with its length in one 16-byte row (consecutive ids, consecutive rows: one
// coalesced load per thread, no offset lookup first); longer pieces are read from the text.
__global__ __launch_bounds__(BLOCK) void k_mask(const MaskArgs a) {
    const int64_t id = (int64_t)blockIdx.x * BLOCK + threadIdx.x;
    bool ok = false;
    if (id < a.V && a.mode != M_NONE) {
        ok = true;
        if (a.mode == M_SCAN) {
            const uint4 row = a.rows[id];
            const uint32_t len = row.w >> 24;
            uint32_t b0 = 0, n = len;
            if (len == LONG) {
                b0 = a.off[id];
                n = a.off[id + 1] - b0;
            }
            auto byte_at = [&](uint32_t i) -> uint32_t {
                if (len == LONG) return a.bytes[b0 + i];
                const uint32_t wsel = i >> 2;
                const uint32_t word = wsel == 0 ? row.x : wsel == 1 ? row.y : wsel == 2 ? row.z : row.w;
                return (word >> (8 * (i & 3u))) & 0xFFu;
            };
            if (a.lit_on) {
                ok = a.lit_ok && (int64_t)n <= (int64_t)a.t.lit_rem && (int32_t)n <= a.t.lit_len;
                for (uint32_t i = 0; ok && i < n; i++) ok = byte_at(i) == a.t.bytes[a.t.lit_off + i];
            }
            if (ok && a.json_on) {
                JState js = a.j0;
                NState ns = a.n0;
                for (uint32_t i = 0; i < n; i++) {
                    const uint32_t c = byte_at(i);
                    j_step(js, c);
                    if (a.tool_on) n_step(ns, c, a.t);
                }
                ok = js.phase != J_DEAD && (!a.tool_on || n_accept(ns, a.t));
            }
        }
    }
    const uint64_t bal = __ballot(ok);
    const int lane = threadIdx.x & 63;
    const int64_t w0 = (id - lane) >> 5;  // the wave's first word
    const int64_t nw = (a.V + 31) >> 5;
    if (lane == 0 && w0 < nw) a.mask[w0] = (uint32_t)bal;
    if (lane == 32 && w0 + 1 < nw) a.mask[w0 + 1] = (uint32_t)(bal >> 32);
}

// ---- host: the grammar string (host/bfi_grammar.hpp, shared with bfi_parse_id_union) ----

using bfig::parse_id_union;
using bfig::parse_literal_root;

}  // namespace bfim

using namespace bfim;

struct bfi_mask_ctx {
    int device = 0;
    std::string err;
    uint8_t* d_bytes = nullptr;
    uint32_t* d_off = nullptr;
    uint4* d_rows = nullptr;
    int64_t V = -1;
    int64_t max_piece = 0;
    std::vector<uint32_t> host_mask;  // id unions
};

namespace {

int fail(bfi_mask_ctx* ctx, int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (ctx) ctx->err = buf;
    return code;
}
int hfail(bfi_mask_ctx* ctx, hipError_t e, const char* what) {
    return fail(ctx, BFI_SMP_EHIP, "%s: %s", what, hipGetErrorString(e));
}

}  // namespace

extern "C" {

int bfi_mask_create(int device, bfi_mask_ctx** out) {
    if (!out) return BFI_SMP_EINVAL;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return BFI_SMP_EHIP;
    bfi_mask_ctx* c = new (std::nothrow) bfi_mask_ctx;
    if (!c) return BFI_SMP_ENOMEM;
    c->device = device;
    *out = c;
    return BFI_SMP_OK;
}

void bfi_mask_destroy(bfi_mask_ctx* ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->d_bytes) (void)hipFree(ctx->d_bytes);
    if (ctx->d_off) (void)hipFree(ctx->d_off);
    if (ctx->d_rows) (void)hipFree(ctx->d_rows);
    delete ctx;
}

const char* bfi_mask_error(const bfi_mask_ctx* ctx) { return ctx ? ctx->err.c_str() : "null context"; }

int bfi_mask_set_vocab(bfi_mask_ctx* ctx, const uint8_t* bytes, const int64_t* offsets, int64_t n_vocab) {
    if (!ctx) return BFI_SMP_EINVAL;
    if (n_vocab < 0 || n_vocab > ((int64_t)1 << 24) || !offsets)
        return fail(ctx, BFI_SMP_EINVAL, "n_vocab out of range or offsets NULL");
    if (offsets[0] != 0) return fail(ctx, BFI_SMP_EINVAL, "offsets[0] must be 0");
    int64_t maxp = 0;
    for (int64_t i = 0; i < n_vocab; i++) {
        const int64_t n = offsets[i + 1] - offsets[i];
        if (n < 0) return fail(ctx, BFI_SMP_EINVAL, "offsets decrease at %lld", (long long)i);
        maxp = n > maxp ? n : maxp;
    }
    const int64_t total = offsets[n_vocab];
    if (total > (int64_t)0xFFFFFF00ll) return fail(ctx, BFI_SMP_EINVAL, "vocabulary text of 4 GiB or more");
    if (total > 0 && !bytes) return fail(ctx, BFI_SMP_EINVAL, "bytes is NULL");
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return hfail(ctx, e, "hipSetDevice");
    if (ctx->d_bytes) (void)hipFree(ctx->d_bytes);
    if (ctx->d_off) (void)hipFree(ctx->d_off);
    if (ctx->d_rows) (void)hipFree(ctx->d_rows);
    ctx->d_bytes = nullptr;
    ctx->d_off = nullptr;
    ctx->d_rows = nullptr;
    ctx->V = -1;
    std::vector<uint32_t> off32((size_t)n_vocab + 1);
    for (int64_t i = 0; i <= n_vocab; i++) off32[(size_t)i] = (uint32_t)offsets[i];
    // 16 bytes of padding past the text
    if ((e = hipMalloc((void**)&ctx->d_bytes, (size_t)total + 16)) != hipSuccess ||
        (e = hipMalloc((void**)&ctx->d_off, off32.size() * sizeof(uint32_t))) != hipSuccess)
        return fail(ctx, BFI_SMP_ENOMEM, "vocabulary allocation failed: %s", hipGetErrorString(e));
    if (total > 0 && (e = hipMemcpy(ctx->d_bytes, bytes, (size_t)total, hipMemcpyHostToDevice)) != hipSuccess)
        return hfail(ctx, e, "hipMemcpy(vocabulary bytes)");
    if ((e = hipMemcpy(ctx->d_off, off32.data(), off32.size() * sizeof(uint32_t), hipMemcpyHostToDevice)) !=
        hipSuccess)
        return hfail(ctx, e, "hipMemcpy(vocabulary offsets)");
    // the 16-byte rows: up to 15 bytes of the piece, its length in the last byte
    std::vector<uint8_t> rows((size_t)(n_vocab > 0 ? n_vocab : 1) * 16, 0);
    for (int64_t i = 0; i < n_vocab; i++) {
        const int64_t n = offsets[i + 1] - offsets[i];
        uint8_t* r = rows.data() + (size_t)i * 16;
        if (n <= 15) {
            if (n > 0) memcpy(r, bytes + offsets[i], (size_t)n);
            r[15] = (uint8_t)n;
        } else {
            r[15] = (uint8_t)LONG;
        }
    }
    if ((e = hipMalloc((void**)&ctx->d_rows, rows.size())) != hipSuccess)
        return fail(ctx, BFI_SMP_ENOMEM, "vocabulary rows allocation failed: %s", hipGetErrorString(e));
    if ((e = hipMemcpy(ctx->d_rows, rows.data(), rows.size(), hipMemcpyHostToDevice)) != hipSuccess)
        return hfail(ctx, e, "hipMemcpy(vocabulary rows)");
    ctx->V = n_vocab;
    ctx->max_piece = maxp;
    return BFI_SMP_OK;
}

int bfi_mask_build(bfi_mask_ctx* ctx, const uint8_t* so_far, int64_t so_far_len, const bfi_constraint* c,
                   uint32_t* d_mask, int32_t* constrained, void* stream) {
    if (!ctx) return BFI_SMP_EINVAL;
    if (!c || !d_mask || so_far_len < 0 || (so_far_len > 0 && !so_far))
        return fail(ctx, BFI_SMP_EINVAL, "NULL argument or negative length");
    if (ctx->V < 0) return fail(ctx, BFI_SMP_EINVAL, "no vocabulary (bfi_mask_set_vocab)");
    if (c->tool_choice < BFI_TOOL_NONE || c->tool_choice > BFI_TOOL_NAMED)
        return fail(ctx, BFI_SMP_EINVAL, "tool_choice %d out of range", c->tool_choice);
    const int64_t V = ctx->V;
    hipStream_t st = (hipStream_t)stream;
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return hfail(ctx, e, "hipSetDevice");
    const bool constrains = c->tool_choice == BFI_TOOL_REQUIRED || c->tool_choice == BFI_TOOL_NAMED;
    const bool has_grammar = c->grammar != nullptr;
    std::string g;
    if (has_grammar) {
        if (c->grammar_len < 0) return fail(ctx, BFI_SMP_EINVAL, "grammar_len < 0");
        g.assign((const char*)c->grammar, (size_t)c->grammar_len);
    }
    MaskArgs a;  // about 3.3 KB with its tables, passed by value (kernel arguments)
    memset(&a, 0, sizeof a);
    a.bytes = ctx->d_bytes;
    a.off = ctx->d_off;
    a.rows = ctx->d_rows;
    a.mask = d_mask;
    a.V = V;
    a.mode = M_SCAN;
    if (constrained) *constrained = 1;
    if (!has_grammar && !c->json_object && !constrains) {  // sample.rs:69-71
        a.mode = M_ALL;
        if (constrained) *constrained = 0;
    } else {
        std::vector<uint32_t> ids;
        if (has_grammar && parse_id_union(g, &ids)) {  // sample.rs:72-80
            const size_t nw = (size_t)((V + 31) / 32);
            ctx->host_mask.assign(nw, 0u);
            for (uint32_t id : ids)
                if ((int64_t)id < V) ctx->host_mask[id >> 5] |= 1u << (id & 31);
            if (nw == 0) return BFI_SMP_OK;
            e = hipMemcpyAsync(d_mask, ctx->host_mask.data(), nw * 4, hipMemcpyHostToDevice, st);
            if (e == hipSuccess) e = hipStreamSynchronize(st);  // the host buffer is reused
            return e == hipSuccess ? BFI_SMP_OK : hfail(ctx, e, "hipMemcpyAsync(id union)");
        }
        std::string lit;
        a.lit_on = has_grammar && parse_literal_root(g, &lit);
        a.json_on = c->json_object || constrains;
        a.tool_on = constrains;
        // the tables
        Tables& t = a.t;
        size_t used = 0;
        auto put = [&](const uint8_t* p, size_t n, uint16_t* at) -> bool {
            if (used + n > (size_t)BFI_MASK_MAX_TABLE_BYTES) return false;
            if (at) *at = (uint16_t)used;
            if (n) memcpy(t.bytes + used, p, n);
            used += n;
            return true;
        };
        t.req_len = -1;
        if (constrains) {
            if (c->n_tool_names < 0 || c->n_tool_names > BFI_MASK_MAX_TOOL_NAMES)
                return fail(ctx, BFI_SMP_EINVAL, "%d tool names (at most %d)", c->n_tool_names,
                            BFI_MASK_MAX_TOOL_NAMES);
            if (c->n_tool_names > 0 && (!c->tool_names || !c->tool_name_lens))
                return fail(ctx, BFI_SMP_EINVAL, "tool_names NULL");
            t.n_names = c->n_tool_names;
            for (int j = 0; j < c->n_tool_names; j++) {
                if (c->tool_name_lens[j] < 0 || (c->tool_name_lens[j] > 0 && !c->tool_names[j]) ||
                    !put(c->tool_names[j], (size_t)c->tool_name_lens[j], &t.name_off[j]))
                    return fail(ctx, BFI_SMP_EINVAL, "tool names exceed %d bytes", BFI_MASK_MAX_TABLE_BYTES);
            }
            t.name_off[c->n_tool_names] = (uint16_t)used;
            if (c->tool_choice == BFI_TOOL_NAMED) {
                if (c->tool_name_len < 0 || (c->tool_name_len > 0 && !c->tool_name) ||
                    !put(c->tool_name, (size_t)c->tool_name_len, &t.req_off))
                    return fail(ctx, BFI_SMP_EINVAL, "named tool exceeds the table");
                t.req_len = (int32_t)c->tool_name_len;
            }
        }
        if (a.lit_on) {
            const bool pre = (int64_t)lit.size() >= so_far_len &&
                             (so_far_len == 0 || memcmp(lit.data(), so_far, (size_t)so_far_len) == 0);
            a.lit_ok = pre;
            const size_t rem = pre ? lit.size() - (size_t)so_far_len : 0;
            const size_t keep = rem < (size_t)ctx->max_piece ? rem : (size_t)ctx->max_piece;
            t.lit_rem = (int32_t)rem;
            t.lit_len = (int32_t)keep;
            if (!put((const uint8_t*)lit.data() + (pre ? so_far_len : 0), keep, &t.lit_off))
                return fail(ctx, BFI_SMP_EINVAL, "literal tail (%zu bytes) exceeds the table", keep);
        }
        // the states after so_far (sample.rs:82, 93)
        a.j0 = JState{J_LEAD, 0, 0, 0};
        a.n0 = NState{N_SEARCH, 0, 0, 0, 0, 0, 0};
        for (int64_t i = 0; i < so_far_len; i++) {
            j_step(a.j0, so_far[i]);
            if (a.tool_on) n_step(a.n0, so_far[i], t);
        }
        // Past a decision in so_far the verdict no longer depends on the piece: a rejected
        // object or name rejects every id; a decided name leaves only the object check.
        if (a.json_on && a.j0.phase == J_DEAD) a.mode = M_NONE;
        if (a.tool_on && (a.n0.phase == N_DONE || a.n0.phase == N_INVALID)) {
            if (n_accept(a.n0, t)) a.tool_on = 0;
            else a.mode = M_NONE;
        }
        if (a.lit_on && !a.lit_ok) a.mode = M_NONE;
    }
    if (V == 0) return BFI_SMP_OK;
    const unsigned grid = (unsigned)((V + BLOCK - 1) / BLOCK);
    hipLaunchKernelGGL(k_mask, dim3(grid), dim3(BLOCK), 0, st, a);
    e = hipGetLastError();
    return e == hipSuccess ? BFI_SMP_OK : hfail(ctx, e, "k_mask launch");
}

}  // extern "C"
