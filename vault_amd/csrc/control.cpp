// Host control logic of the decode loop, next to the device hot path:
//   * segment-memory resonance: a shingle index over the segment bank's tokens and, per step, the
//     per-token attention biases that the biased heads add on the segment span;
//   * the authority-spoof quarantine of the segment scorer;
//   * the output governor, which masks continuations that would spell a forbidden rule.
// All three read token byte strings (the VLT3 VTOK table) and small integer state; none touches
// the KV cache.  The device side gives them their inputs (token ids, the bank's tokens and segment
// ids, the top candidates of a logits row) and takes their outputs (bias rows, a score override,
// the ids to mask).
//
// Reference semantics: runtime/vault3.c:142-151 (the double logarithm of the posting weights),
// 1034-1176 (byte normalisation and tagged FNV-1a shingles), 1178-1260 (index over the bank's
// segments), 1262-1786 (query resonance, clause refinement, continuation halo), 1798-1831 (spoof
// quarantine), 2329-2349 (strict UTF-8 decoding), 2814-3193 (governor); the reference's Python model
// states the same rules (src/vault_v3_model.py:397-560, 1249-1830).  The rules, constants and
// capacities are the reference's: the outputs must be the same bits.
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <new>
#include <vector>

#include "vault_amd.h"

namespace {

constexpr uint32_t kNone = 0xFFFFFFFFu;

// ---------------------------------------------------------------- token byte strings
}  // namespace

struct vgx_tokens {
    std::vector<uint8_t> pool;
    std::vector<uint64_t> off;   // n + 1 offsets into pool
    uint32_t n = 0;
    bool get(uint32_t id, const uint8_t *&b, uint32_t &len) const {
        if (id >= n) {
            b = nullptr;
            len = 0;
            return false;
        }
        b = pool.data() + off[id];
        len = (uint32_t)(off[id + 1] - off[id]);
        return true;
    }
    bool has_byte(uint32_t id, uint8_t ch) const {
        const uint8_t *b;
        uint32_t bl;
        if (!get(id, b, bl)) return false;
        for (uint32_t i = 0; i < bl; ++i)
            if (b[i] == ch) return true;
        return false;
    }
};

namespace {

// ln(x) for normal x > 0 as the reference computes it (runtime/vault3.c:142-151): x = m 2^e with m in
// [1, 2), halved above sqrt(2); ln m = 2 atanh(s), s = (m - 1) / (m + 1), from the first 30 odd terms
// of the series, in this order.  The posting weights round mult * ln^2 to integers, so the same
// double arithmetic is needed, not merely a correct logarithm.
double log_series(double x) {
    uint64_t u;
    std::memcpy(&u, &x, 8);
    int e = (int)((u >> 52) & 0x7FF) - 1023;
    u = (u & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull;
    double m;
    std::memcpy(&m, &u, 8);
    if (m > 1.4142135623730951) {
        m *= 0.5;
        e += 1;
    }
    const double s = (m - 1.0) / (m + 1.0), s2 = s * s;
    double term = s, sum = 0.0;
    for (int i = 1; i < 60; i += 2) {
        sum += term / (double)i;
        term *= s2;
    }
    return 2.0 * sum + (double)e * 0.69314718055994530942;
}

// ---------------------------------------------------------------- normalised text and shingles

// A byte buffer of normalised text: lower-case [0-9a-z_-] runs separated by single spaces.  Index 0
// is always a space, so "the previous byte" is defined; bytes past cap - 2 are dropped.
struct NormText {
    std::vector<uint8_t> b;
    uint32_t n = 0;
    uint32_t cap = 0;
    explicit NormText(uint32_t c = 0) : b(c + 1), cap(c) {}
    void start() {
        n = 0;
        b[n++] = ' ';
    }
    void add(const uint8_t *p, uint32_t len) {
        for (uint32_t i = 0; i < len; ++i) {
            uint8_t c = p[i];
            if (c >= 'A' && c <= 'Z') c = (uint8_t)(c + 32u);
            const bool keep = (c >= '0' && c <= '9') || (c >= 'a' && c <= 'z') || c == '_' || c == '-';
            if (keep) {
                if (n + 2u < cap) b[n++] = c;
            } else if (b[n - 1u] != ' ') {
                if (n + 2u < cap) b[n++] = ' ';
            }
        }
    }
    void add_token(const vgx_tokens &t, uint32_t id) {
        const uint8_t *p;
        uint32_t len;
        if (t.get(id, p, len)) add(p, len);
    }
    void close() {
        if (b[n - 1u] != ' ' && n < cap) b[n++] = ' ';
    }
};

inline uint32_t fnv_step(uint32_t h, uint8_t c) { return (h ^ (uint32_t)c) * 16777619u; }

// FNV-1a of a word framed by a space on each side.
uint32_t word_hash(const uint8_t *p, uint32_t len) {
    uint32_t h = fnv_step(2166136261u, ' ');
    for (uint32_t i = 0; i < len; ++i) h = fnv_step(h, p[i]);
    return fnv_step(h, ' ');
}

bool id_char(uint8_t c) { return (c >= '0' && c <= '9') || c == '_' || c == '-'; }

bool word_is(const uint8_t *p, uint32_t len, const char *w) {
    return std::strlen(w) == len && std::memcmp(p, w, len) == 0;
}

// Words of five or more letters that carry no content in a question (plus four-letter ones that
// the hyphenated-compound rule tests).
bool stopword(const uint8_t *p, uint32_t len) {
    static const char *const kWords[] = {
        "what", "with", "only", "from", "that", "this", "into", "find",
        "which", "where", "there", "their", "about", "after", "under", "above", "state", "reply", "exact",
        "value", "query", "using", "token", "first", "other", "these", "those", "would", "could",
        "before", "string", "single", "should", "active",
        "current", "through", "between",
        "original", "assigned"};
    if (len < 4 || len > 8) return false;
    for (const char *w : kWords)
        if (word_is(p, len, w)) return true;
    return false;
}

// Tagged shingles of normalised text, sorted ascending and unique (runtime/vault3.c:1099-1176):
//   low bits 01: 4-byte sub-shingle of an identifier (a word with letters and digits / '_');
//   low bits 11: a whole identifier, or a one-letter word followed by a 1-3 digit number ("t 5");
//   low bits 00: a content word of five or more letters (not a stopword), or the parts and the whole
//                of a hyphenated compound of such parts.
uint32_t shingles(const NormText &t, uint32_t *out, uint32_t max_out) {
    const uint8_t *s = t.b.data();
    const uint32_t nl = t.n;
    if (nl < 4u || max_out == 0u) return 0u;
    uint32_t cnt = 0, i = 0;
    while (i < nl && cnt < max_out) {
        if (s[i] == ' ') {
            ++i;
            continue;
        }
        const uint32_t l = i;
        bool alpha = false, numus = false, hyph = false;
        for (; i < nl && s[i] != ' '; ++i) {
            const uint8_t c = s[i];
            if (c >= 'a' && c <= 'z') alpha = true;
            else if ((c >= '0' && c <= '9') || c == '_') numus = true;
            else if (c == '-') hyph = true;
        }
        const uint32_t r = i, len = r - l;
        if (len >= 3u && alpha && numus) {
            const bool trail = r < nl;       // a byte (the separating space) follows the word
            if (trail || len >= 4u) {
                const uint32_t k_end = trail ? r - 3u : r - 4u;
                for (uint32_t k = l; k <= k_end && cnt < max_out; ++k) {
                    if (!id_char(s[k]) && !id_char(s[k + 1]) && !id_char(s[k + 2]) && !id_char(s[k + 3])) continue;
                    uint32_t h = 2166136261u;
                    for (int q = 0; q < 4; ++q) h = fnv_step(h, s[k + q]);
                    out[cnt++] = (h | 1u) & ~2u;
                }
            }
            if (cnt < max_out) out[cnt++] = word_hash(s + l, len) | 3u;
        } else if (len == 1u && alpha && !numus && r + 1u < nl) {
            uint32_t nl0 = r + 1u;
            while (nl0 < nl && s[nl0] == ' ') ++nl0;
            uint32_t nr = nl0;
            bool digits = true;
            for (; nr < nl && s[nr] != ' '; ++nr)
                if (!(s[nr] >= '0' && s[nr] <= '9')) digits = false;
            if (digits && nr - nl0 >= 1u && nr - nl0 <= 3u && nl0 == r + 1u && cnt < max_out)
                out[cnt++] = word_hash(s + l, nr - l) | 3u;
        } else if (!numus && alpha && len >= 5u) {
            if (!hyph) {
                if (!stopword(s + l, len) && cnt < max_out) out[cnt++] = word_hash(s + l, len) & ~3u;
            } else {
                uint32_t p0 = l, parts = 0;
                bool parts_ok = true;
                for (uint32_t k = l; k <= r; ++k) {
                    if (k == r || s[k] == '-') {
                        const uint32_t plen = k - p0;
                        ++parts;
                        if (plen < 4u || stopword(s + p0, plen)) parts_ok = false;
                        if (plen >= 5u && !stopword(s + p0, plen) && cnt < max_out)
                            out[cnt++] = word_hash(s + p0, plen) & ~3u;
                        p0 = k + 1u;
                    }
                }
                if (parts >= 2u && parts_ok && cnt < max_out) out[cnt++] = word_hash(s + l, len) & ~3u;
            }
        }
    }
    if (cnt <= 1u) return cnt;
    std::sort(out, out + cnt);
    return (uint32_t)(std::unique(out, out + cnt) - out);
}

// murmur3's 32-bit finaliser: the probe start of a shingle in the open-addressing index.
uint32_t slot_hash(uint32_t k) {
    k ^= k >> 16;
    k *= 0x85ebca6bu;
    k ^= k >> 13;
    k *= 0xc2b2ae35u;
    k ^= k >> 16;
    return k;
}

bool in_sorted(const uint32_t *a, uint32_t n, uint32_t x) { return std::binary_search(a, a + n, x); }

// First position of needle in hay, or -1.
int32_t find_sub(const uint8_t *hay, uint32_t hlen, const char *needle) {
    const uint32_t nlen = (uint32_t)std::strlen(needle);
    if (hlen < nlen || nlen == 0u) return -1;
    for (uint32_t i = 0; i + nlen <= hlen; ++i)
        if (std::memcmp(hay + i, needle, nlen) == 0) return (int32_t)i;
    return -1;
}

int32_t rollback_cue(const uint8_t *lc, uint32_t n) {
    for (const char *kw : {"rollback", "revert", "restore"}) {
        const int32_t p = find_sub(lc, n, kw);
        if (p >= 0) return p;
    }
    const int32_t p = find_sub(lc, n, "roll ");
    if (p >= 0 && find_sub(lc + p, n - (uint32_t)p, " back") >= 0) return p;
    return -1;
}

}  // namespace

// ---------------------------------------------------------------- resonance state
struct vgx_resonance {
    const vgx_tokens *tok;
    uint32_t window, seg_cap, n_sink, im_start, im_end;
    // shingle index: open addressing over cap (a power of two) keys; postings as linked lists
    uint32_t cap, post_cap;
    std::vector<uint64_t> keys;
    std::vector<uint32_t> df, head, last_sid;
    std::vector<uint32_t> post_sid, post_w, post_next;
    uint32_t n_post = 0;
    // the bank the index describes
    std::vector<uint32_t> mem_tok, mem_seg, seg_inv;
    uint32_t mem_cnt = 0, n_segs = 0;
    bool indexed = false;
    // per-query scratch
    std::vector<uint32_t> q_scores, q_hits, q_matched;
    std::vector<uint64_t> q_mask;
    std::vector<float> seg_arch, seg_sup, seg_hop1;
    std::vector<uint32_t> q_sh, piv_sh, cl_sh, seg_sh;
    NormText nt_query{4096}, nt_seg{8192}, nt_clause{2048}, nt_pivot{4096}, nt_halo{512};
    std::vector<uint8_t> raw_lc, raw_cl;

    uint32_t probe(uint32_t key) const {
        const uint32_t mask = cap - 1u;
        uint32_t slot = slot_hash(key) & mask;
        while (keys[slot] != ~0ull && keys[slot] != (uint64_t)key) slot = (slot + 1u) & mask;
        return slot;
    }
    bool found(uint32_t slot) const { return keys[slot] != ~0ull; }
    uint32_t tok_at(const uint32_t *prev, const uint32_t *cur, uint32_t idx) const {
        return idx < window ? prev[idx] : cur[idx - window];
    }
    void segment_text(uint32_t &j, uint32_t sid) {
        nt_seg.start();
        while (j < mem_cnt && seg_inv[j] == sid) nt_seg.add_token(*tok, mem_tok[j++]);
        nt_seg.close();
    }
    void rebuild();
    int update(const uint32_t *prev, const uint32_t *cur, uint32_t c, uint64_t pos, uint32_t n_pin, float *arch,
               float *sup, float *hop1);
    void refine(uint32_t n_m, uint32_t n_q, bool tier_a, float sib_val, float *arch, float *sup);
};

// Document frequencies of the shingles over the bank's distinct segments, then postings (segment,
// integer weight) for the selective ones (runtime/vault3.c:1178-1260).
void vgx_resonance::rebuild() {
    indexed = false;
    n_post = 0;
    if (mem_cnt == 0u) {
        n_segs = 0;
        return;
    }
    uint32_t ns = 0;
    for (uint32_t j = 0; j < mem_cnt; ++j) {
        if (j > 0 && mem_seg[j] != mem_seg[j - 1]) ++ns;
        seg_inv[j] = ns;
    }
    n_segs = ns + 1;
    if (n_segs <= 2u) return;
    std::fill(keys.begin(), keys.end(), ~0ull);
    uint32_t used = 0;
    uint32_t j = 0;
    for (uint32_t sid = 0; sid < n_segs; ++sid) {
        segment_text(j, sid);
        const uint32_t n = shingles(nt_seg, seg_sh.data(), 2048u);
        for (uint32_t k = 0; k < n; ++k) {
            const uint32_t key = seg_sh[k], slot = probe(key);
            if (!found(slot)) {
                if (used + 1u >= cap) break;
                keys[slot] = key;
                df[slot] = 1;
                head[slot] = kNone;
                last_sid[slot] = sid;
                ++used;
            } else if (last_sid[slot] != sid) {
                ++df[slot];
                last_sid[slot] = sid;
            }
        }
    }
    j = 0;
    for (uint32_t sid = 0; sid < n_segs; ++sid) {
        segment_text(j, sid);
        const uint32_t n = shingles(nt_seg, seg_sh.data(), 2048u);
        for (uint32_t k = 0; k < n; ++k) {
            const uint32_t key = seg_sh[k], slot = probe(key);
            if (!found(slot) || n_post >= post_cap) continue;
            const uint32_t d = df[slot];
            const bool is_id = (key & 1u) != 0u;
            const bool keep = is_id ? (((key & 3u) == 3u && d == 2u) || (uint64_t)d * 4u <= (uint64_t)n_segs + 6u)
                                    : (d <= 16u && (uint64_t)d * 5u <= (uint64_t)n_segs * 2u + 4u);
            if (!keep) continue;
            const double lg = log_series(((double)n_segs + 1.0) / ((double)d + 0.5));
            const double mult = (key & 3u) == 3u ? 2048.0 : (is_id ? 1024.0 : 768.0);
            post_sid[n_post] = sid;
            post_w[n_post] = (uint32_t)(mult * lg * lg + 0.5);
            post_next[n_post] = head[slot];
            head[slot] = n_post++;
        }
    }
    indexed = true;
}

// Sub-clauses of the matched segments (split at '\n' '|' '\t' ';' tokens) that score well below the
// best clause of their segment are set back to the sibling value (runtime/vault3.c:1307-1424).
void vgx_resonance::refine(uint32_t n_m, uint32_t n_q, bool tier_a, float sib_val, float *arch, float *sup) {
    auto in_tier = [&](uint32_t h) { return tier_a ? (h & 1u) != 0u : (h & 3u) == 0u; };
    bool any = false;
    for (uint32_t qi = 0; qi < n_q && !any; ++qi) {
        const uint32_t h = q_sh[qi];
        if (!in_tier(h)) continue;
        const uint32_t slot = probe(h);
        any = found(slot) && head[slot] != kNone;
    }
    if (!any) return;
    uint32_t cl_beg[32], cl_end[32], cl_sc[32];
    bool cl_ok[32];
    for (uint32_t mi = 0; mi < n_m; ++mi) {
        const uint32_t sid = q_matched[mi];
        uint32_t kb = mem_cnt, ke = 0;
        for (uint32_t k = 0; k < mem_cnt; ++k)
            if (seg_inv[k] == sid) {
                kb = std::min(kb, k);
                ke = k + 1u;
            }
        if (ke <= kb || ke - kb < 8u) continue;
        uint32_t n_cl = 0, c0 = kb;
        for (uint32_t k = kb; k < ke; ++k) {
            const uint8_t *b;
            uint32_t bl;
            bool delim = false;
            if (tok->get(mem_tok[k], b, bl))
                for (uint32_t i = 0; i < bl && !delim; ++i)
                    delim = b[i] == '\n' || b[i] == '|' || b[i] == '\t' || b[i] == ';';
            if (delim && k - c0 + 1u >= 4u && ke - (k + 1u) >= 4u && n_cl + 1u < 32u) {
                cl_beg[n_cl] = c0;
                cl_end[n_cl++] = k + 1u;
                c0 = k + 1u;
            }
        }
        if (c0 < ke && n_cl < 32u) {
            cl_beg[n_cl] = c0;
            cl_end[n_cl++] = ke;
        }
        if (n_cl < 2u) continue;
        uint32_t best = 0;
        for (uint32_t ci = 0; ci < n_cl; ++ci) {
            nt_clause.start();
            for (uint32_t k = cl_beg[ci]; k < cl_end[ci]; ++k) nt_clause.add_token(*tok, mem_tok[k]);
            nt_clause.close();
            const uint32_t n_c = shingles(nt_clause, cl_sh.data(), 512u);
            uint32_t n_tier = 0, sc = 0;
            for (uint32_t si = 0; si < n_c; ++si) {
                const uint32_t h = cl_sh[si];
                if (!in_tier(h)) continue;
                ++n_tier;
                if (!in_sorted(q_sh.data(), n_q, h)) continue;
                const uint32_t slot = probe(h);
                if (!found(slot)) continue;
                for (uint32_t p = head[slot]; p != kNone; p = post_next[p])
                    if (post_sid[p] == sid) {
                        sc += post_w[p];
                        break;
                    }
            }
            // the clause's raw bytes, trailing separators dropped: a key = value clause?
            uint32_t rcl = 0;
            for (uint32_t k = cl_beg[ci]; k < cl_end[ci]; ++k) {
                const uint8_t *b;
                uint32_t bl;
                if (tok->get(mem_tok[k], b, bl))
                    for (uint32_t i = 0; i < bl && rcl < 2048u; ++i) raw_cl[rcl++] = b[i];
            }
            while (rcl > 0u) {
                const uint8_t ch = raw_cl[rcl - 1u];
                if (ch == ' ' || ch == '\t' || ch == '\r' || ch == '\n' || ch == '|' || ch == ',' || ch == ';') --rcl;
                else break;
            }
            bool kv = false;
            if (rcl > 2u)
                for (uint32_t i = 0; i + 1u < rcl && !kv; ++i) kv = raw_cl[i] == '=' || raw_cl[i] == ':';
            const uint32_t clen = cl_end[ci] - cl_beg[ci];
            cl_sc[ci] = sc;
            cl_ok[ci] = (clen >= 9u || kv) && n_tier >= 2u;
            best = std::max(best, sc);
        }
        if (best == 0u) continue;
        bool weaker = false;
        for (uint32_t ci = 0; ci < n_cl; ++ci)
            if (cl_sc[ci] < best && cl_ok[ci]) weaker = true;
        if (!weaker) continue;
        for (uint32_t ci = 0; ci < n_cl; ++ci)
            if ((uint64_t)cl_sc[ci] * 4u < (uint64_t)best * 3u && cl_ok[ci])
                for (uint32_t k = cl_beg[ci]; k < cl_end[ci]; ++k) arch[k] = sup[k] = sib_val;
    }
}

// One step's query resonance (runtime/vault3.c:1426-1786).  Returns the mode: 0 = no bias, 1 = the
// arch / sup biases, 2 = those plus the hop-1 bias of the early biased layers.
int vgx_resonance::update(const uint32_t *prev, const uint32_t *cur, uint32_t c, uint64_t pos, uint32_t n_pin,
                          float *arch, float *sup, float *hop1) {
    const uint32_t M = mem_cnt, N = n_segs, W = window;
    if (M == 0u || N <= 2u || !indexed) return 0;
    // the query: the last user line before an <|im_end|> at most 37 tokens back, outside the pins
    const uint32_t hi = W + c;
    const uint32_t lo_search = hi >= 127u ? hi - 127u : 0u;
    int32_t p_end = -1;
    for (int32_t p = (int32_t)hi; p >= (int32_t)lo_search; --p)
        if (tok_at(prev, cur, (uint32_t)p) == im_end) {
            p_end = p;
            break;
        }
    if (p_end <= 0) return 0;
    const uint32_t gen = hi - (uint32_t)p_end;
    if (gen >= 38u) return 0;
    if (pos - (uint64_t)gen < (uint64_t)n_pin) return 0;
    const float atten = gen <= 18u ? 1.0f : (float)(38u - gen) * 0.05f;
    const uint32_t from = (uint32_t)p_end - 1u;
    const uint32_t stop = from >= 48u ? from - 48u : 0u;
    uint32_t lo_t = stop;
    for (int32_t p = (int32_t)from; p >= (int32_t)stop; --p) {
        const uint32_t id = tok_at(prev, cur, (uint32_t)p);
        if (id == im_start || ((uint32_t)p + 4u <= from && tok->has_byte(id, '\n'))) {
            lo_t = (uint32_t)p + 1u;
            break;
        }
    }
    if (lo_t > from) return 0;
    nt_query.start();
    for (uint32_t t = lo_t; t <= from; ++t) nt_query.add_token(*tok, tok_at(prev, cur, t));
    nt_query.close();
    const uint32_t n_q = shingles(nt_query, q_sh.data(), 1024u);
    if (n_q < 2u) return 0;
    uint32_t n_q_id = 0, n_q_alpha = 0;
    for (uint32_t qi = 0; qi < n_q; ++qi) ((q_sh[qi] & 1u) ? n_q_id : n_q_alpha)++;

    const uint64_t whole = 1ull << 63, qbits = whole - 1ull;
    uint32_t mx = 0, n_m = 0, max_hits = 0;
    bool tier_a = false;
    // accumulate the postings of the query shingles that `take` selects, each with its query bit
    auto score = [&](auto take, bool tag_whole) {
        std::fill(q_scores.begin(), q_scores.begin() + N, 0u);
        std::fill(q_hits.begin(), q_hits.begin() + N, 0u);
        std::fill(q_mask.begin(), q_mask.begin() + N, 0ull);
        mx = 0;
        uint32_t bit_i = 0;
        for (uint32_t qi = 0; qi < n_q; ++qi) {
            const uint32_t kh = q_sh[qi];
            if (!take(kh)) continue;
            const uint64_t bit = (1ull << (bit_i % 63u)) | ((tag_whole && (kh & 3u) == 3u) ? whole : 0ull);
            ++bit_i;
            const uint32_t slot = probe(kh);
            if (!found(slot)) continue;
            for (uint32_t p = head[slot]; p != kNone; p = post_next[p]) {
                const uint32_t sid = post_sid[p];
                q_scores[sid] += post_w[p];
                ++q_hits[sid];
                q_mask[sid] |= bit;
                mx = std::max(mx, q_scores[sid]);
            }
        }
    };
    // tier A: identifier shingles, whenever the query holds two or more
    if (n_q_id >= 2u) {
        score([](uint32_t h) { return (h & 1u) != 0u; }, true);
        if (mx >= 2048u) {
            uint32_t n_top = 0;
            uint64_t top_whole = 0, top_bits = 0;
            for (uint32_t sid = 0; sid < N; ++sid)
                if (q_hits[sid] >= 2u && q_scores[sid] == mx) {
                    ++n_top;
                    top_whole |= q_mask[sid] & whole;
                    top_bits |= q_mask[sid] & qbits;
                }
            for (uint32_t sid = 0; sid < N; ++sid) {
                if (q_hits[sid] < 2u || (uint64_t)q_scores[sid] * 2u < (uint64_t)mx) continue;
                const uint64_t ms = q_mask[sid];
                // one best segment that carries a whole identifier: drop the ones whose query bits it
                // covers without one of their own
                if (n_top == 1u && top_whole && !(ms & whole) && !((ms & qbits) & ~top_bits)) continue;
                q_matched[n_m++] = sid;
            }
            tier_a = n_m > 0u;
        }
    }
    // tier B: content words, when tier A matched nothing
    if (n_m == 0u && n_q_alpha >= 2u) {
        score([](uint32_t h) { return (h & 3u) == 0u; }, false);
        if (mx >= 2500u) {
            uint32_t n_top = 0, hits_top = 0;
            uint64_t top_bits = 0;
            for (uint32_t sid = 0; sid < N; ++sid)
                if (q_hits[sid] >= 2u && q_scores[sid] == mx) {
                    ++n_top;
                    top_bits |= q_mask[sid] & qbits;
                    hits_top = std::max(hits_top, q_hits[sid]);
                }
            for (uint32_t sid = 0; sid < N; ++sid) {
                const bool close = hits_top >= 3u ? (uint64_t)q_scores[sid] * 4u >= (uint64_t)mx * 3u
                                                  : (uint64_t)q_scores[sid] * 2u >= (uint64_t)mx;
                if (q_hits[sid] < 2u || !close) continue;
                const uint64_t ms = q_mask[sid] & qbits;
                if (n_top == 1u && q_scores[sid] < mx && !(ms & ~top_bits)) continue;
                q_matched[n_m++] = sid;
                max_hits = std::max(max_hits, q_hits[sid]);
            }
        }
    }
    if (n_m == 0u) return 0;

    float bg = 0.0f;
    if (!tier_a && max_hits >= 3u) {
        const float shift = M > 1024u ? (float)log_series((double)M * (1.0 / 1024.0)) : 0.0f;
        bg = -(1.0f + shift);
    }
    std::fill(seg_arch.begin(), seg_arch.begin() + N, bg);
    std::fill(seg_sup.begin(), seg_sup.begin() + N, bg);
    std::fill(seg_hop1.begin(), seg_hop1.begin() + N, 0.0f);

    int mode = 1;
    const uint32_t pivot = q_matched[n_m - 1u];
    uint32_t rlen = 0;
    for (uint32_t j = 0; j < M; ++j) {
        if (seg_inv[j] != pivot) continue;
        const uint8_t *b;
        uint32_t bl;
        if (tok->get(mem_tok[j], b, bl))
            for (uint32_t i = 0; i < bl && rlen < 4096u; ++i) {
                const uint8_t ch = b[i];
                raw_lc[rlen++] = (ch >= 'A' && ch <= 'Z') ? (uint8_t)(ch + 32u) : ch;
            }
    }
    // whole-identifier shingles of some pivot text that the query does not hold
    auto pivot_ids = [&](uint32_t from_byte) {
        nt_pivot.start();
        nt_pivot.add(raw_lc.data() + from_byte, rlen - from_byte);
        nt_pivot.close();
        return shingles(nt_pivot, piv_sh.data(), 1024u);
    };
    // case 1: a rollback cue in the pivot segment points at an earlier segment
    int32_t rb = -1;
    const int32_t cue = rollback_cue(raw_lc.data(), rlen);
    if (cue >= 0 && pivot > 0u) {
        const int32_t to = find_sub(raw_lc.data() + cue, rlen - (uint32_t)cue, " to ");
        uint32_t starts[2], n_st = 0;
        if (to >= 0) starts[n_st++] = (uint32_t)(cue + to);
        starts[n_st++] = (uint32_t)cue;
        for (uint32_t si = 0; si < n_st && rb < 0; ++si) {
            const uint32_t n_p = pivot_ids(starts[si]);
            for (uint32_t pi = 0; pi < n_p; ++pi) {
                const uint32_t kh = piv_sh[pi];
                if ((kh & 3u) != 3u || in_sorted(q_sh.data(), n_q, kh)) continue;
                const uint32_t slot = probe(kh);
                if (!found(slot) || df[slot] > 3u) continue;
                for (uint32_t p = head[slot]; p != kNone; p = post_next[p]) {
                    const uint32_t cs = post_sid[p];
                    if (cs < pivot && (int32_t)cs > rb) rb = (int32_t)cs;
                }
            }
        }
    }
    // case 2: one tier-A match whose whole identifiers bridge (df == 2) to at most two other segments
    uint32_t hop2[2] = {0, 0}, n_hop2 = 0;
    if (rb < 0 && n_m == 1u && tier_a) {
        const uint32_t s0 = q_matched[0];
        const uint32_t n_p = pivot_ids(0);
        bool overflow = false;
        for (uint32_t pi = 0; pi < n_p; ++pi) {
            const uint32_t kh = piv_sh[pi];
            if ((kh & 3u) != 3u || in_sorted(q_sh.data(), n_q, kh)) continue;
            const uint32_t slot = probe(kh);
            if (!found(slot) || df[slot] != 2u) continue;
            for (uint32_t p = head[slot]; p != kNone; p = post_next[p]) {
                const uint32_t cs = post_sid[p];
                if (cs == s0) continue;
                bool dup = false;
                for (uint32_t h2 = 0; h2 < n_hop2; ++h2) dup = dup || hop2[h2] == cs;
                if (dup) continue;
                if (n_hop2 < 2u) hop2[n_hop2++] = cs;
                else overflow = true;
            }
        }
        if (overflow) n_hop2 = 0;
    }

    const uint32_t pin_thr = std::max(n_sink, 16u);
    const bool sys_pin = n_pin > pin_thr;
    if (rb >= 0) {
        mode = 2;
        std::fill(seg_arch.begin(), seg_arch.begin() + N, 0.0f);
        std::fill(seg_sup.begin(), seg_sup.begin() + N, 0.0f);
        for (uint32_t mi = 0; mi < n_m; ++mi) {
            const uint32_t sid = q_matched[mi];
            seg_hop1[sid] = -0.3f;
            seg_arch[sid] = 0.4f;
            seg_sup[sid] = -0.5f;
        }
        const uint32_t r = (uint32_t)rb;
        seg_hop1[pivot] = 2.0f;
        seg_hop1[r] = 2.0f;
        seg_arch[pivot] = 1.2f;
        seg_arch[r] = 2.2f;
        seg_sup[pivot] = 0.8f;
        seg_sup[r] = 2.8f;
    } else if (n_hop2 > 0u) {
        mode = 2;
        std::fill(seg_arch.begin(), seg_arch.begin() + N, 0.0f);
        std::fill(seg_sup.begin(), seg_sup.begin() + N, 0.0f);
        const uint32_t s0 = q_matched[0];
        seg_hop1[s0] = 2.4f;
        seg_arch[s0] = 1.0f;
        seg_sup[s0] = 0.6f;
        for (uint32_t h2 = 0; h2 < n_hop2; ++h2) {
            seg_hop1[hop2[h2]] = 1.0f;
            seg_arch[hop2[h2]] = 2.4f;
            seg_sup[hop2[h2]] = 2.8f;
        }
    } else if (n_m == 1u) {
        const uint32_t s0 = q_matched[0];
        if (!tier_a) {
            float ba = max_hits >= 3u ? 2.2f : 0.5f, bs = max_hits >= 3u ? 2.5f : 0.7f;
            if (sys_pin) {
                ba = std::min(ba, 1.5f);
                bs = std::min(bs, 1.9f);
            }
            seg_arch[s0] = ba;
            seg_sup[s0] = bs;
        } else {
            seg_arch[s0] = sys_pin ? 1.5f : 2.2f;
            seg_sup[s0] = sys_pin ? 1.9f : 2.5f;
        }
    } else {
        const uint32_t last = q_matched[n_m - 1u];
        const uint64_t last_bits = q_mask[last] & qbits;
        const float inv_mx = 1.0f / (float)mx;
        const float scale = (tier_a || max_hits >= 3u) ? 1.0f : 0.5f;
        for (uint32_t mi = 0; mi < n_m; ++mi) {
            const uint32_t sid = q_matched[mi];
            const float rel = (float)q_scores[sid] * inv_mx * scale;
            if (sid == last) {
                seg_arch[sid] = 1.5f * rel;
                seg_sup[sid] = 2.5f * rel;
            } else if (q_mask[sid] & last_bits) {
                seg_arch[sid] = 1.5f * rel;
                seg_sup[sid] = -0.4f;
            } else {
                seg_arch[sid] = 1.8f * rel;
                seg_sup[sid] = 2.0f * rel;
            }
        }
    }
    // per token slot, faded with the distance from <|im_end|>
    for (uint32_t k = 0; k < M; ++k) {
        const uint32_t sid = seg_inv[k];
        arch[k] = seg_arch[sid] * atten;
        sup[k] = seg_sup[sid] * atten;
        if (mode == 2) hop1[k] = seg_hop1[sid] * atten;
    }
    if (mode == 1 && n_m <= 2u) refine(n_m, n_q, tier_a, (bg < 0.0f ? bg * 0.5f : 0.0f) * atten, arch, sup);
    // continuation halo: one matched segment ending in a newline token whose value continues in the
    // next segment's first line (at most ten tokens, fewer than two content words)
    if (mode == 1 && n_m == 1u) {
        const uint32_t s0 = q_matched[0];
        if (s0 + 1u < N) {
            uint32_t k = 0;
            while (k < M && seg_inv[k] < s0) ++k;
            const uint32_t b0 = k;
            while (k < M && seg_inv[k] == s0) ++k;
            const uint32_t e0 = k, b1 = k;
            while (k < M && seg_inv[k] == s0 + 1u) ++k;
            const uint32_t e1 = k;
            if (e0 > b0 && e1 > b1 && mem_seg[b1] == mem_seg[b0] + 1u) {
                const uint32_t last = e0 - 1u;
                if (arch[last] > 0.0f && tok->has_byte(mem_tok[last], '\n')) {
                    const uint32_t lim = std::min(e1 - b1, 10u);
                    int32_t nl_at = -1;
                    for (uint32_t j = 0; j < lim && nl_at < 0; ++j)
                        if (tok->has_byte(mem_tok[b1 + j], '\n')) nl_at = (int32_t)j;
                    if (nl_at >= 0) {
                        nt_halo.start();
                        for (uint32_t j = 0; j <= (uint32_t)nl_at; ++j) nt_halo.add_token(*tok, mem_tok[b1 + j]);
                        nt_halo.close();
                        const uint32_t n_h = shingles(nt_halo, piv_sh.data(), 64u);
                        uint32_t words = 0;
                        for (uint32_t pi = 0; pi < n_h; ++pi) words += (piv_sh[pi] & 3u) == 0u;
                        if (words < 2u) {
                            const float a0 = arch[last], s0v = sup[last];
                            for (uint32_t j = 0; j <= (uint32_t)nl_at; ++j) {
                                arch[b1 + j] = a0;
                                sup[b1 + j] = s0v;
                            }
                        }
                    }
                }
            }
        }
    }
    return mode;
}

// ---------------------------------------------------------------- governor
namespace {
constexpr uint32_t kGovRules = 8, kGovRuleCap = 32, kGovHist = 64, kGovRaw = 96;

// UTF-8 decoding of one code point at s[i] (runtime/vault3.c:2329-2349): overlong forms, surrogates,
// values past U+10FFFF and truncated sequences decode as 0x110000 | lead byte, length 1.
uint32_t utf8_strict(const uint8_t *s, size_t n, size_t i, uint32_t *len) {
    const uint8_t c = s[i];
    *len = 1u;
    if (c < 0x80u) return c;
    uint32_t need, cp, min_cp;
    if ((c & 0xE0u) == 0xC0u) {
        need = 1u;
        cp = c & 0x1Fu;
        min_cp = 0x80u;
    } else if ((c & 0xF0u) == 0xE0u) {
        need = 2u;
        cp = c & 0x0Fu;
        min_cp = 0x800u;
    } else if ((c & 0xF8u) == 0xF0u) {
        need = 3u;
        cp = c & 0x07u;
        min_cp = 0x10000u;
    } else {
        return 0x110000u | c;
    }
    if (need > n - 1u - i) return 0x110000u | c;
    for (uint32_t k = 1u; k <= need; ++k) {
        if ((s[i + k] & 0xC0u) != 0x80u) return 0x110000u | c;
        cp = (cp << 6) | (uint32_t)(s[i + k] & 0x3Fu);
    }
    if (cp < min_cp || cp > 0x10FFFFu || (cp >= 0xD800u && cp <= 0xDFFFu)) return 0x110000u | c;
    *len = need + 1u;
    return cp;
}

// Canonical byte of a code point: 0 = dropped (controls, space, quotes, backslash, '+', '_', '-',
// zero-width and bidi formatting, smart quotes), ASCII letters lower-cased, fullwidth ASCII folded,
// Cyrillic / Greek look-alikes mapped to the Latin letter they imitate, anything else '?'.
uint8_t fold_cp(uint32_t cp) {
    if (cp >= 0xFF01u && cp <= 0xFF5Eu) cp -= 0xFEE0u;
    if (cp < 0x80u) {
        if (cp <= 0x20u || cp == 0x7Fu || cp == '\'' || cp == '"' || cp == '`' || cp == '+' || cp == '\\' ||
            cp == '_' || cp == '-')
            return 0;
        return (cp >= 'A' && cp <= 'Z') ? (uint8_t)(cp + 32u) : (uint8_t)cp;
    }
    if (cp == 0x00ADu || cp == 0x034Fu || cp == 0x061Cu || cp == 0x180Eu || (cp >= 0x200Bu && cp <= 0x200Fu) ||
        (cp >= 0x2018u && cp <= 0x201Fu) || (cp >= 0x202Au && cp <= 0x202Eu) || (cp >= 0x2060u && cp <= 0x206Fu) ||
        cp == 0xFEFFu)
        return 0;
    struct Glyph {
        uint32_t cp;
        uint8_t ch;
    };
    static const Glyph kGlyphs[] = {
        {0x0410, 'a'}, {0x0430, 'a'}, {0x0391, 'a'}, {0x03B1, 'a'}, {0x0412, 'b'}, {0x0432, 'b'}, {0x0392, 'b'},
        {0x03B2, 'b'}, {0x0421, 'c'}, {0x0441, 'c'}, {0x0415, 'e'}, {0x0435, 'e'}, {0x0395, 'e'}, {0x03B5, 'e'},
        {0x041D, 'h'}, {0x043D, 'h'}, {0x0397, 'h'}, {0x0406, 'i'}, {0x0456, 'i'}, {0x0399, 'i'}, {0x03B9, 'i'},
        {0x0408, 'j'}, {0x0458, 'j'}, {0x041A, 'k'}, {0x043A, 'k'}, {0x039A, 'k'}, {0x03BA, 'k'}, {0x041C, 'm'},
        {0x043C, 'm'}, {0x039C, 'm'}, {0x039D, 'n'}, {0x03BD, 'n'}, {0x041E, 'o'}, {0x043E, 'o'}, {0x039F, 'o'},
        {0x03BF, 'o'}, {0x0420, 'p'}, {0x0440, 'p'}, {0x03A1, 'p'}, {0x03C1, 'p'}, {0x0405, 's'}, {0x0455, 's'},
        {0x03A3, 's'}, {0x03C3, 's'}, {0x03C2, 's'}, {0x0422, 't'}, {0x0442, 't'}, {0x03A4, 't'}, {0x03C4, 't'},
        {0x0425, 'x'}, {0x0445, 'x'}, {0x03A7, 'x'}, {0x03C7, 'x'}, {0x0423, 'y'}, {0x0443, 'y'}, {0x03A5, 'y'},
        {0x03C5, 'y'}, {0x0396, 'z'}};
    for (const Glyph &g : kGlyphs)
        if (g.cp == cp) return g.ch;
    return '?';
}

// A rolling window of canonical bytes (the oldest drops out when full) plus a pending partial UTF-8
// sequence.
struct Canon {
    uint8_t h[kGovHist];
    uint32_t n = 0;
    uint8_t rem[4];
    uint32_t rn = 0;
    void push(uint8_t ch, uint32_t cap) {
        if (ch == 0u) return;
        if (n < cap) {
            h[n++] = ch;
        } else {
            std::memmove(h, h + 1, cap - 1u);
            h[cap - 1u] = ch;
        }
    }
    void feed(const uint8_t *b, size_t bl, uint32_t cap) {
        for (size_t i = 0; i < bl; ++i) {
            const uint8_t c = b[i];
            if (rn > 0u) {
                if ((c & 0xC0u) == 0x80u) {
                    rem[rn++] = c;
                    const uint8_t lead = rem[0];
                    const uint32_t need = (lead & 0xE0u) == 0xC0u ? 2u : ((lead & 0xF0u) == 0xE0u ? 3u : 4u);
                    if (rn == need) {
                        uint32_t cl;
                        const uint32_t cp = utf8_strict(rem, need, 0, &cl);
                        rn = 0;
                        if (cp < 0x110000u) push(fold_cp(cp), cap);
                    }
                    continue;
                }
                rn = 0;
            }
            if (c < 0x80u) push(fold_cp(c), cap);
            else if ((c & 0xE0u) == 0xC0u || (c & 0xF0u) == 0xE0u || (c & 0xF8u) == 0xF0u) {
                rem[0] = c;
                rn = 1;
            }
        }
    }
};

int b64_val(uint8_t c) {
    if (c >= 'A' && c <= 'Z') return c - 'A';
    if (c >= 'a' && c <= 'z') return c - 'a' + 26;
    if (c >= '0' && c <= '9') return c - '0' + 52;
    if (c == '+' || c == '-') return 62;
    if (c == '/' || c == '_') return 63;
    return -1;
}
int hex_val(uint8_t c) {
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    return -1;
}
bool hex_sep(uint8_t c) {
    return c == ' ' || c == '\\' || c == 'x' || c == 'X' || c == ':' || c == ',' || c == '-' || c == '_' || c == '\r' ||
           c == '\n';
}
bool contains_ci(const uint8_t *s, size_t n, const char *kw) {
    const size_t kl = std::strlen(kw);
    for (size_t i = 0; i + kl <= n; ++i) {
        size_t k = 0;
        for (; k < kl; ++k) {
            uint8_t c = s[i + k];
            if (c >= 'A' && c <= 'Z') c = (uint8_t)(c + 32u);
            if (c != (uint8_t)kw[k]) break;
        }
        if (k == kl) return true;
    }
    return false;
}
}  // namespace

struct vgx_governor {
    const vgx_tokens *tok;
    uint32_t eos, im_start, im_end;
    uint32_t n_rules = 0;
    uint8_t rules[kGovRules][kGovRuleCap];
    uint32_t rule_len[kGovRules];
    bool active = false;
    Canon hist;
    uint8_t raw[kGovRaw];
    uint32_t raw_n = 0;

    void reset_stream() {
        hist.n = 0;
        hist.rn = 0;
        raw_n = 0;
    }
    void clear() {
        n_rules = 0;
        active = false;
        reset_stream();
    }
    int add_rule(const uint8_t *pat, size_t len) {
        if (!pat || len == 0u) return VGX_E_SIZE;
        Canon c;
        c.feed(pat, len, kGovRuleCap);
        if (c.n < 4u) return VGX_E_SIZE;
        for (uint32_t r = 0; r < n_rules; ++r)
            if (rule_len[r] == c.n && std::memcmp(rules[r], c.h, c.n) == 0) {
                active = true;
                return VGX_OK;
            }
        if (n_rules >= kGovRules) return VGX_E_LIMIT;
        std::memcpy(rules[n_rules], c.h, c.n);
        rule_len[n_rules++] = c.n;
        active = true;
        return VGX_OK;
    }
    // A rule, forward or reversed, in the window at an alignment that ends after `prev` bytes.
    bool violates(const uint8_t *h, uint32_t n, uint32_t prev) const {
        for (uint32_t r = 0; r < n_rules; ++r) {
            const uint32_t rl = rule_len[r];
            if (n < rl) continue;
            for (uint32_t p = prev >= rl ? prev - rl + 1u : 0u; p + rl <= n; ++p) {
                uint32_t kf = 0, kr = 0;
                while (kf < rl && h[p + kf] == rules[r][kf]) ++kf;
                if (kf == rl) return true;
                while (kr < rl && h[p + kr] == rules[r][rl - 1u - kr]) ++kr;
                if (kr == rl) return true;
            }
        }
        return false;
    }
    bool decoded_violates(const uint8_t *dec, uint32_t dlen, uint32_t bound) const {
        Canon d;
        d.feed(dec, dlen, kGovHist);
        return violates(d.h, d.n, d.n > bound ? d.n - bound : 0u);
    }
    // The raw tail plus a candidate token read as Base64 (four alignments) or hex (two) that decodes
    // to a rule (runtime/vault3.c:3032-3131).
    bool encoded_violates(const uint8_t *tb, uint32_t tbl) const {
        const uint32_t take = std::min(tbl, 64u);
        bool b64 = false, hex = false;
        for (uint32_t i = 0; i < take; ++i) {
            b64 = b64 || b64_val(tb[i]) >= 0;
            hex = hex || hex_val(tb[i]) >= 0;
        }
        if (!b64 && !hex) return false;
        uint8_t comb[kGovRaw + 64];
        uint8_t vals[192];
        uint8_t dec[96];
        uint32_t cn = 0;
        for (uint32_t i = 0; i < raw_n; ++i) comb[cn++] = raw[i];
        for (uint32_t i = 0; i < take; ++i) comb[cn++] = tb[i];
        const uint32_t bound = take + 3u;
        if (b64) {
            uint32_t end = cn;
            while (end > 0u && (comb[end - 1u] == '\r' || comb[end - 1u] == '\n')) --end;
            for (uint32_t eq = 0; end > 0u && comb[end - 1u] == '=' && eq < 2u; ++eq) --end;
            uint32_t start = end, cnt = 0;
            while (start > 0u && cnt < 128u) {
                const uint8_t ch = comb[start - 1u];
                if (ch == '\r' || ch == '\n') {
                    --start;
                } else if (b64_val(ch) >= 0) {
                    --start;
                    ++cnt;
                } else {
                    break;
                }
            }
            if (cnt >= 8u) {
                uint32_t nv = 0;
                for (uint32_t i = start; i < end && nv < 128u; ++i) {
                    const int v = b64_val(comb[i]);
                    if (v >= 0) vals[nv++] = (uint8_t)v;
                }
                for (uint32_t off = 0; off < 4u && off + 6u <= nv; ++off) {
                    uint32_t left = nv - off, p = off, dl = 0;
                    while (left >= 4u && dl + 3u <= sizeof(dec)) {
                        const uint32_t v = ((uint32_t)vals[p] << 18) | ((uint32_t)vals[p + 1] << 12) |
                                           ((uint32_t)vals[p + 2] << 6) | (uint32_t)vals[p + 3];
                        dec[dl++] = (uint8_t)(v >> 16);
                        dec[dl++] = (uint8_t)(v >> 8);
                        dec[dl++] = (uint8_t)v;
                        p += 4u;
                        left -= 4u;
                    }
                    if (left == 3u && dl + 2u <= sizeof(dec)) {
                        const uint32_t v =
                            ((uint32_t)vals[p] << 18) | ((uint32_t)vals[p + 1] << 12) | ((uint32_t)vals[p + 2] << 6);
                        dec[dl++] = (uint8_t)(v >> 16);
                        dec[dl++] = (uint8_t)(v >> 8);
                    } else if (left == 2u && dl + 1u <= sizeof(dec)) {
                        const uint32_t v = ((uint32_t)vals[p] << 18) | ((uint32_t)vals[p + 1] << 12);
                        dec[dl++] = (uint8_t)(v >> 16);
                    }
                    if (decoded_violates(dec, dl, bound)) return true;
                }
            }
        }
        if (hex) {
            uint32_t start = cn, cnt = 0;
            while (start > 0u && cnt < 192u) {
                const uint8_t ch = comb[start - 1u];
                if (hex_val(ch) >= 0) {
                    --start;
                    ++cnt;
                } else if (hex_sep(ch)) {
                    --start;
                } else {
                    break;
                }
            }
            if (cnt >= 8u) {
                uint32_t nn = 0;
                for (uint32_t i = start; i < cn && nn < 192u;) {
                    if (comb[i] == '0' && i + 2u < cn && (comb[i + 1] == 'x' || comb[i + 1] == 'X') &&
                        hex_val(comb[i + 2]) >= 0) {
                        i += 2u;
                        continue;
                    }
                    const int v = hex_val(comb[i]);
                    if (v >= 0) vals[nn++] = (uint8_t)v;
                    ++i;
                }
                if (nn >= 8u)
                    for (uint32_t off = 0; off < 2u && off + 8u <= nn; ++off) {
                        uint32_t dl = 0;
                        for (uint32_t p = off; p + 1u < nn && dl < sizeof(dec); p += 2u)
                            dec[dl++] = (uint8_t)((vals[p] << 4) | vals[p + 1]);
                        if (decoded_violates(dec, dl, bound)) return true;
                    }
            }
        }
        return false;
    }
    // Would emitting token `id` next complete a rule (in the canonical window or an encoded tail)?
    bool blocks(uint32_t id) const {
        const uint8_t *tb;
        uint32_t tbl;
        if (!tok->get(id, tb, tbl) || tbl == 0u) return false;
        Canon t = hist;
        // at most 31 bytes of history before the candidate, so the window never drops `prev`
        if (t.n > 31u) {
            std::memmove(t.h, t.h + (t.n - 31u), 31u);
            t.n = 31u;
        }
        const uint32_t prev = t.n;
        t.feed(tb, tbl, kGovHist);
        return violates(t.h, t.n, prev) || encoded_violates(tb, tbl);
    }
    void commit(uint32_t id) {
        if (!active) return;
        if (id == eos || id == im_end || id == im_start) {
            reset_stream();
            return;
        }
        const uint8_t *tb;
        uint32_t tbl;
        if (!tok->get(id, tb, tbl) || tbl == 0u) return;
        hist.feed(tb, tbl, kGovHist);
        for (uint32_t i = 0; i < tbl; ++i) {
            if (raw_n < kGovRaw) {
                raw[raw_n++] = tb[i];
            } else {
                std::memmove(raw, raw + 1, kGovRaw - 1u);
                raw[kGovRaw - 1u] = tb[i];
            }
        }
    }
};

// ---------------------------------------------------------------- C ABI
extern "C" {

vgx_tokens *vgx_tokens_create(const uint8_t *pool, const uint64_t *offsets, uint32_t n_tokens) {
    if (!offsets || (n_tokens > 0 && !pool && offsets[n_tokens] > 0)) return nullptr;
    for (uint32_t i = 0; i < n_tokens; ++i)
        if (offsets[i + 1] < offsets[i]) return nullptr;
    auto *t = new (std::nothrow) vgx_tokens();
    if (!t) return nullptr;
    t->n = n_tokens;
    t->off.assign(offsets, offsets + n_tokens + 1);
    t->pool.assign(pool ? pool : (const uint8_t *)"", pool ? pool + offsets[n_tokens] : (const uint8_t *)"");
    return t;
}

void vgx_tokens_destroy(vgx_tokens *t) { delete t; }

vgx_resonance *vgx_res_create(const vgx_tokens *t, uint32_t window, uint32_t seg_cap, uint32_t n_sink,
                              uint32_t im_start_id, uint32_t im_end_id) {
    if (!t || window == 0u || seg_cap == 0u) return nullptr;
    auto *r = new (std::nothrow) vgx_resonance();
    if (!r) return nullptr;
    r->tok = t;
    r->window = window;
    r->seg_cap = seg_cap;
    r->n_sink = n_sink;
    r->im_start = im_start_id;
    r->im_end = im_end_id;
    // index capacities of the reference state for this many bank slots (runtime/vault3.c:718-721)
    const uint32_t want = 16u * seg_cap + 4096u;
    r->cap = 16384u;
    while (r->cap < want && r->cap < (1u << 22)) r->cap <<= 1;
    r->post_cap = 24u * seg_cap + 1024u;
    try {
        r->keys.assign(r->cap, ~0ull);
        r->df.assign(r->cap, 0);
        r->head.assign(r->cap, kNone);
        r->last_sid.assign(r->cap, 0);
        r->post_sid.assign(r->post_cap, 0);
        r->post_w.assign(r->post_cap, 0);
        r->post_next.assign(r->post_cap, 0);
        r->mem_tok.assign(seg_cap, 0);
        r->mem_seg.assign(seg_cap, 0);
        r->seg_inv.assign(seg_cap, 0);
        r->q_scores.assign(seg_cap + 1u, 0);
        r->q_hits.assign(seg_cap + 1u, 0);
        r->q_matched.assign(seg_cap + 1u, 0);
        r->q_mask.assign(seg_cap + 1u, 0);
        r->seg_arch.assign(seg_cap + 1u, 0.0f);
        r->seg_sup.assign(seg_cap + 1u, 0.0f);
        r->seg_hop1.assign(seg_cap + 1u, 0.0f);
        r->q_sh.assign(1024, 0);
        r->piv_sh.assign(1024, 0);
        r->cl_sh.assign(512, 0);
        r->seg_sh.assign(2048, 0);
        r->raw_lc.assign(4096, 0);
        r->raw_cl.assign(2048, 0);
    } catch (...) {
        delete r;
        return nullptr;
    }
    return r;
}

void vgx_res_destroy(vgx_resonance *r) { delete r; }

int vgx_res_rebuild(vgx_resonance *r, const uint32_t *mem_tok, const uint32_t *mem_seg, uint32_t mem_cnt) {
    if (!r || (mem_cnt > 0u && (!mem_tok || !mem_seg))) return VGX_E_ARG;
    if (mem_cnt > r->seg_cap) return VGX_E_LIMIT;
    std::copy(mem_tok, mem_tok + mem_cnt, r->mem_tok.begin());
    std::copy(mem_seg, mem_seg + mem_cnt, r->mem_seg.begin());
    r->mem_cnt = mem_cnt;
    r->rebuild();
    return (int)r->n_segs;
}

int vgx_res_update(vgx_resonance *r, const uint32_t *tok_prev, const uint32_t *tok_cur, uint32_t c, uint64_t pos,
                   uint32_t n_pin, float *arch, float *sup, float *hop1) {
    if (!r || !tok_prev || !tok_cur || !arch || !sup || !hop1) return VGX_E_ARG;
    if (c >= r->window) return VGX_E_SIZE;
    return r->update(tok_prev, tok_cur, c, pos, n_pin, arch, sup, hop1);
}

int vgx_spoof_check(const vgx_tokens *t, const uint32_t *tok_prev, const uint32_t *tok_cur, uint32_t window,
                    uint32_t c, uint64_t pos, uint32_t n_pin, uint32_t n_sink) {
    if (!t || !tok_prev || !tok_cur || c >= window) return VGX_E_ARG;
    if (n_pin <= n_sink || pos < (uint64_t)n_pin) return 0;
    // the lower-cased bytes of the last min(24, pos - n_pin + 1) tokens of the window
    const uint64_t post_pin = pos - (uint64_t)n_pin + 1u;
    uint32_t lb = post_pin < 24u ? (uint32_t)post_pin : 24u;
    const uint32_t cur_n = c + 1u, tot = pos >= window ? window + cur_n : cur_n;
    lb = std::min(lb, tot);
    const uint32_t need_prev = cur_n < lb ? lb - cur_n : 0u;
    const uint32_t cur_from = cur_n > lb ? cur_n - lb : 0u;
    std::vector<uint8_t> buf;
    buf.reserve(4096);
    auto add = [&](uint32_t id) {
        const uint8_t *b;
        uint32_t bl;
        if (!t->get(id, b, bl)) return;
        for (uint32_t i = 0; i < bl && buf.size() < 4096u; ++i)
            buf.push_back((b[i] >= 'A' && b[i] <= 'Z') ? (uint8_t)(b[i] + 32u) : b[i]);
    };
    for (uint32_t k = window - need_prev; k < window; ++k) add(tok_prev[k]);
    for (uint32_t k = cur_from; k <= c; ++k) add(tok_cur[k]);
    return find_sub(buf.data(), (uint32_t)buf.size(), "opi_signed_directive") >= 0 ||
           find_sub(buf.data(), (uint32_t)buf.size(), "urgent opi delegation") >= 0;
}

vgx_governor *vgx_gov_create(const vgx_tokens *t, uint32_t eos_id, uint32_t im_start_id, uint32_t im_end_id) {
    if (!t) return nullptr;
    auto *g = new (std::nothrow) vgx_governor();
    if (!g) return nullptr;
    g->tok = t;
    g->eos = eos_id;
    g->im_start = im_start_id;
    g->im_end = im_end_id;
    return g;
}

void vgx_gov_destroy(vgx_governor *g) { delete g; }

void vgx_gov_reset_stream(vgx_governor *g) {
    if (g) g->reset_stream();
}

int vgx_gov_add_rule(vgx_governor *g, const uint8_t *pat, size_t len) { return g ? g->add_rule(pat, len) : VGX_E_ARG; }

int vgx_gov_arm_system(vgx_governor *g, const uint8_t *text, size_t len) {
    if (!g) return VGX_E_ARG;
    g->clear();
    if (!text || len == 0u) return 0;
    const bool prohibits = contains_ci(text, len, "never") || contains_ci(text, len, "forbid") ||
                           contains_ci(text, len, "prohibit") || contains_ci(text, len, "must not") ||
                           contains_ci(text, len, "do not output") || contains_ci(text, len, "do not emit");
    if (!prohibits) return 0;
    if (contains_ci(text, len, "syscall_exec")) {
        g->add_rule((const uint8_t *)"syscall_exec", 12);
        g->add_rule((const uint8_t *)"syscallexec", 11);
    }
    // quoted literals ('...', "...", `...`) with a '_' or '(' inside: the literal, without a trailing
    // '(' and without underscores
    for (size_t i = 0; i < len; ++i) {
        const uint8_t q = text[i];
        if (q != '\'' && q != '"' && q != '`') continue;
        size_t j = i + 1;
        bool sig = false;
        while (j < len && text[j] != q && (j - i - 1) < kGovRuleCap) {
            sig = sig || text[j] == '_' || text[j] == '(';
            ++j;
        }
        const size_t sl = j - (i + 1);
        if (!(j < len && text[j] == q && sig && sl >= 5u && sl < kGovRuleCap)) continue;
        const uint8_t *lit = text + i + 1;
        g->add_rule(lit, sl);
        const bool paren = lit[sl - 1] == '(';
        if (paren && sl >= 6u) g->add_rule(lit, sl - 1);
        uint8_t bare[kGovRuleCap];
        size_t bn = 0;
        for (size_t k = 0; k < (paren ? sl - 1 : sl) && bn < kGovRuleCap; ++k)
            if (lit[k] != '_') bare[bn++] = lit[k];
        if (bn >= 5u) g->add_rule(bare, bn);
        i = j;
    }
    return (int)g->n_rules;
}

int vgx_gov_active(const vgx_governor *g) { return g && g->active && g->n_rules > 0u; }

int vgx_gov_screen(const vgx_governor *g, const int64_t *cand, const float *cand_val, uint32_t n_cand,
                   uint32_t top_k_guard, uint32_t vocab, int64_t *masked, uint32_t max_masked) {
    if (!g || (n_cand > 0u && (!cand || !cand_val)) || !masked) return VGX_E_ARG;
    if (!vgx_gov_active(g)) return 0;
    uint32_t k = (top_k_guard == 0u || top_k_guard > 64u) ? 64u : top_k_guard;
    k = std::min(k, vocab);
    // Up to four passes over the best k still unmasked candidates (value desc, index asc, values at or
    // below -3e38 excluded, as the logits would be re-scanned after each pass).
    std::vector<uint8_t> gone(n_cand, 0);
    uint32_t n_masked = 0;
    for (int pass = 0; pass < 4; ++pass) {
        bool any = false;
        uint32_t seen = 0;
        for (uint32_t i = 0; i < n_cand && seen < k; ++i) {
            if (gone[i] || !(cand_val[i] > -3.0e38f)) continue;
            ++seen;
            if (cand[i] < 0 || cand[i] >= (int64_t)vocab) continue;
            if (g->blocks((uint32_t)cand[i])) {
                gone[i] = 1;
                any = true;
                if (n_masked >= max_masked) return VGX_E_LIMIT;
                masked[n_masked++] = cand[i];
            }
        }
        if (!any) break;
    }
    return (int)n_masked;
}

int vgx_gov_commit(vgx_governor *g, uint32_t id) {
    if (!g) return VGX_E_ARG;
    g->commit(id);
    return VGX_OK;
}

}  // extern "C"
