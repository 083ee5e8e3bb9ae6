// Split-K GQA decode attention over up to four key spans (sink | segment memory | prev | cur).
//
// Reference semantics: src/vault_v3_model.py:1098-1136 (concat spans, _expand_kv, optional fp32
// bias on the segment span, softmax, P V) and runtime/vault3.c:1958-2032 (attn_run).
//
// Mapping.  One workgroup = kWaves waves = one (batch b, kv group g, key split).  Every wave holds
// the GRP query heads of group g, so each K/V row is fetched once for all GRP heads (the reference
// re-reads K/V per head).  The split's keys are dealt to the waves in 16-key tiles; inside a wave
// the 4 DPP rows (16 lanes each) take 4 keys of the tile each, one key row spread over the 16 lanes
// of a DPP row (D/16 contiguous elements per lane: one 128-bit load for bf16 D=128, two for fp32),
// so one load instruction fetches four whole key rows.  q.k partials are reduced over the 16 lanes
// with DPP; every DPP row keeps its own online-softmax state (m, l, acc).  The states are merged
// across DPP rows with lane shuffles and across the waves of the workgroup through LDS; with more
// than one split, each split writes (m, l, acc) partials to the workspace; up to 8 splits are
// combined by the workgroup that finishes a (b, g) pair last (ticket_merge: agent-scope atomic
// stores and loads of the partials instead of a release fence, whose write-back of the whole L2
// measured 2x slower), more by attn_merge_kernel, a second launch spread over B * H workgroups.
#include "common.h"

#include <mutex>

using namespace vgx;

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;    // waves per workgroup
constexpr int kTargetWaves = 2048;
constexpr int kMaxSplits = 64;
constexpr float kNegBig = -1.0e30f;

struct SpanArgs {
    const void *k[4];
    const void *v[4];
    int64_t len[4];
    int64_t bstride[4];
    int64_t gstride[4];
    const int32_t *dyn_len[4];
    int n;
};

// Merging the splits of a (b, g) pair without a second launch.  Every workgroup writes its partials
// with agent-scope atomic stores (written through to the device-coherent level, no L2 write-back of
// the whole cache as a release fence would need), waits for them to complete, then takes a ticket
// from the pair's counter; the workgroup that draws the last ticket reads every split's partials with
// agent-scope atomic loads, combines them in split order (deterministic) and resets the counter to
// zero for the next launch (no memset, so a captured graph replays it).
constexpr int kTicketMaxSplits = 32;                // splits merged by the last workgroup of a pair
constexpr int kMergeFast = 8;                       // splits the last workgroup merges in one round trip

template <int GRP, int D>
__device__ __forceinline__ void store_partial(float *pp, int d, float A, float M, float L) {
    __hip_atomic_store(pp + d, A, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (d == 0) {
        __hip_atomic_store(pp + D, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(pp + D + 1, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int GRP, int D>
__device__ __forceinline__ void ticket_merge(const float *__restrict__ part_pair, int *__restrict__ cnt, int n_splits,
                                             float *__restrict__ outp, float *sc, int *flag) {
    constexpr int SLOT = D + 2;
    const int tid = threadIdx.x, nt = blockDim.x;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this thread's partial stores have completed
    __syncthreads();
    if (tid == 0) {
        const int old = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag = old == n_splits - 1;
    }
    __syncthreads();
    if (!*flag) return;
    if (n_splits <= kMergeFast) {
        // one round trip: every thread requests, for PB outputs at a time, each split's value and the
        // split's (m, l) of the output's head before using any of them
        constexpr int PB = 3;
        for (int t0 = 0; t0 < GRP * D; t0 += nt * PB) {
            float v[PB][kMergeFast], mm[PB][kMergeFast], ll[PB][kMergeFast];
#pragma unroll
            for (int j = 0; j < PB; ++j) {
                const int t = min(t0 + tid + nt * j, GRP * D - 1);
                const int hh = t / D, d = t - hh * D;
#pragma unroll
                for (int u = 0; u < kMergeFast; ++u) {
                    const float *pp = part_pair + ((int64_t)min(u, n_splits - 1) * GRP + hh) * SLOT;
                    v[j][u] = __hip_atomic_load(pp + d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    mm[j][u] = __hip_atomic_load(pp + D, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    ll[j][u] = __hip_atomic_load(pp + D + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
#pragma unroll
            for (int j = 0; j < PB; ++j) {
                const int t = t0 + tid + nt * j;
                if (t >= GRP * D) continue;
                const int hh = t / D, d = t - hh * D;
                float M = kNegBig;
#pragma unroll
                for (int u = 0; u < kMergeFast; ++u)
                    if (u < n_splits) M = fmaxf(M, mm[j][u]);
                float L = 0.0f, A = 0.0f;
#pragma unroll
                for (int u = 0; u < kMergeFast; ++u) {
                    if (u < n_splits) {
                        const float w = __expf(mm[j][u] - M);
                        L = fmaf(w, ll[j][u], L);
                        A = fmaf(w, v[j][u], A);
                    }
                }
                outp[(int64_t)hh * D + d] = A * (1.0f / L);
            }
        }
        if (tid == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    float *wm = sc, *wl = sc + GRP * kMaxSplits, *inv = sc + 2 * GRP * kMaxSplits;
    for (int i = tid; i < GRP * n_splits; i += nt) {
        const int hh = i / n_splits, sp = i - hh * n_splits;
        const float *pp = part_pair + ((int64_t)sp * GRP + hh) * SLOT;
        wm[hh * kMaxSplits + sp] = __hip_atomic_load(pp + D, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        wl[hh * kMaxSplits + sp] = __hip_atomic_load(pp + D + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (tid < GRP) {
        float M = kNegBig;
        for (int sp = 0; sp < n_splits; ++sp) M = fmaxf(M, wm[tid * kMaxSplits + sp]);
        float L = 0.0f;
        for (int sp = 0; sp < n_splits; ++sp) {
            const float w = __expf(wm[tid * kMaxSplits + sp] - M);
            wm[tid * kMaxSplits + sp] = w;
            L = fmaf(w, wl[tid * kMaxSplits + sp], L);
        }
        inv[tid] = 1.0f / L;
    }
    __syncthreads();
    // every split of an output requested at once (n_splits <= kTicketMaxSplits)
    for (int t = tid; t < GRP * D; t += nt) {
        const int hh = t / D, d = t - hh * D;
        float v[kTicketMaxSplits];
#pragma unroll
        for (int u = 0; u < kTicketMaxSplits; ++u)
            v[u] = __hip_atomic_load(part_pair + ((int64_t)min(u, n_splits - 1) * GRP + hh) * SLOT + d,
                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        float A = 0.0f;
#pragma unroll
        for (int u = 0; u < kTicketMaxSplits; ++u)
            if (u < n_splits) A = fmaf(wm[hh * kMaxSplits + u], v[u], A);
        outp[(int64_t)hh * D + d] = A * inv[hh];
    }
    if (tid == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One lane's DPL elements of a key row as raw words (F32: DPL words, BF16: DPL / 2 words), loaded
// with 128-bit (or 64-bit) loads and converted to fp32 at use.
template <int KV, int DPL>
struct RowRaw {
    static constexpr int W = KV == VGX_F32 ? DPL : DPL / 2;
    uint32_t w[W];
};

// fp32 rows of D = 128: a lane's 8 elements are two quads 64 apart (dims 4 l .. + 3 and 64 + 4 l ..),
// so each load instruction of a DPP row reads one contiguous half row (256 bytes) instead of 16-byte
// pieces with 16-byte gaps; the query, the accumulators and the LDS combine use the same mapping.
template <int KV, int DPL>
constexpr bool kSpreadQuads = KV == VGX_F32 && DPL == 8;

// Element offset in its row of quad d4 of lane l16.
template <int KV, int DPL>
__device__ __forceinline__ int lane_quad(int l16, int d4) {
    return kSpreadQuads<KV, DPL> ? d4 * 64 + l16 * 4 : l16 * DPL + 4 * d4;
}

template <int KV, int DPL>
__device__ __forceinline__ void load_raw(const void *base, int64_t elem_off, RowRaw<KV, DPL> &r) {
    constexpr int W = RowRaw<KV, DPL>::W;
    const uint32_t *p = reinterpret_cast<const uint32_t *>(static_cast<const char *>(base) +
                                                           elem_off * (KV == VGX_F32 ? 4 : 2));
    if constexpr (kSpreadQuads<KV, DPL>) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint4 t = *reinterpret_cast<const uint4 *>(p + 64 * i);
            r.w[4 * i] = t.x; r.w[4 * i + 1] = t.y; r.w[4 * i + 2] = t.z; r.w[4 * i + 3] = t.w;
        }
    } else if constexpr (W % 4 == 0) {
#pragma unroll
        for (int i = 0; i < W / 4; ++i) {
            const uint4 t = reinterpret_cast<const uint4 *>(p)[i];
            r.w[4 * i] = t.x; r.w[4 * i + 1] = t.y; r.w[4 * i + 2] = t.z; r.w[4 * i + 3] = t.w;
        }
    } else if constexpr (W == 2) {
        const uint2 t = *reinterpret_cast<const uint2 *>(p);
        r.w[0] = t.x; r.w[1] = t.y;
    } else {
#pragma unroll
        for (int i = 0; i < W; ++i) r.w[i] = p[i];
    }
}

template <int KV, int DPL>
__device__ __forceinline__ float raw_at(const RowRaw<KV, DPL> &r, int d) {
    if constexpr (KV == VGX_F32) return __uint_as_float(r.w[d]);
    else return (d & 1) ? __uint_as_float(r.w[d >> 1] & 0xFFFF0000u) : __uint_as_float(r.w[d >> 1] << 16);
}

// The KB keys of one DPP row of a 4 KB-key tile.
template <int KV, int DPL, int KB>
struct KeyTile {
    RowRaw<KV, DPL> k[KB], v[KB];
};

template <typename T>
__device__ __forceinline__ T pick4(int s, T a0, T a1, T a2, T a3) {
    return s == 0 ? a0 : s == 1 ? a1 : s == 2 ? a2 : a3;
}

// Workspace layout: partials per (b, g, split, head): D accumulators, then m, l.
//
// Split z covers global keys [z kps, (z + 1) kps) of the concatenated spans (by capacity).  Inside
// each span the split's keys are dealt to the waves in TK = 4 KB-key tiles (wave w: tiles lo + TK w +
// NW TK i).  Tile addresses depend only on the span capacities (host values), so the first tile's K/V
// loads are issued before the query and the device-side lengths arrive; keys at or beyond a span's
// effective length (device length, causal limit) are masked, and no row beyond a span's capacity is
// read.  With PIPE the next tile's loads are issued before the current tile is reduced.
//
// The online-softmax states of the 4 NW DPP rows are combined in two stages: RS steps of VALU lane
// swaps inside each wave (RS = 2: one state per wave), then the remaining P = NW (4 >> RS) states
// through LDS: per head, the running maxima give P weights e^{m_p - M} (computed once), and each
// output is a P-term weighted sum.  RS = 0 costs no cross-lane traffic at all (measured faster at
// batch 1, where a wave's serial instruction count is the latency).
template <int KV, int GRP, int DPL, int NW, int KB, int RS>
__global__ __launch_bounds__(64 * NW) void attn_decode_kernel(
    const float *__restrict__ q, int64_t ldq, SpanArgs sp, const float *__restrict__ bias, int64_t bias_hstride,
    int bias_span, float *__restrict__ out, float *__restrict__ part, int *__restrict__ cnt, int H, int G,
    float scale, int64_t n_tot, int64_t kps, int n_splits, int64_t causal_base) {
    constexpr int D = DPL * 16;
    constexpr int SLOT = D + 2;
    constexpr int TK = 4 * KB;                      // keys per wave tile
    constexpr int P = NW * (4 >> RS);               // states combined through LDS
    constexpr bool PIPE = KV == VGX_BF16;
    static_assert(RS >= 0 && RS <= 2, "0, 1 or 2 lane-swap steps");
    __shared__ float red[P][GRP][SLOT];
    __shared__ float wgt[GRP][P];
    __shared__ float mrg[2][GRP];

    const int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x & 63, l16 = lane & 15, row = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

    // per-span key ranges of this split, local to the span: [lo, hi) by capacity (uniform)
    const int64_t k0 = (int64_t)split * kps;
    const int64_t k1 = min(n_tot, k0 + kps);
    int lo[4], hi[4], eff[4];
    {
        int64_t base = 0;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int64_t len = s < sp.n ? sp.len[s] : 0;
            lo[s] = (int)(max(k0, base) - base);
            hi[s] = (int)(max(min(k1, base + len) - base, (int64_t)lo[s]));
            base += len;
        }
    }
    // the wave's first tile: span s, local start t (s = 4: none)
    auto first_in = [&](int s0) -> int2 {
#pragma unroll
        for (int s = 0; s < 4; ++s)
            if (s >= s0 && lo[s] + wave * TK < hi[s]) return make_int2(s, lo[s] + wave * TK);
        return make_int2(4, 0);
    };
    auto next = [&](int2 c) -> int2 {
        if (c.y + NW * TK < pick4(c.x, hi[0], hi[1], hi[2], hi[3])) return make_int2(c.x, c.y + NW * TK);
        return first_in(c.x + 1);
    };
    auto fetch = [&](KeyTile<KV, DPL, KB> &t, int2 c) {
        const int s = c.x;
        const void *kb = pick4(s, sp.k[0], sp.k[1], sp.k[2], sp.k[3]);
        const void *vb = pick4(s, sp.v[0], sp.v[1], sp.v[2], sp.v[3]);
        const int64_t o = (int64_t)b * pick4(s, sp.bstride[0], sp.bstride[1], sp.bstride[2], sp.bstride[3]) +
                          (int64_t)g * pick4(s, sp.gstride[0], sp.gstride[1], sp.gstride[2], sp.gstride[3]) +
                          (int64_t)(c.y + row * KB) * D + lane_quad<KV, DPL>(l16, 0);
        // rows past the split's end in this span re-read its last row (in bounds; masked at use)
        const int last = pick4(s, hi[0], hi[1], hi[2], hi[3]) - 1 - c.y - row * KB;
#pragma unroll
        for (int j = 0; j < KB; ++j) {
            const int64_t oj = o + (int64_t)min(j, last) * D;
            load_raw<KV, DPL>(kb, oj, t.k[j]);
            load_raw<KV, DPL>(vb, oj, t.v[j]);
        }
    };

    // q of the GRP heads, then the first tile, then the device-side lengths
    float qr[GRP][DPL];
#pragma unroll
    for (int hh = 0; hh < GRP; ++hh) {
        const float *qp = q + (int64_t)b * ldq + ((int64_t)g * GRP + hh) * D;
#pragma unroll
        for (int d4 = 0; d4 < DPL / 4; ++d4) {
            const float4 t = *reinterpret_cast<const float4 *>(qp + lane_quad<KV, DPL>(l16, d4));
            qr[hh][4 * d4] = t.x; qr[hh][4 * d4 + 1] = t.y; qr[hh][4 * d4 + 2] = t.z; qr[hh][4 * d4 + 3] = t.w;
        }
    }
    KeyTile<KV, DPL, KB> tA, tB;
    int2 cur = first_in(0);
    if (cur.x < 4) fetch(tA, cur);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        int64_t e = s < sp.n ? sp.len[s] : 0;
        if (s < sp.n && sp.dyn_len[s] != nullptr) e = min(e, (int64_t)*sp.dyn_len[s]);
        if (causal_base >= 0 && s == sp.n - 1) e = min(e, causal_base + (int64_t)b + 1);
        eff[s] = (int)min((int64_t)hi[s], max(e, (int64_t)0));
    }
#pragma unroll
    for (int hh = 0; hh < GRP; ++hh)
#pragma unroll
        for (int d = 0; d < DPL; ++d) qr[hh][d] *= scale;

    float m[GRP], l[GRP], acc[GRP][DPL];
#pragma unroll
    for (int hh = 0; hh < GRP; ++hh) {
        m[hh] = kNegBig;
        l[hh] = 0.0f;
#pragma unroll
        for (int d = 0; d < DPL; ++d) acc[hh][d] = 0.0f;
    }

    auto compute = [&](const KeyTile<KV, DPL, KB> &t, int2 c) {
        const int s = c.x;
        const int e = pick4(s, eff[0], eff[1], eff[2], eff[3]);
        const float *bb = (bias != nullptr && s == bias_span) ? bias + (int64_t)g * GRP * bias_hstride : nullptr;
        float sc[GRP][KB];
#pragma unroll
        for (int j = 0; j < KB; ++j)
#pragma unroll
            for (int hh = 0; hh < GRP; ++hh) {
                float p = 0.0f;
#pragma unroll
                for (int d = 0; d < DPL; ++d) p = fmaf(qr[hh][d], raw_at<KV, DPL>(t.k[j], d), p);
                sc[hh][j] = row16_sum(p);
            }
#pragma unroll
        for (int j = 0; j < KB; ++j) {
            const int key = c.y + row * KB + j;
            const bool valid = key < e;
#pragma unroll
            for (int hh = 0; hh < GRP; ++hh) {
                float v = sc[hh][j];
                if (bb != nullptr && valid) v += bb[hh * bias_hstride + key];
                sc[hh][j] = valid ? v : -INFINITY;
            }
        }
#pragma unroll
        for (int hh = 0; hh < GRP; ++hh) {
            float mb = sc[hh][0];
#pragma unroll
            for (int j = 1; j < KB; ++j) mb = fmaxf(mb, sc[hh][j]);
            const float mn = fmaxf(m[hh], mb);
            const float corr = __expf(m[hh] - mn);
            m[hh] = mn;
            float ls = l[hh] * corr;
#pragma unroll
            for (int j = 0; j < KB; ++j) {
                const float p = __expf(sc[hh][j] - mn);
                sc[hh][j] = p;
                ls += p;
            }
            l[hh] = ls;
#pragma unroll
            for (int d = 0; d < DPL; ++d) {
                float a = acc[hh][d] * corr;
#pragma unroll
                for (int j = 0; j < KB; ++j) a = fmaf(sc[hh][j], raw_at<KV, DPL>(t.v[j], d), a);
                acc[hh][d] = a;
            }
        }
    };
    // Masked rows of a tile may hold anything (e.g. unwritten ring slots): their values are replaced
    // by zeros before use so that p = 0 cannot meet a non-finite value.
    auto clean = [&](KeyTile<KV, DPL, KB> &t, int2 c) {
        const int e = pick4(c.x, eff[0], eff[1], eff[2], eff[3]);
        if (c.y + TK <= e) return;                 // uniform: the whole tile is valid
#pragma unroll
        for (int j = 0; j < KB; ++j) {
            const bool valid = c.y + row * KB + j < e;
#pragma unroll
            for (int w = 0; w < RowRaw<KV, DPL>::W; ++w) {
                t.k[j].w[w] = valid ? t.k[j].w[w] : 0u;
                t.v[j].w[w] = valid ? t.v[j].w[w] : 0u;
            }
        }
    };

    if constexpr (PIPE) {
        while (cur.x < 4) {
            int2 nx = next(cur);
            if (nx.x < 4) fetch(tB, nx);
            clean(tA, cur);
            compute(tA, cur);
            cur = nx;
            if (cur.x >= 4) break;
            nx = next(cur);
            if (nx.x < 4) fetch(tA, nx);
            clean(tB, cur);
            compute(tB, cur);
            cur = nx;
        }
    } else {
        while (cur.x < 4) {
            clean(tA, cur);
            compute(tA, cur);
            cur = next(cur);
            if (cur.x < 4) fetch(tA, cur);
        }
    }

    // RS steps of the in-wave merge: rows r and r ^ 1, then the two halves, with the VALU lane swaps
    // (each gives a lane its own and its partner's value, the lower row's first in every lane of a row
    // pair, so both rows of a pair compute the same merge).
#pragma unroll
    for (int step = 0; step < RS; ++step) {
        auto pair = [&](float x) {
            const auto r = step == 0
                               ? __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false)
                               : __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
            return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
        };
#pragma unroll
        for (int hh = 0; hh < GRP; ++hh) {
            const float2 mp = pair(m[hh]), lp = pair(l[hh]);
            const float mn = fmaxf(mp.x, mp.y);
            const float c1 = __expf(mp.x - mn), c2 = __expf(mp.y - mn);
            l[hh] = fmaf(lp.x, c1, lp.y * c2);
#pragma unroll
            for (int d = 0; d < DPL; ++d) {
                const float2 ap = pair(acc[hh][d]);
                acc[hh][d] = fmaf(ap.x, c1, ap.y * c2);
            }
            m[hh] = mn;
        }
    }
    // the P remaining states to LDS: state p = wave (4 >> RS) + row >> RS, written by rows with
    // row % (1 << RS) == 0
    if ((row & ((1 << RS) - 1)) == 0) {
        const int p = wave * (4 >> RS) + (row >> RS);
#pragma unroll
        for (int hh = 0; hh < GRP; ++hh) {
#pragma unroll
            for (int d4 = 0; d4 < DPL / 4; ++d4)
                *reinterpret_cast<float4 *>(&red[p][hh][lane_quad<KV, DPL>(l16, d4)]) =
                    make_float4(acc[hh][4 * d4], acc[hh][4 * d4 + 1], acc[hh][4 * d4 + 2], acc[hh][4 * d4 + 3]);
            if (l16 == 0) {
                red[p][hh][D] = m[hh];
                red[p][hh][D + 1] = l[hh];
            }
        }
    }
    __syncthreads();
    // per head: M = max_p m_p, weights w_p = e^{m_p - M}, L = sum_p w_p l_p
    for (int i = threadIdx.x; i < GRP * P; i += 64 * NW) {
        const int hh = i / P, pi = i - hh * P;
        float M = kNegBig;
#pragma unroll
        for (int p = 0; p < P; ++p) M = fmaxf(M, red[p][hh][D]);
        wgt[hh][pi] = __expf(red[pi][hh][D] - M);
        if (pi == 0) {
            float L = 0.0f;
#pragma unroll
            for (int p = 0; p < P; ++p) L = fmaf(__expf(red[p][hh][D] - M), red[p][hh][D + 1], L);
            mrg[0][hh] = M;
            mrg[1][hh] = L;
        }
    }
    __syncthreads();

    // thread t owns (head t / D, dim t % D)
    const int64_t pair = (int64_t)b * G + g;
    for (int t = threadIdx.x; t < GRP * D; t += 64 * NW) {
        const int hh = t / D, d = t - hh * D;
        float A = 0.0f;
#pragma unroll
        for (int p = 0; p < P; ++p) A = fmaf(wgt[hh][p], red[p][hh][d], A);
        if (n_splits == 1) out[((int64_t)b * H + (int64_t)g * GRP + hh) * D + d] = A / mrg[1][hh];
        else store_partial<GRP, D>(part + ((pair * n_splits + split) * GRP + hh) * SLOT, d, A, mrg[0][hh], mrg[1][hh]);
    }
    if (n_splits > 1 && cnt != nullptr) {
        __shared__ int last;
        ticket_merge<GRP, D>(part + pair * n_splits * GRP * SLOT, cnt + pair, n_splits,
                             out + ((int64_t)b * H + (int64_t)g * GRP) * D, &red[0][0][0], &last);
    }
}

// bf16 state, D = 128: the same split decode attention on v_mfma_f32_16x16x32_bf16.  The GRP query
// heads of a KV group are the 16 MFMA columns (GRP <= 16), so per 32-key tile a wave computes
//   S^T (keys x heads) = K Q^T     A = K rows straight from HBM (lane: key l % 16, dims 8 (l / 16) ..
//                                  + 7 of a 32-dim chunk), B = Q^T as a bf16 hi + lo pair (fp32-level
//                                  scores);
//   O^T (dims x heads) += V^T P^T  A = V^T from a wave-private transposed LDS copy of the tile, B = P^T
//                                  straight from the S^T accumulators as a bf16 hi + lo pair.
// A lane of the 16 x 16 outputs owns one head, so the online softmax is lane-local (two cross-lane
// steps for the max and the final sum), exactly as in the prefill kernel.  The K-slot assignment of
// the second product (keys 4 lg .. + 3 and 16 + 4 lg .. + 3) is the same in A and B.  The tile walk,
// masking (rows past a span's device length are zeroed before use) and the partial format are those
// of attn_decode_kernel, and the splits are combined the same way.
constexpr int kMT = 32;                 // keys per MFMA tile
constexpr int kMVRow = kMT + 8;         // LDS row of V^T (bf16, 16 bytes of padding)

template <int GRP>
__global__ __launch_bounds__(64 * kWaves) void attn_decode_mfma_kernel(
    const float *__restrict__ q, int64_t ldq, SpanArgs sp, const float *__restrict__ bias, int64_t bias_hstride,
    int bias_span, float *__restrict__ out, float *__restrict__ part, int *__restrict__ cnt, int H, int G, float scale,
    int64_t n_tot, int64_t kps, int n_splits) {
    constexpr int D = 128;
    constexpr int SLOT = D + 2;
    static_assert(GRP <= 16, "heads per KV group must fit the 16 MFMA columns");
    __shared__ float red[kWaves][GRP][SLOT];
    __shared__ __align__(16) uint16_t vt[kWaves][D * kMVRow];

    const int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x & 63, l16 = lane & 15, lg = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint16_t *vw = vt[wave];

    const int64_t k0 = (int64_t)split * kps;
    const int64_t k1 = min(n_tot, k0 + kps);
    int lo[4], hi[4], eff[4];
    {
        int64_t base = 0;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int64_t len = s < sp.n ? sp.len[s] : 0;
            lo[s] = (int)(max(k0, base) - base);
            hi[s] = (int)(max(min(k1, base + len) - base, (int64_t)lo[s]));
            base += len;
        }
    }
    auto first_in = [&](int s0) -> int2 {
#pragma unroll
        for (int s = 0; s < 4; ++s)
            if (s >= s0 && lo[s] + wave * kMT < hi[s]) return make_int2(s, lo[s] + wave * kMT);
        return make_int2(4, 0);
    };
    auto next = [&](int2 c) -> int2 {
        if (c.y + kWaves * kMT < pick4(c.x, hi[0], hi[1], hi[2], hi[3])) return make_int2(c.x, c.y + kWaves * kMT);
        return first_in(c.x + 1);
    };

    // tile registers: K as the A operand (2 x 16 keys x 4 dim chunks), V rows as loaded
    uint4 kr[2][4], vr[4][2];
    auto fetch = [&](int2 c) {
        const int s = c.x;
        const uint16_t *kb = static_cast<const uint16_t *>(pick4(s, sp.k[0], sp.k[1], sp.k[2], sp.k[3]));
        const uint16_t *vb = static_cast<const uint16_t *>(pick4(s, sp.v[0], sp.v[1], sp.v[2], sp.v[3]));
        const int64_t o = (int64_t)b * pick4(s, sp.bstride[0], sp.bstride[1], sp.bstride[2], sp.bstride[3]) +
                          (int64_t)g * pick4(s, sp.gstride[0], sp.gstride[1], sp.gstride[2], sp.gstride[3]);
        const int last = pick4(s, hi[0], hi[1], hi[2], hi[3]) - 1;   // rows past it re-read it (masked)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            const int64_t row = min(c.y + kt * 16 + l16, last);
#pragma unroll
            for (int kc = 0; kc < 4; ++kc)
                kr[kt][kc] = *reinterpret_cast<const uint4 *>(kb + o + row * D + kc * 32 + lg * 8);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int ci = lane + 64 * i, rp = ci & 15, cc = ci >> 4;
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
                const int64_t row = min(c.y + 2 * rp + h2, last);
                vr[i][h2] = *reinterpret_cast<const uint4 *>(vb + o + row * D + cc * 8);
            }
        }
    };

    int2 cur = first_in(0);
    if (cur.x < 4) fetch(cur);

    // Q^T fragments of the group's heads: column l16 = head, dims 32 kc + 8 lg .. + 7, bf16 hi + lo
    bf16x8_t qh[4], ql[4];
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
        float e[8];
        if (l16 < GRP) {
            const float *qp = q + (int64_t)b * ldq + ((int64_t)g * GRP + l16) * D + kc * 32 + lg * 8;
            const float4 a0 = reinterpret_cast<const float4 *>(qp)[0], a1 = reinterpret_cast<const float4 *>(qp)[1];
            e[0] = a0.x; e[1] = a0.y; e[2] = a0.z; e[3] = a0.w; e[4] = a1.x; e[5] = a1.y; e[6] = a1.z; e[7] = a1.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) e[j] = 0.0f;
        }
        uint4 hw, lw;
        split_bf16x2(e[0], e[1], hw.x, lw.x);
        split_bf16x2(e[2], e[3], hw.y, lw.y);
        split_bf16x2(e[4], e[5], hw.z, lw.z);
        split_bf16x2(e[6], e[7], hw.w, lw.w);
        qh[kc] = __builtin_bit_cast(bf16x8_t, hw);
        ql[kc] = __builtin_bit_cast(bf16x8_t, lw);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        int64_t e = s < sp.n ? sp.len[s] : 0;
        if (s < sp.n && sp.dyn_len[s] != nullptr) e = min(e, (int64_t)*sp.dyn_len[s]);
        eff[s] = (int)min((int64_t)hi[s], max(e, (int64_t)0));
    }

    float m = kNegBig, lsum = 0.0f;
    f32x4_t o[8];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[dt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    const float *bh = (bias != nullptr && l16 < GRP) ? bias + ((int64_t)g * GRP + l16) * bias_hstride : nullptr;

    while (cur.x < 4) {
        const int s = cur.x;
        const int e = pick4(s, eff[0], eff[1], eff[2], eff[3]);
        // S^T = K Q^T
        f32x4_t sc[2];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            sc[kt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int kc = 0; kc < 4; ++kc) {
                const bf16x8_t a = __builtin_bit_cast(bf16x8_t, kr[kt][kc]);
                sc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qh[kc], sc[kt], 0, 0, 0);
                sc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, ql[kc], sc[kt], 0, 0, 0);
            }
        }
        // V^T of the tile into the wave's LDS copy; rows past the effective length become zeros
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int ci = lane + 64 * i, rp = ci & 15, cc = ci >> 4;
            const bool v0 = cur.y + 2 * rp < e, v1 = cur.y + 2 * rp + 1 < e;
            const uint32_t a0[4] = {vr[i][0].x, vr[i][0].y, vr[i][0].z, vr[i][0].w};
            const uint32_t a1[4] = {vr[i][1].x, vr[i][1].y, vr[i][1].z, vr[i][1].w};
#pragma unroll
            for (int q2 = 0; q2 < 4; ++q2) {
                const uint32_t x0 = v0 ? a0[q2] : 0u, x1 = v1 ? a1[q2] : 0u;
                *reinterpret_cast<uint32_t *>(vw + (cc * 8 + 2 * q2) * kMVRow + 2 * rp) = (x0 & 0xFFFFu) | (x1 << 16);
                *reinterpret_cast<uint32_t *>(vw + (cc * 8 + 2 * q2 + 1) * kMVRow + 2 * rp) =
                    (x0 >> 16) | (x1 & 0xFFFF0000u);
            }
        }
        // K and V of this tile are consumed: request the next tile now, behind the softmax and P V
        const int2 nx = next(cur);
        if (nx.x < 4) fetch(nx);
        // online softmax of head l16 over the tile's 32 keys (keys kt * 16 + 4 lg + i of this lane)
        float v[8];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int kk = cur.y + kt * 16 + lg * 4 + i;
                float t = sc[kt][i] * scale;
                if (bh != nullptr && s == bias_span && kk < e) t += bh[kk];
                v[kt * 4 + i] = kk < e ? t : -INFINITY;
            }
        float mt = v[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) mt = fmaxf(mt, v[i]);
        mt = xor32_max(xor16_max(mt));
        const float mn = fmaxf(m, mt);
        const float corr = __expf(m - mn);
        m = mn;
        float ps = 0.0f, pv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            pv[i] = __expf(v[i] - mn);
            ps += pv[i];
        }
        uint4 hw, lw;
        split_bf16x2(pv[0], pv[1], hw.x, lw.x);
        split_bf16x2(pv[2], pv[3], hw.y, lw.y);
        split_bf16x2(pv[4], pv[5], hw.z, lw.z);
        split_bf16x2(pv[6], pv[7], hw.w, lw.w);
        const bf16x8_t ph = __builtin_bit_cast(bf16x8_t, hw), pl = __builtin_bit_cast(bf16x8_t, lw);
        lsum = lsum * corr + ps;
        if (__ballot(corr != 1.0f)) {
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) o[dt] *= corr;
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the wave's V^T stores before its reads
        // O^T += V^T P^T
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            const uint16_t *vrow = vw + (dt * 16 + l16) * kMVRow + lg * 4;
            const uint2 x0 = *reinterpret_cast<const uint2 *>(vrow);
            const uint2 x1 = *reinterpret_cast<const uint2 *>(vrow + 16);
            const bf16x8_t va = __builtin_bit_cast(bf16x8_t, make_uint4(x0.x, x0.y, x1.x, x1.y));
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, ph, o[dt], 0, 0, 0);
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pl, o[dt], 0, 0, 0);
        }
        cur = nx;
    }

    // wave state -> LDS: lane (lg, head l16) holds dims dt * 16 + 4 lg + i
    const float L = xor32_sum(xor16_sum(lsum));
    if (l16 < GRP) {
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[wave][l16][dt * 16 + lg * 4 + i] = o[dt][i];
        if (lg == 0) {
            red[wave][l16][D] = m;
            red[wave][l16][D + 1] = L;
        }
    }
    __syncthreads();

    const int64_t pair = (int64_t)b * G + g;
    for (int t = threadIdx.x; t < GRP * D; t += 64 * kWaves) {
        const int hh = t / D, d = t - hh * D;
        float M = kNegBig;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) M = fmaxf(M, red[w][hh][D]);
        float Ls = 0.0f, A = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float c = __expf(red[w][hh][D] - M);
            Ls = fmaf(c, red[w][hh][D + 1], Ls);
            A = fmaf(c, red[w][hh][d], A);
        }
        if (n_splits == 1) out[((int64_t)b * H + (int64_t)g * GRP + hh) * D + d] = A / Ls;
        else store_partial<GRP, D>(part + ((pair * n_splits + split) * GRP + hh) * SLOT, d, A, M, Ls);
    }
    if (n_splits > 1 && cnt != nullptr) {
        __shared__ int last;
        ticket_merge<GRP, D>(part + pair * n_splits * GRP * SLOT, cnt + pair, n_splits,
                             out + ((int64_t)b * H + (int64_t)g * GRP) * D, &red[0][0][0], &last);
    }
}

// One workgroup of D threads per (b, h): out = sum_s e^{m_s - M} acc_s / sum_s e^{m_s - M} l_s.
// Every load is issued before the one barrier: thread d requests acc_s[d] of all n_splits splits, and
// the first wave also (m_s, l_s) of split s = lane; that wave turns them into the split weights in
// LDS.  One round trip to the partials instead of one per dependent step.
__global__ __launch_bounds__(128) void attn_merge_kernel(const float *__restrict__ part, float *__restrict__ out,
                                                         int H, int G, int D, int n_splits) {
    __shared__ float wgt[kMaxSplits];
    __shared__ float inv_l;
    const int bh = blockIdx.x;
    const int b = bh / H, h = bh - b * H;
    const int grp = H / G, g = h / grp, hh = h - g * grp;
    const int64_t stride = (int64_t)grp * (D + 2);
    const float *p0 = part + (((int64_t)b * G + g) * n_splits * grp + hh) * (D + 2);
    const int d = threadIdx.x;
    // Unconditional loads (splits past n_splits re-read the last one and get weight 0): a branch per
    // load would make the compiler wait for each load before the next.
    float v[kMaxSplits];
#pragma unroll
    for (int s = 0; s < kMaxSplits; ++s) v[s] = p0[min(s, n_splits - 1) * stride + d];
    if (threadIdx.x < 64) {
        const int s = threadIdx.x;
        const float *ps = p0 + min(s, n_splits - 1) * stride;
        const float ms = s < n_splits ? ps[D] : kNegBig;
        const float ls = s < n_splits ? ps[D + 1] : 0.0f;
        const float M = wave_max(ms);
        const float w = s < n_splits ? __expf(ms - M) : 0.0f;
        const float L = wave_sum(w * ls);
        wgt[s] = w;
        if (s == 0) inv_l = 1.0f / L;
    }
    __syncthreads();
    float a = 0.0f;
#pragma unroll
    for (int s = 0; s < kMaxSplits; ++s) a = fmaf(wgt[s], v[s], a);
    out[((int64_t)b * H + h) * D + d] = a * inv_l;
}

// Few (batch, group) pairs (the batch-1 decode step), D = 128: one split of 4 KB NW keys per
// workgroup, every wave on one 4 KB-key tile, so each wave's serial chain is short and many splits
// keep most CUs streaming the keys.
//   q        staged once per workgroup in LDS (scaled), read by every DPP row;
//   scores   the wave's 4 DPP rows take KB keys each (a key row over the 16 lanes of a row: dims
//            4 l .. + 3 and 64 + 4 l .. + 3 of lane l), q . k summed over the row by DPP; lane hh of a
//            row writes head hh's score to LDS;
//   softmax  over the workgroup's keys per head (one wave per head), exactly: max, exp, sum;
//   P V      each lane weights its own K/V rows' V by the probabilities (read back from LDS), the 4
//            rows of a wave are summed by two lane-swap steps, the waves through LDS in a fixed order;
//   splits   MERGE: every workgroup stores (m, l, acc) with agent-scope stores and takes a ticket; the
//            last workgroup of the pair merges every split (agent-scope vector loads issued at once,
//            weights e^{m_s - M} / L), then resets the ticket (the ordering argument of ticket_merge).
//            Otherwise the partials are plain stores and b1_merge_kernel, a second launch spread over
//            (head, 32 dims) workgroups, merges them.
// Keys are dealt by capacity over the concatenated spans; a key at or past its span's device length, or
// past the last span, gets score -inf and weight 0 (its V row is zeroed) and reads an existing row.
constexpr int kB1MaxSplits = 128;
constexpr int kB1MaxPairs = 4;               // (batch, group) pairs the kernel takes (beyond: the tiled kernels)
constexpr int kB1Chunk = 32;                 // split partials one merging thread requests at once
constexpr int kSC1 = 16;                     // the sc1 cache-policy bit of a buffer access: agent coherent

// One lane's dims 4 l .. + 3 (at elem_off) and 64 + 4 l .. + 3 of a key row, as fp32.
template <int KV>
__device__ __forceinline__ void load_quads(const void *base, int64_t elem_off, float (&f)[8]) {
    if constexpr (KV == VGX_F32) {
        const float *p = static_cast<const float *>(base) + elem_off;
        const float4 a = ld_stream(reinterpret_cast<const float4 *>(p)), c = ld_stream(reinterpret_cast<const float4 *>(p + 64));
        f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = c.x; f[5] = c.y; f[6] = c.z; f[7] = c.w;
    } else {
        const uint16_t *p = static_cast<const uint16_t *>(base) + elem_off;
        const uint2 a = ld_stream(reinterpret_cast<const uint2 *>(p)), c = ld_stream(reinterpret_cast<const uint2 *>(p + 64));
        f[0] = __uint_as_float(a.x << 16); f[1] = __uint_as_float(a.x & 0xFFFF0000u);
        f[2] = __uint_as_float(a.y << 16); f[3] = __uint_as_float(a.y & 0xFFFF0000u);
        f[4] = __uint_as_float(c.x << 16); f[5] = __uint_as_float(c.x & 0xFFFF0000u);
        f[6] = __uint_as_float(c.y << 16); f[7] = __uint_as_float(c.y & 0xFFFF0000u);
    }
}

// Partials of the kernel: acc [pair][split][head][128] floats, then (m, l) [pair][split][head][2] from
// float offset ml_off (the acc region rounded up to 256 bytes).
inline int64_t b1_ml_off(int64_t pairs, int64_t grp, int ns) { return (pairs * ns * grp * 128 + 63) / 64 * 64; }
inline int64_t b1_part_bytes(int64_t pairs, int64_t grp, int ns) {
    return (b1_ml_off(pairs, grp, ns) + pairs * ns * grp * 2) * (int64_t)sizeof(float);
}

template <int KV, int GRP, int NW, int KB, int MERGE, bool ALIGNED>
__global__ __launch_bounds__(64 * NW) void attn_decode_b1_kernel(
    const float *__restrict__ q, int64_t ldq, SpanArgs sp, const float *__restrict__ bias, int64_t bias_hstride,
    int bias_span, float *__restrict__ out, float *__restrict__ part, int64_t ml_off, int *__restrict__ cnt, int H,
    int G, float scale, int64_t n_tot, int n_splits) {
    constexpr int D = 128, NT = 64 * NW, KWV = 4 * KB, KWG = NW * KWV;
    constexpr int KPL = (KWG + 63) / 64;               // keys per lane in the softmax
    constexpr int NTASK = GRP * (D / 4);               // merge tasks: (head, 4 dims)
    constexpr int NSUB = NT / NTASK;                   // threads per merge task
    static_assert(!MERGE || NSUB >= 1, "a thread per merge task");
    __shared__ __align__(16) float qs[GRP][D];
    constexpr int RB = NW * GRP * D > 2 * GRP * kB1MaxSplits + 4 * NSUB * NTASK ? NW * GRP * D
                                                                                  : 2 * GRP * kB1MaxSplits + 4 * NSUB * NTASK;
    __shared__ float sc[GRP + 1][KWG];                // row GRP: the writes of lanes with no head
    __shared__ __align__(16) float redbuf[RB];         // per-wave P V sums; the merge's scratch after
    float (*red)[GRP][D] = reinterpret_cast<float (*)[GRP][D]>(redbuf);
    __shared__ float mh[GRP], lh[GRP];
    __shared__ int last;

    const int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, row = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // span bases by capacity
    int64_t base[5];
    base[0] = 0;
#pragma unroll
    for (int s = 0; s < 4; ++s) base[s + 1] = base[s] + (s < sp.n ? sp.len[s] : 0);

    // Requests first, in the order they are used: q (staged to LDS before the first barrier), V of the
    // wave's KWV keys (lane l: dims 2 l, 2 l + 1 of each, so the P V product needs no exchange between
    // lanes), K of this lane's KB keys in the DPP-row layout.  Device lengths and the bias after them.
    float4 qv[(GRP * 32 + 64 * NW - 1) / (64 * NW)];
#pragma unroll
    for (int u = 0; u < (GRP * 32 + 64 * NW - 1) / (64 * NW); ++u) {
        const int i = tid + u * 64 * NW;
        if (i < GRP * 32) qv[u] = *reinterpret_cast<const float4 *>(q + (int64_t)b * ldq + (int64_t)g * GRP * D + 4 * i);
    }
    // row 0 of every span for this (batch, group)
    constexpr int ESZ = KV == VGX_F32 ? 4 : 2;
    const char *kp[4], *vp[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int64_t o = ((int64_t)b * sp.bstride[s] + (int64_t)g * sp.gstride[s]) * ESZ;
        kp[s] = static_cast<const char *>(sp.k[s]) + o;
        vp[s] = static_cast<const char *>(sp.v[s]) + o;
    }
    // V: lane l holds dims 4 (l % 32) .. + 3 of the wave's keys 2 j + l / 32 (j < KWV / 2): every load
    // instruction reads two whole rows.  K: this lane's KB keys in the DPP-row layout.  ALIGNED (every
    // span's capacity a multiple of KWV): a wave's keys lie in one span, found once per wave.
    constexpr int KVH = KWV / 2;
    float vf[KVH][4];
    int vs_[KVH];
    int64_t vl_[KVH];
    const int half = lane >> 5, l32 = lane & 31;
    int ks[KB];
    int64_t kl[KB];
    float kf[KB][8];
    if constexpr (ALIGNED) {
        const int64_t kw0 = (int64_t)split * KWG + wave * KWV;                     // wave-uniform
        const bool live = kw0 < n_tot;                                             // then all KWV keys are
        int s = 0;
#pragma unroll
        for (int t = 1; t < 4; ++t) s = min(kw0, n_tot - 1) >= base[t] ? t : s;
        s = __builtin_amdgcn_readfirstlane(s);
        const int64_t r0 = live ? kw0 - pick4(s, base[0], base[1], base[2], base[3]) : 0;
        const char *vrow = pick4(s, vp[0], vp[1], vp[2], vp[3]) + r0 * D * ESZ;
        const char *krow = pick4(s, kp[0], kp[1], kp[2], kp[3]) + r0 * D * ESZ;
#pragma unroll
        for (int j = 0; j < KVH; ++j) {
            vs_[j] = live ? s : -1;
            vl_[j] = r0 + 2 * j + half;
            const char *vr = vrow + (int64_t)(2 * j + half) * D * ESZ;
            if constexpr (KV == VGX_F32) {
                const float4 t = ld_stream(reinterpret_cast<const float4 *>(vr) + l32);
                vf[j][0] = t.x; vf[j][1] = t.y; vf[j][2] = t.z; vf[j][3] = t.w;
            } else {
                const uint2 t = ld_stream(reinterpret_cast<const uint2 *>(vr) + l32);
                vf[j][0] = __uint_as_float(t.x << 16); vf[j][1] = __uint_as_float(t.x & 0xFFFF0000u);
                vf[j][2] = __uint_as_float(t.y << 16); vf[j][3] = __uint_as_float(t.y & 0xFFFF0000u);
            }
        }
#pragma unroll
        for (int kk = 0; kk < KB; ++kk) {
            ks[kk] = live ? s : -1;
            kl[kk] = r0 + row * KB + kk;
            load_quads<KV>(krow, (int64_t)(row * KB + kk) * D + 4 * l16, kf[kk]);
        }
    } else {
#pragma unroll
        for (int j = 0; j < KVH; ++j) {
            const int64_t gk = (int64_t)split * KWG + wave * KWV + 2 * j + half;
            const int64_t ga = min(gk, n_tot - 1);
            int s = 0;
#pragma unroll
            for (int t = 1; t < 4; ++t) s = ga >= base[t] ? t : s;
            const int64_t lr = ga - pick4(s, base[0], base[1], base[2], base[3]);
            vs_[j] = gk < n_tot ? s : -1;
            vl_[j] = lr;
            const char *vrow = pick4(s, vp[0], vp[1], vp[2], vp[3]) + lr * D * ESZ;
            if constexpr (KV == VGX_F32) {
                const float4 t = ld_stream(reinterpret_cast<const float4 *>(vrow) + l32);
                vf[j][0] = t.x; vf[j][1] = t.y; vf[j][2] = t.z; vf[j][3] = t.w;
            } else {
                const uint2 t = ld_stream(reinterpret_cast<const uint2 *>(vrow) + l32);
                vf[j][0] = __uint_as_float(t.x << 16); vf[j][1] = __uint_as_float(t.x & 0xFFFF0000u);
                vf[j][2] = __uint_as_float(t.y << 16); vf[j][3] = __uint_as_float(t.y & 0xFFFF0000u);
            }
        }
#pragma unroll
        for (int kk = 0; kk < KB; ++kk) {
            const int64_t gk = (int64_t)split * KWG + wave * KWV + row * KB + kk;
            const int64_t ga = min(gk, n_tot - 1);          // an existing key for the address
            int s = 0;
#pragma unroll
            for (int t = 1; t < 4; ++t) s = ga >= base[t] ? t : s;
            ks[kk] = gk < n_tot ? s : -1;
            kl[kk] = ga - pick4(s, base[0], base[1], base[2], base[3]);
            load_quads<KV>(pick4(s, kp[0], kp[1], kp[2], kp[3]), kl[kk] * D + 4 * l16, kf[kk]);
        }
    }
    // bias rows of the biased span (clamped to its last column; used only where it applies)
    float bv[GRP][KB];
    if (bias != nullptr) {
        const int64_t bl = sp.len[bias_span] - 1;
#pragma unroll
        for (int kk = 0; kk < KB; ++kk)
#pragma unroll
            for (int hh = 0; hh < GRP; ++hh)
                bv[hh][kk] = bias[((int64_t)g * GRP + hh) * bias_hstride + min(kl[kk], bl)];
    }
    // q -> LDS, scaled
#pragma unroll
    for (int u = 0; u < (GRP * 32 + 64 * NW - 1) / (64 * NW); ++u) {
        const int i = tid + u * 64 * NW;
        if (i < GRP * 32)
            *reinterpret_cast<float4 *>(&qs[0][0] + 4 * i) =
                make_float4(qv[u].x * scale, qv[u].y * scale, qv[u].z * scale, qv[u].w * scale);
    }
    // effective span lengths (device lengths) and the keys' validity
    int64_t eff[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        eff[s] = s < sp.n ? sp.len[s] : 0;
        if (s < sp.n && sp.dyn_len[s] != nullptr) eff[s] = min(eff[s], (int64_t)*sp.dyn_len[s]);
    }
    bool vok[KVH], valid[KB];
#pragma unroll
    for (int j = 0; j < KVH; ++j) vok[j] = vs_[j] >= 0 && vl_[j] < pick4(max(vs_[j], 0), eff[0], eff[1], eff[2], eff[3]);
#pragma unroll
    for (int kk = 0; kk < KB; ++kk) {
        valid[kk] = ks[kk] >= 0 && kl[kk] < pick4(max(ks[kk], 0), eff[0], eff[1], eff[2], eff[3]);
        const bool biased = bias != nullptr && valid[kk] && ks[kk] == bias_span;
#pragma unroll
        for (int hh = 0; hh < GRP; ++hh) bv[hh][kk] = biased ? bv[hh][kk] : 0.0f;
    }
    __syncthreads();
    // scores: the GRP * KB row sums interleaved step by step (independent DPP operations between
    // dependent ones); lane hh of each row writes head hh, lanes past the heads a spare row
    {
        float sv[GRP][KB];
#pragma unroll
        for (int hh = 0; hh < GRP; ++hh) {
            const float4 qa = *reinterpret_cast<const float4 *>(&qs[hh][4 * l16]);
            const float4 qc = *reinterpret_cast<const float4 *>(&qs[hh][64 + 4 * l16]);
            const float qv[8] = {qa.x, qa.y, qa.z, qa.w, qc.x, qc.y, qc.z, qc.w};
#pragma unroll
            for (int kk = 0; kk < KB; ++kk) {
                float p = 0.0f;
#pragma unroll
                for (int dd = 0; dd < 8; ++dd) p = fmaf(qv[dd], kf[kk][dd], p);
                sv[hh][kk] = p;
            }
        }
#pragma unroll
        for (int hh = 0; hh < GRP; ++hh)
#pragma unroll
            for (int kk = 0; kk < KB; ++kk) sv[hh][kk] += dpp_f<DPP_QUAD_1032>(sv[hh][kk]);
#pragma unroll
        for (int hh = 0; hh < GRP; ++hh)
#pragma unroll
            for (int kk = 0; kk < KB; ++kk) sv[hh][kk] += dpp_f<DPP_QUAD_2301>(sv[hh][kk]);
#pragma unroll
        for (int hh = 0; hh < GRP; ++hh)
#pragma unroll
            for (int kk = 0; kk < KB; ++kk) sv[hh][kk] += dpp_f<DPP_ROW_HALF_MIRROR>(sv[hh][kk]);
#pragma unroll
        for (int hh = 0; hh < GRP; ++hh)
#pragma unroll
            for (int kk = 0; kk < KB; ++kk) sv[hh][kk] += dpp_f<DPP_ROW_MIRROR>(sv[hh][kk]);
        const int wr = l16 < GRP ? l16 : GRP;
#pragma unroll
        for (int kk = 0; kk < KB; ++kk) {
            float mine = 0.0f;
#pragma unroll
            for (int hh = 0; hh < GRP; ++hh) mine = l16 == hh ? sv[hh][kk] + bv[hh][kk] : mine;
            sc[wr][wave * KWV + row * KB + kk] = valid[kk] ? mine : -INFINITY;
        }
    }
    __syncthreads();
    // softmax of head hh over the workgroup's keys
    for (int hh = wave; hh < GRP; hh += NW) {
        float x[KPL];
        float mx = -INFINITY;
#pragma unroll
        for (int u = 0; u < KPL; ++u) {
            x[u] = lane + 64 * u < KWG ? sc[hh][lane + 64 * u] : -INFINITY;
            mx = fmaxf(mx, x[u]);
        }
        float m = wave_max(mx);
        float ps = 0.0f;
        const bool none = m == -INFINITY;                // no valid key: weight 0 everywhere
        if (none) m = kNegBig;
#pragma unroll
        for (int u = 0; u < KPL; ++u) {
            const float p = none ? 0.0f : __expf(x[u] - m);
            ps += p;
            if (lane + 64 * u < KWG) sc[hh][lane + 64 * u] = p;
        }
        const float l = wave_sum(ps);
        if (lane == 0) {
            mh[hh] = m;
            lh[hh] = l;
        }
    }
    __syncthreads();
    // P V: lane l accumulates dims 4 (l % 32) .. + 3 of every head over its half of the wave's keys (a
    // key past its span's device length weighs 0; its V row, which may hold anything, is replaced by
    // zeros), the halves summed by one lane swap
#pragma unroll
    for (int hh = 0; hh < GRP; ++hh) {
        float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < KVH; ++j) {
            const float p = sc[hh][wave * KWV + 2 * j + half];
#pragma unroll
            for (int e = 0; e < 4; ++e) a[e] = fmaf(p, vok[j] ? vf[j][e] : 0.0f, a[e]);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) a[e] = xor32_sum(a[e]);
        if (half == 0) *reinterpret_cast<float4 *>(&red[wave][hh][4 * l32]) = make_float4(a[0], a[1], a[2], a[3]);
    }
    __syncthreads();
    const int64_t pair = (int64_t)b * G + g;
    float *pa = part + (pair * n_splits + split) * GRP * D;
    for (int t = tid; t < GRP * D; t += NT) {
        const int hh = t / D, d = t - hh * D;
        float a = red[0][hh][d];
#pragma unroll
        for (int w = 1; w < NW; ++w) a += red[w][hh][d];
        if (n_splits == 1) out[((int64_t)b * H + (int64_t)g * GRP + hh) * D + d] = a * (1.0f / lh[hh]);
        else if constexpr (MERGE) __hip_atomic_store(pa + t, a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else pa[t] = a;
    }
    if (n_splits == 1) return;
    if (tid < GRP) {
        float *pm = part + ml_off + ((pair * n_splits + split) * GRP + tid) * 2;
        if constexpr (MERGE) {
            __hip_atomic_store(pm, mh[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(pm + 1, lh[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            pm[0] = mh[tid];
            pm[1] = lh[tid];
        }
    }
    if constexpr (!MERGE) return;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");    // this thread's partial stores have completed
    __syncthreads();
    if (tid == 0)
        last = __hip_atomic_fetch_add(cnt + pair, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == n_splits - 1;
    __syncthreads();
    if (!last) return;
    // MERGE 2: an agent-scope acquire (the L2 lines that may hold stale partials are invalidated), then
    // plain loads; MERGE 1: loads that read the device-coherent level (sc1)
    if constexpr (MERGE == 2) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    constexpr int kLoadAux = MERGE == 2 ? 0 : kSC1;

    // The last workgroup.  (m, l) of every (split, head) and the first chunk of each thread's split
    // values are requested before any is used; tasks (head, 4 dims) with NSUB threads each, thread sub
    // taking splits sub, sub + NSUB, ...  Buffer bounds end at the pair's partials: requests past the
    // last split read zeros.
    float *mm = redbuf;                           // [GRP][kB1MaxSplits] m, then weights
    float *ll = mm + GRP * kB1MaxSplits;                 // [GRP][kB1MaxSplits] l
    float4 *rsum = reinterpret_cast<float4 *>(ll + GRP * kB1MaxSplits);   // [NSUB][NTASK]
    const __amdgpu_buffer_rsrc_t ars =
        __builtin_amdgcn_make_buffer_rsrc(part + pair * n_splits * GRP * D, 0, n_splits * GRP * D * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t mrs =
        __builtin_amdgcn_make_buffer_rsrc(part + ml_off + pair * n_splits * GRP * 2, 0, n_splits * GRP * 8, 0x00020000);
    constexpr int NE = (GRP * kB1MaxSplits + NT - 1) / NT;
    uint32_t mlw[NE][2];
#pragma unroll
    for (int u = 0; u < NE; ++u) {
        const auto w = __builtin_amdgcn_raw_buffer_load_b64(mrs, (tid + u * NT) * 8, 0, kLoadAux);
        mlw[u][0] = w[0];
        mlw[u][1] = w[1];
    }
    const int task = tid % NTASK, sub = tid / NTASK;
    const bool active = sub < NSUB;
    const int th = task / (D / 4), td4 = task % (D / 4);
    float4 vals[kB1Chunk];
    auto request = [&](int c0) {
#pragma unroll
        for (int u = 0; u < kB1Chunk; ++u) {
            const int s = c0 + sub + u * NSUB;
            const auto w = __builtin_amdgcn_raw_buffer_load_b128(ars, (s * GRP + th) * D * 4 + td4 * 16, 0, kLoadAux);
            vals[u] = make_float4(__uint_as_float(w[0]), __uint_as_float(w[1]), __uint_as_float(w[2]),
                                  __uint_as_float(w[3]));
        }
    };
    if (active) request(0);
#pragma unroll
    for (int u = 0; u < NE; ++u) {
        const int e = tid + u * NT;                      // entry (split e / GRP, head e % GRP)
        if (e < n_splits * GRP) {
            const int s = e / GRP, hh = e - s * GRP;
            mm[hh * kB1MaxSplits + s] = __uint_as_float(mlw[u][0]);
            ll[hh * kB1MaxSplits + s] = __uint_as_float(mlw[u][1]);
        }
    }
    __syncthreads();
    // weights w_s / L per head: one wave per head, two splits per lane
    for (int hh = wave; hh < GRP; hh += NW) {
        const int s0 = lane, s1 = lane + 64;
        const float m0 = s0 < n_splits ? mm[hh * kB1MaxSplits + s0] : kNegBig;
        const float m1 = s1 < n_splits ? mm[hh * kB1MaxSplits + s1] : kNegBig;
        const float M = wave_max(fmaxf(m0, m1));
        const float w0 = s0 < n_splits ? __expf(m0 - M) : 0.0f;
        const float w1 = s1 < n_splits ? __expf(m1 - M) : 0.0f;
        const float L = wave_sum(fmaf(w0, s0 < n_splits ? ll[hh * kB1MaxSplits + s0] : 0.0f,
                                      w1 * (s1 < n_splits ? ll[hh * kB1MaxSplits + s1] : 0.0f)));
        const float inv = 1.0f / L;
        if (s0 < n_splits) mm[hh * kB1MaxSplits + s0] = w0 * inv;
        if (s1 < n_splits) mm[hh * kB1MaxSplits + s1] = w1 * inv;
    }
    __syncthreads();
    float4 a4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (active) {
        for (int c0 = 0; c0 < n_splits; c0 += kB1Chunk * NSUB) {
            if (c0) request(c0);
#pragma unroll
            for (int u = 0; u < kB1Chunk; ++u) {
                const int s = c0 + sub + u * NSUB;
                if (s < n_splits) {
                    const float w = mm[th * kB1MaxSplits + s];
                    a4.x = fmaf(w, vals[u].x, a4.x);
                    a4.y = fmaf(w, vals[u].y, a4.y);
                    a4.z = fmaf(w, vals[u].z, a4.z);
                    a4.w = fmaf(w, vals[u].w, a4.w);
                }
            }
        }
        rsum[sub * NTASK + task] = a4;
    }
    __syncthreads();
    if (active && sub == 0) {
#pragma unroll
        for (int u = 1; u < NSUB; ++u) {
            const float4 r = rsum[u * NTASK + task];
            a4.x += r.x; a4.y += r.y; a4.z += r.z; a4.w += r.w;
        }
        *reinterpret_cast<float4 *>(out + ((int64_t)b * H + (int64_t)g * GRP + th) * D + td4 * 4) = a4;
    }
    if (tid == 0) __hip_atomic_store(cnt + pair, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The second launch of the kernel above (partials as plain stores): one wave per (batch, head, 32 dims).
// Lane l takes float4 l & 7 of the 32 dims over splits l >> 3, + 8, ...; (m, l) of split = lane (two per
// lane up to 128 splits); all requested before any is used, as unconditional buffer loads (requests
// past the last split read zeros), so the loads stay in flight together; lanes sharing a float4 summed
// by swaps.
__global__ __launch_bounds__(64) void b1_merge_kernel(const float *__restrict__ part, int64_t ml_off,
                                                      float *__restrict__ out, int H, int G, int n_splits) {
    constexpr int D = 128;
    const int bh = blockIdx.x, dq = blockIdx.y, lane = threadIdx.x;
    const int b = bh / H, h = bh - b * H, grp = H / G, g = h / grp, hh = h - g * grp;
    const int64_t pair = (int64_t)b * G + g;
    const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(part) + pair * n_splits * grp * D, 0, n_splits * grp * D * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t mrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(part) + ml_off + pair * n_splits * grp * 2, 0, n_splits * grp * 8, 0x00020000);
    constexpr int kPer = kB1MaxSplits / 8;
    const int nper = (n_splits + 7) / 8;                  // splits per lane group (uniform)
    float4 v[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        if (u < nper) {
            const int s = (lane >> 3) + 8 * u;
            const auto w = __builtin_amdgcn_raw_buffer_load_b128(ars, ((s * grp + hh) * D + dq * 32 + (lane & 7) * 4) * 4, 0, 0);
            v[u] = make_float4(__uint_as_float(w[0]), __uint_as_float(w[1]), __uint_as_float(w[2]), __uint_as_float(w[3]));
        }
    }
    const auto ml0 = __builtin_amdgcn_raw_buffer_load_b64(mrs, (lane * grp + hh) * 8, 0, 0);
    const auto ml1 = __builtin_amdgcn_raw_buffer_load_b64(mrs, ((lane + 64) * grp + hh) * 8, 0, 0);
    const float m0 = lane < n_splits ? __uint_as_float(ml0[0]) : kNegBig;
    const float l0 = lane < n_splits ? __uint_as_float(ml0[1]) : 0.0f;
    const float m1 = lane + 64 < n_splits ? __uint_as_float(ml1[0]) : kNegBig;
    const float l1 = lane + 64 < n_splits ? __uint_as_float(ml1[1]) : 0.0f;
    const float M = wave_max(fmaxf(m0, m1));
    const float w0 = lane < n_splits ? __expf(m0 - M) : 0.0f;
    const float w1 = lane + 64 < n_splits ? __expf(m1 - M) : 0.0f;
    const float inv = 1.0f / wave_sum(fmaf(w0, l0, w1 * l1));
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        if (u < nper) {
            const int s = (lane >> 3) + 8 * u;           // split s's weight: w0 (s < 64) or w1 of lane s % 64
            const float wlo = __shfl(w0, s & 63, 64), whi = __shfl(w1, s & 63, 64);
            const float w = s < n_splits ? (s < 64 ? wlo : whi) : 0.0f;
            a.x = fmaf(w, v[u].x, a.x); a.y = fmaf(w, v[u].y, a.y);
            a.z = fmaf(w, v[u].z, a.z); a.w = fmaf(w, v[u].w, a.w);
        }
    }
#pragma unroll
    for (int off = 8; off < 64; off <<= 1) {
        a.x += __shfl_xor(a.x, off, 64); a.y += __shfl_xor(a.y, off, 64);
        a.z += __shfl_xor(a.z, off, 64); a.w += __shfl_xor(a.w, off, 64);
    }
    if (lane < 8)
        *reinterpret_cast<float4 *>(out + ((int64_t)b * H + h) * D + dq * 32 + lane * 4) =
            make_float4(a.x * inv, a.y * inv, a.z * inv, a.w * inv);
}

// The shape of the kernel and how its splits merge: waves per workgroup, keys per DPP row, and the
// merge in the last workgroup (ticket) or in b1_merge_kernel.
constexpr int kB1NW = 8, kB1KB = 2;
constexpr int kB1Ticket = 0;              // 0: b1_merge_kernel, 1 / 2: the last workgroup (sc1 / acquire)
constexpr int kB1Keys = 4 * kB1KB * kB1NW;       // keys per workgroup (one split)
// Splits of the kernel for a call, 0 when it does not take the call's shape.
inline int b1_splits(int64_t B, int64_t G, int64_t D, int64_t n_keys) {
    if (D != 128 || B * G > kB1MaxPairs) return 0;
    const int64_t ns = (n_keys + kB1Keys - 1) / kB1Keys;
    return ns <= kB1MaxSplits ? (int)ns : 0;
}

// Workgroup shapes of the VALU kernel: waves per workgroup, keys per DPP row of a wave tile.
struct Tiling {
    int nw, kb;
};
constexpr Tiling kTilings[] = {{4, 4}, {8, 2}};
constexpr int kNumTilings = sizeof(kTilings) / sizeof(kTilings[0]);

// Measured on MI355X, fp32 K/V, 12 query / 2 KV heads, 3584 keys (attention + merge per layer): batch 1
// 11.7 us with 4 waves x 16-key tiles against 12.0 us with 8 waves x 8-key tiles (and 13.0 / 15.8 us for
// 4 x 8 / 8 x 16); batch 4 16.4 vs 20.0 us; batch 16 36.6 vs 34.1 us; batch 64 101.7 vs 90.3 us.
int pick_tiling(int64_t B, int64_t G) { return B * G >= 32 ? 1 : 0; }

// LDS budget of the cross-row merge: RS lane-swap steps first when the P states would not fit.
constexpr int pick_rs(int grp, int dpl, int nw) {
    return nw * 4 * grp * (dpl * 16 + 2) * 4 <= 52 * 1024 ? 0 : nw * 2 * grp * (dpl * 16 + 2) * 4 <= 52 * 1024 ? 1 : 2;
}

int choose_splits(int64_t B, int64_t G, int64_t n_tot, int64_t *kps, int tiling) {
    // About kTargetWaves waves in flight, at least one tile per wave, at most kMaxSplits.
    const int nw = kTilings[tiling].nw, tk = 4 * kTilings[tiling].kb;
    const int64_t pairs = B * G;
    int64_t want = (kTargetWaves / nw + pairs - 1) / pairs;
    const int64_t cap = (n_tot + nw * tk - 1) / (nw * tk);
    want = std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>(want, cap), kMaxSplits));
    int64_t k = (n_tot + want - 1) / want;
    k = (k + tk - 1) / tk * tk;
    *kps = k;
    return (int)((n_tot + k - 1) / k);
}

// Splits of the MFMA kernel: the same target, 32-key tiles, at least one tile per wave.
int choose_splits_mfma(int64_t B, int64_t G, int64_t n_tot, int64_t *kps) {
    const int64_t pairs = B * G;
    int64_t want = (kTargetWaves / kWaves + pairs - 1) / pairs;
    const int64_t cap = (n_tot + kWaves * kMT - 1) / (kWaves * kMT);
    want = std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>(want, cap), kMaxSplits));
    int64_t k = (n_tot + want - 1) / want;
    k = (k + kMT - 1) / kMT * kMT;
    *kps = k;
    return (int)((n_tot + k - 1) / k);
}

int64_t partial_bytes(int64_t B, int64_t H, int64_t D, int ns) {
    return B * H * (int64_t)ns * (D + 2) * (int64_t)sizeof(float);
}

// Workspace: a fixed region of kTicketPairs split tickets (one int32 per (b, g), kept at zero between
// launches) first, then the partials.  The region's size does not depend on the call, so the partials
// of one call never overlap the tickets of another call sharing the workspace, whatever their batch
// and group counts.  Up to kTicketMaxSplits splits of a pair are merged by the pair's last workgroup
// when the pair has a ticket (b * G + g < kTicketPairs); otherwise attn_merge_kernel spreads the
// merge over B * H workgroups.
constexpr int64_t kTicketPairs = 4096;
int64_t ticket_bytes(int64_t, int64_t) { return kTicketPairs * 4; }
bool use_tickets(int64_t B, int64_t G, int ns) { return ns <= kTicketMaxSplits && B * G <= kTicketPairs; }

template <int KV, int GRP, int DPL, int NW, int KB>
void launch_tiled(dim3 grid, hipStream_t st, const float *q, int64_t ldq, const SpanArgs &sp, const float *bias,
                  int64_t bhs, int bspan, float *out, float *part, int *cnt, int H, int G, float scale,
                  int64_t n_tot, int64_t kps, int ns, int64_t cb) {
    constexpr int RS = pick_rs(GRP, DPL, NW);
    hipLaunchKernelGGL((attn_decode_kernel<KV, GRP, DPL, NW, KB, RS>), grid, dim3(64 * NW), 0, st, q, ldq, sp, bias,
                       bhs, bspan, out, part, cnt, H, G, scale, n_tot, kps, ns, cb);
}

template <int KV, int GRP, int DPL>
void launch_decode(dim3 grid, hipStream_t st, const float *q, int64_t ldq, const SpanArgs &sp, const float *bias,
                   int64_t bhs, int bspan, float *out, float *part, int *cnt, int H, int G, float scale,
                   int64_t n_tot, int64_t kps, int ns, int64_t cb, int tiling) {
    switch (tiling) {
#define VGX_AT(T)                                                                                              \
    case T:                                                                                                    \
        launch_tiled<KV, GRP, DPL, kTilings[T].nw, kTilings[T].kb>(grid, st, q, ldq, sp, bias, bhs, bspan, out, \
                                                                   part, cnt, H, G, scale, n_tot, kps, ns, cb); \
        break;
        VGX_AT(0)
        VGX_AT(1)
#undef VGX_AT
    }
}

template <int KV, int GRP>
bool dispatch_dpl(int D, dim3 grid, hipStream_t st, const float *q, int64_t ldq, const SpanArgs &sp,
                  const float *bias, int64_t bhs, int bspan, float *out, float *part, int *cnt, int H, int G,
                  float scale, int64_t n_tot, int64_t kps, int ns, int64_t cb, int tiling) {
    switch (D) {
        case 64: launch_decode<KV, GRP, 4>(grid, st, q, ldq, sp, bias, bhs, bspan, out, part, cnt, H, G, scale, n_tot, kps, ns, cb, tiling); return true;
        case 128: launch_decode<KV, GRP, 8>(grid, st, q, ldq, sp, bias, bhs, bspan, out, part, cnt, H, G, scale, n_tot, kps, ns, cb, tiling); return true;
    }
    return false;
}

template <int KV>
bool dispatch_grp(int grp, int D, dim3 grid, hipStream_t st, const float *q, int64_t ldq, const SpanArgs &sp,
                  const float *bias, int64_t bhs, int bspan, float *out, float *part, int *cnt, int H, int G,
                  float scale, int64_t n_tot, int64_t kps, int ns, int64_t cb, int tiling) {
    switch (grp) {
        case 1: return dispatch_dpl<KV, 1>(D, grid, st, q, ldq, sp, bias, bhs, bspan, out, part, cnt, H, G, scale, n_tot, kps, ns, cb, tiling);
        case 2: return dispatch_dpl<KV, 2>(D, grid, st, q, ldq, sp, bias, bhs, bspan, out, part, cnt, H, G, scale, n_tot, kps, ns, cb, tiling);
        case 4: return dispatch_dpl<KV, 4>(D, grid, st, q, ldq, sp, bias, bhs, bspan, out, part, cnt, H, G, scale, n_tot, kps, ns, cb, tiling);
        case 6: return dispatch_dpl<KV, 6>(D, grid, st, q, ldq, sp, bias, bhs, bspan, out, part, cnt, H, G, scale, n_tot, kps, ns, cb, tiling);
        case 8: return dispatch_dpl<KV, 8>(D, grid, st, q, ldq, sp, bias, bhs, bspan, out, part, cnt, H, G, scale, n_tot, kps, ns, cb, tiling);
    }
    return false;
}

int attn_decode_impl(int kv_dtype, const float *q, int64_t ldq, const vgx_kv_span *spans, int n_spans,
                     const float *bias, int64_t bias_hstride, int bias_span, int64_t causal_base, float *out, int64_t B,
                     int64_t H, int64_t G, int64_t D, float scale, void *workspace, int64_t workspace_bytes,
                     void *stream);

// ---------------------------------------------------------------------------------------------
// Scratch of the allocation-free entry point: one fixed array per GPU (the split tickets, then the
// partials, as in a caller's workspace), never allocated at run time.  Host code uses only the
// per-device address that hipGetSymbolAddress returns for it (the array's name is a host-side
// stand-in, not a device address).  The address is looked up, and the ticket region cleared, once
// per device by the first call on that device, which must come outside any stream capture.
constexpr int64_t kScratchBytes = 2ll << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch[kMaxDevices] = {};

__global__ void zero_words_kernel(uint32_t *__restrict__ p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

int device_scratch(hipStream_t st, void **out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return VGX_E_HIP;
    if (dev >= kMaxDevices) return VGX_E_LIMIT;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch[dev]) {
        // the set-up launches a fill kernel, which a stream capture would record instead of running
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(st, &cs) != hipSuccess) return VGX_E_HIP;
        if (cs != hipStreamCaptureStatusNone) return VGX_E_STATE;
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return VGX_E_HIP;
        // the tickets must start at zero (every call leaves them so); a fill kernel, ordered before the
        // first use on the caller's stream
        hipLaunchKernelGGL(zero_words_kernel, dim3(16), dim3(256), 0, st, static_cast<uint32_t *>(p),
                           ticket_bytes(0, 0) / 4);
        if (hipGetLastError() != hipSuccess) return VGX_E_HIP;
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return VGX_OK;
}

}  // namespace

extern "C" {

int64_t vgx_attn_decode_workspace_bytes(int64_t B, int64_t H, int64_t G, int64_t D, int64_t n_keys) {
    if (B <= 0 || H <= 0 || G <= 0 || D <= 0 || n_keys <= 0 || H % G) return VGX_E_SIZE;
    int64_t kps = 0;
    int ns = 0;   // the most splits of any workgroup shape, so the caller's workspace fits every choice
    for (int t = 0; t < kNumTilings; ++t) ns = std::max(ns, choose_splits(B, G, n_keys, &kps, t));
    int64_t need = ns <= 1 ? 0 : ticket_bytes(B, G) + partial_bytes(B, H, D, ns);
    const int nb1 = b1_splits(B, G, D, n_keys);
    if (nb1 > 1) need = std::max(need, ticket_bytes(B, G) + b1_part_bytes(B * G, H / G, nb1));
    return need;
}

int vgx_attn_decode(int kv_dtype, const float *q, int64_t ldq, const vgx_kv_span *spans, int n_spans,
                    const float *bias, int64_t bias_hstride, int bias_span, int64_t causal_base, float *out, int64_t B,
                    int64_t H, int64_t G, int64_t D, float scale, void *workspace, int64_t workspace_bytes,
                    void *stream) {
    return attn_decode_impl(kv_dtype, q, ldq, spans, n_spans, bias, bias_hstride, bias_span, causal_base, out, B, H, G,
                            D, scale, workspace, workspace_bytes, stream);
}

int vgx_attn_decode_noalloc(int kv_dtype, const float *q, int64_t ldq, const vgx_kv_span *spans, int n_spans,
                            const float *bias, int64_t bias_hstride, int bias_span, int64_t causal_base, float *out,
                            int64_t B, int64_t H, int64_t G, int64_t D, float scale, void *stream) {
    if (!spans || n_spans < 1 || n_spans > 4) return spans ? VGX_E_LIMIT : VGX_E_ARG;
    if (B <= 0 || H <= 0 || G <= 0 || D <= 0 || H % G) return VGX_E_SIZE;
    int64_t n_keys = 0;
    for (int i = 0; i < n_spans; ++i) {
        if (spans[i].len < 0 || spans[i].len > 0x3FFFFFFF) return VGX_E_SIZE;
        n_keys += spans[i].len;
    }
    if (n_keys <= 0) return VGX_E_SIZE;
    const int64_t need = vgx_attn_decode_workspace_bytes(B, H, G, D, n_keys);
    if (need < 0) return (int)need;
    if (need > kScratchBytes) return VGX_E_LIMIT;   // beyond the fixed scratch: use vgx_attn_decode
    void *ws = nullptr;
    if (need > 0) {
        const int rc = device_scratch(static_cast<hipStream_t>(stream), &ws);
        if (rc != VGX_OK) return rc;
    }
    return attn_decode_impl(kv_dtype, q, ldq, spans, n_spans, bias, bias_hstride, bias_span, causal_base, out, B, H, G,
                            D, scale, ws, need > 0 ? kScratchBytes : 0, stream);
}

}  // extern "C"

namespace {

int attn_decode_impl(int kv_dtype, const float *q, int64_t ldq, const vgx_kv_span *spans, int n_spans,
                     const float *bias, int64_t bias_hstride, int bias_span, int64_t causal_base, float *out, int64_t B,
                     int64_t H, int64_t G, int64_t D, float scale, void *workspace, int64_t workspace_bytes,
                     void *stream) {
    if (kv_dtype != VGX_F32 && kv_dtype != VGX_BF16) return VGX_E_DTYPE;
    if (!q || !spans || !out) return VGX_E_ARG;
    if (n_spans < 1 || n_spans > 4) return VGX_E_LIMIT;
    if (B <= 0 || H <= 0 || G <= 0 || H % G) return VGX_E_SIZE;
    if (D != 64 && D != 128) return VGX_E_LIMIT;
    if (B > 65535 || G > 65535) return VGX_E_LIMIT;
    if (bias && (bias_span < 0 || bias_span >= n_spans)) return VGX_E_ARG;
    if (ldq < H * D) return VGX_E_SIZE;
    SpanArgs sp{};
    sp.n = n_spans;
    int64_t n_tot = 0;
    const int elem = kv_dtype == VGX_F32 ? 4 : 2;
    for (int s = 0; s < n_spans; ++s) {
        if (spans[s].len < 0) return VGX_E_SIZE;
        if (spans[s].len > 0x3FFFFFFF) return VGX_E_LIMIT;
        if (spans[s].len > 0 && (!spans[s].k || !spans[s].v)) return VGX_E_ARG;
        if (spans[s].len > 0 && (((uintptr_t)spans[s].k | (uintptr_t)spans[s].v) % 16)) return VGX_E_ALIGN;
        if (spans[s].len > 0 && ((spans[s].batch_stride * elem) % 16 || (spans[s].group_stride * elem) % 16)) return VGX_E_ALIGN;
        sp.k[s] = spans[s].k;
        sp.v[s] = spans[s].v;
        sp.len[s] = spans[s].len;
        sp.bstride[s] = spans[s].batch_stride;
        sp.gstride[s] = spans[s].group_stride;
        sp.dyn_len[s] = spans[s].dyn_len;
        n_tot += spans[s].len;
    }
    if (n_tot <= 0) return VGX_E_SIZE;
    if (n_tot > 0x3FFFFFFF) return VGX_E_LIMIT;
    const int grp = (int)(H / G);
    hipStream_t st = (hipStream_t)stream;
    // few (batch, group) pairs at D = 128: one split per workgroup, then the split merge
    const int nb1 = causal_base < 0 && grp <= 8 && ((uintptr_t)q & 15) == 0 && ldq % 4 == 0 &&
                            ((uintptr_t)out & 15) == 0
                        ? b1_splits(B, G, D, n_tot)
                        : 0;
    if (nb1 > 0) {
        float *part = nullptr;
        int *cnt = nullptr;
        const int64_t ml_off = b1_ml_off(B * G, grp, nb1);
        if (nb1 > 1) {
            if (!workspace || workspace_bytes < ticket_bytes(B, G) + b1_part_bytes(B * G, grp, nb1)) return VGX_E_ARENA;
            if ((uintptr_t)workspace % 256) return VGX_E_ALIGN;
            cnt = static_cast<int *>(workspace);
            part = reinterpret_cast<float *>(static_cast<char *>(workspace) + ticket_bytes(B, G));
        }
        const dim3 grid((unsigned)nb1, (unsigned)G, (unsigned)B);
#define VGX_B1(KVV, GRPV, ALV)                                                                                   \
    hipLaunchKernelGGL((attn_decode_b1_kernel<KVV, GRPV, kB1NW, kB1KB, kB1Ticket, ALV>), grid, dim3(64 * kB1NW), 0, st, q, \
                       ldq, sp, bias, bias_hstride, bias_span, out, part, ml_off, cnt, (int)H, (int)G, scale, n_tot, nb1)
#define VGX_B1A(KVV, ALV)                             \
    switch (grp) {                                    \
        case 1: VGX_B1(KVV, 1, ALV); break;           \
        case 2: VGX_B1(KVV, 2, ALV); break;           \
        case 3: VGX_B1(KVV, 3, ALV); break;           \
        case 4: VGX_B1(KVV, 4, ALV); break;           \
        case 5: VGX_B1(KVV, 5, ALV); break;           \
        case 6: VGX_B1(KVV, 6, ALV); break;           \
        case 7: VGX_B1(KVV, 7, ALV); break;           \
        default: VGX_B1(KVV, 8, ALV); break;          \
    }
#define VGX_B1G(KVV) do { if (aligned) { VGX_B1A(KVV, true) } else { VGX_B1A(KVV, false) } } while (0)
        bool aligned = true;    // every span's capacity a multiple of a wave's keys
        for (int i = 0; i < n_spans; ++i) aligned = aligned && spans[i].len % (4 * kB1KB) == 0;
        if (kv_dtype == VGX_F32) VGX_B1G(VGX_F32); else VGX_B1G(VGX_BF16);
#undef VGX_B1G
#undef VGX_B1A
#undef VGX_B1
        VGX_CHECK_LAUNCH();
        if (nb1 > 1 && !kB1Ticket) {
            hipLaunchKernelGGL(b1_merge_kernel, dim3((unsigned)(B * H), 4), dim3(64), 0, st, part, ml_off, out, (int)H,
                               (int)G, nb1);
            VGX_CHECK_LAUNCH();
        }
        return VGX_OK;
    }
    const bool mfma = kv_dtype == VGX_BF16 && D == 128 && causal_base < 0 &&
                      (grp == 1 || grp == 2 || grp == 4 || grp == 6 || grp == 8) &&
                      ((uintptr_t)q & 15) == 0 && ldq % 4 == 0;
    if (mfma) {
        int64_t kps = 0;
        const int ns = choose_splits_mfma(B, G, n_tot, &kps);   // never more splits than the VALU path
        float *part = nullptr;
        int *cnt = nullptr;
        if (ns > 1) {
            if (!workspace || workspace_bytes < ticket_bytes(B, G) + partial_bytes(B, H, D, ns)) return VGX_E_ARENA;
            if ((uintptr_t)workspace % 256) return VGX_E_ALIGN;
            if (use_tickets(B, G, ns)) cnt = static_cast<int *>(workspace);
            part = reinterpret_cast<float *>(static_cast<char *>(workspace) + ticket_bytes(B, G));
        }
        const dim3 grid((unsigned)ns, (unsigned)G, (unsigned)B);
#define VGX_AM(GRPV)                                                                                         \
    hipLaunchKernelGGL(attn_decode_mfma_kernel<GRPV>, grid, dim3(64 * kWaves), 0, st, q, ldq, sp, bias, bias_hstride, \
                       bias_span, out, part, cnt, (int)H, (int)G, scale, n_tot, kps, ns)
        switch (grp) {
            case 1: VGX_AM(1); break;
            case 2: VGX_AM(2); break;
            case 4: VGX_AM(4); break;
            case 6: VGX_AM(6); break;
            default: VGX_AM(8); break;
        }
#undef VGX_AM
        VGX_CHECK_LAUNCH();
        if (ns > 1 && cnt == nullptr) {
            hipLaunchKernelGGL(attn_merge_kernel, dim3((unsigned)(B * H)), dim3((unsigned)D), 0, st, part, out,
                               (int)H, (int)G, (int)D, ns);
            VGX_CHECK_LAUNCH();
        }
        return VGX_OK;
    }
    const int tiling = pick_tiling(B, G);
    int64_t kps = 0;
    const int ns = choose_splits(B, G, n_tot, &kps, tiling);
    float *part = nullptr;
    int *cnt = nullptr;
    if (ns > 1) {
        if (!workspace || workspace_bytes < ticket_bytes(B, G) + partial_bytes(B, H, D, ns)) return VGX_E_ARENA;
        if ((uintptr_t)workspace % 256) return VGX_E_ALIGN;
        if (use_tickets(B, G, ns)) cnt = static_cast<int *>(workspace);
        part = reinterpret_cast<float *>(static_cast<char *>(workspace) + ticket_bytes(B, G));
    }
    dim3 grid((unsigned)ns, (unsigned)G, (unsigned)B);
    bool ok = kv_dtype == VGX_F32
                  ? dispatch_grp<VGX_F32>(grp, (int)D, grid, st, q, ldq, sp, bias, bias_hstride, bias_span, out,
                                          part, cnt, (int)H, (int)G, scale, n_tot, kps, ns, causal_base, tiling)
                  : dispatch_grp<VGX_BF16>(grp, (int)D, grid, st, q, ldq, sp, bias, bias_hstride, bias_span, out,
                                           part, cnt, (int)H, (int)G, scale, n_tot, kps, ns, causal_base, tiling);
    if (!ok) return VGX_E_LIMIT;
    VGX_CHECK_LAUNCH();
    if (ns > 1 && cnt == nullptr) {
        hipLaunchKernelGGL(attn_merge_kernel, dim3((unsigned)(B * H)), dim3((unsigned)D), 0, st, part, out, (int)H,
                           (int)G, (int)D, ns);
        VGX_CHECK_LAUNCH();
    }
    return VGX_OK;
}

}  // namespace
