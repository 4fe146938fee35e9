// The streaming pass of the sampler (k_scan): one read of the logits.
//
// One workgroup of 256 threads per (tile, row); a tile is 8192 tokens held in
// registers (32 per thread) after coalesced 128-bit loads.  Per tile it writes:
//   maxc   (key << 32 | ~index) of the tile's largest penalised logit
//   sw     sum of token weights floor(cexp(y - m_t) * 2^40) over the tile
//          (rows that need the whole-row mass)
//   cand   the tile's top tokens as (key, index) composites, every token whose key
//          is >= bound; at least min(c, tile size) of them, at most kCap
//   nu     distinct penalised ids inside the tile (the penalty scatter width)
// Keys here are of the penalised logit x before temperature scaling: y = x / s is
// non-decreasing in x, so the order, the maxima and the top tokens carry over and
// the finish kernel converts the few values it needs.
#pragma once

#include "common.h"
#include "fie_sampler.h"

namespace fie {

constexpr int kScanThreads = 256;
constexpr int kEPT = kTile / kScanThreads;   // tokens per thread
constexpr int kCap = 128;                    // candidates per tile, at most
constexpr int kCandMin = 64;                 // candidates per tile, at least (if present)
constexpr int kMaxTiles = 64;                // vocab <= 64 * 8192

// Result of one row kept for fie_sampler_kept().
struct RowRes {
    uint64_t cut;        // last top-p survivor composite (0 = no top-p cut)
    uint64_t klo, khi;   // kept mass
    uint32_t tau;        // survivors have y-key >= tau (top-k / min-p), 0 = all
    uint32_t greedy;     // 1 for greedy rows
    int64_t token;
    float M;
    float s;
};

// Device pointers into the caller's workspace.
struct Ws {
    uint64_t* maxc;      // [rows * NT]
    uint64_t* sw;        // [rows * NT]
    uint32_t* bound;     // [rows * NT]
    uint32_t* ncand;     // [rows * NT]
    uint32_t* nu;        // [rows * NT]
    uint64_t* cand;      // [rows * NT * kCap]
    float* tok0x;        // [rows] token 0's logit (fp32, unpenalised)
    uint32_t* tok0c;     // [rows] occurrences of token 0 in the row's history
    uint32_t* bad;       // [rows] history ids >= vocab seen
    RowRes* res;         // [rows]
    float* mt;           // [rows * (NT + 1)] tile maxima of y, slot 0 = token 0
    uint64_t* ct;        // [rows * (NT + 1)] tile scales C_t
};

struct KParams {
    fie_sampler_args a;
    Ws w;
    int NT;
};

// ---------------------------------------------------------------- element access
template <int DT> struct DTy;
template <> struct DTy<FIE_F32> { static constexpr int EPL = 4, SZ = 4; };
template <> struct DTy<FIE_F16> { static constexpr int EPL = 8, SZ = 2; };
template <> struct DTy<FIE_BF16> { static constexpr int EPL = 8, SZ = 2; };

// Element e of a 16-byte load, as fp32 (exact for every input dtype).
template <int DT>
FIE_DEV float lane_get(const uint4& r, int e)
{
    const uint32_t* w = &r.x;
    if constexpr (DT == FIE_F32) {
        return __uint_as_float(w[e]);
    } else if constexpr (DT == FIE_F16) {
        uint32_t v = w[e >> 1];
        uint16_t h = (e & 1) ? (uint16_t)(v >> 16) : (uint16_t)(v & 0xFFFFu);
        return (float)__builtin_bit_cast(_Float16, h);
    } else {
        uint32_t v = w[e >> 1];
        return __uint_as_float((e & 1) ? (v & 0xFFFF0000u) : (v << 16));
    }
}

// One 16-byte group of tokens [e0, e0 + EPL) of a row; tokens at or past V read 0.
template <int DT, bool VEC>
FIE_DEV uint4 load_group(const char* rowp, int e0, int V)
{
    constexpr int EPL = DTy<DT>::EPL, SZ = DTy<DT>::SZ;
    if (VEC && e0 + EPL <= V) return *(const uint4*)(rowp + (size_t)e0 * SZ);
    uint4 r = make_uint4(0, 0, 0, 0);
    uint32_t* w = &r.x;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
        if (e0 + e < V) {
            if constexpr (SZ == 4) {
                w[e] = ((const uint32_t*)rowp)[e0 + e];
            } else {
                uint32_t h = ((const uint16_t*)rowp)[e0 + e];
                w[e >> 1] |= h << ((e & 1) * 16);
            }
        }
    }
    return r;
}

// sampler.py:169-173, one element: transformers' repetition convention, then the
// presence and frequency terms, each one fp32 operation.
FIE_DEV float penalize(float g, float rep, float pres, float freq, uint32_t count)
{
    float pen = (g > 0.0f) ? g / rep : g * rep;
    pen = pen - pres;
    pen = pen - freq * (float)count;
    return pen;
}

// Scaled logit from a key of the unscaled one (s = 1 skips the divide).
FIE_DEV float y_of_xkey(uint32_t k, float s)
{
    float x = key_to_float(k);
    return s == 1.0f ? x : scaled(x, s);
}

// Candidates per tile a row asks for: enough that the union over tiles holds the
// row's top-k when the top tokens spread about evenly.
FIE_DEV uint32_t cand_target(int topk, int NT)
{
    int c = kCandMin;
    if (topk > 0) {
        int need = 2 * ((topk + NT - 1) / NT) + 16;
        c = need > c ? need : c;
    }
    return (uint32_t)(c < kCap ? c : kCap);
}

// Descending selection over an LDS count histogram of NB bins (bin NB-1 = largest
// keys): the bin holding the target-th largest element, the count above it and its
// own count.  bin = -1 when fewer than `target` elements were counted.
struct Pick {
    int bin;
    uint32_t above;
    uint32_t inbin;
};

template <int NB, int NT>
FIE_DEV Pick pick_desc(const uint32_t* h, uint32_t target, uint32_t* scratch, Pick* out)
{
    constexpr int PER = NB / NT;
    static_assert(PER >= 1 && NB % NT == 0, "bins per thread");
    const int t = threadIdx.x;
    uint32_t loc[PER];
    uint32_t sum = 0;
#pragma unroll
    for (int q = 0; q < PER; ++q) {
        loc[q] = h[NB - 1 - (t * PER + q)];
        sum += loc[q];
    }
    uint32_t total;
    uint32_t before = block_excl_scan_u32<NT>(sum, scratch, &total);
    if (before < target && target <= before + sum) {
        uint32_t run = before;
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            if (run < target && run + loc[q] >= target) {
                out->bin = NB - 1 - (t * PER + q);
                out->above = run;
                out->inbin = loc[q];
            }
            run += loc[q];
        }
    }
    if (t == 0 && total < target) {
        out->bin = -1;
        out->above = total;
        out->inbin = 0;
    }
    __syncthreads();
    Pick p = *out;
    __syncthreads();
    return p;
}

// ---------------------------------------------------------------- k_scan
template <int DT, bool VEC, bool LONGH>
__global__ __launch_bounds__(kScanThreads) void k_scan(const KParams P)
{
    constexpr int EPL = DTy<DT>::EPL, SZ = DTy<DT>::SZ, NL = kEPT / EPL;
    // Penalty counts of the tile's tokens: u16 halves (u32 words for long histories).
    constexpr int CW = LONGH ? kTile : kTile / 2;
    __shared__ uint32_t cnt[CW];
    __shared__ uint32_t hist[2048];
    __shared__ uint32_t scr[32];
    __shared__ Pick pick;
    __shared__ uint32_t zc, badc, nc;

    const fie_sampler_args& a = P.a;
    const int tile = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    const int NT = P.NT, V = a.vocab;
    const int lo = tile * kTile;
    const int hi = min(lo + kTile, V);
    const size_t slot = (size_t)row * NT + tile;
    const int32_t fl = a.flags[row];
    const bool greedy = fl & FIE_FLAG_GREEDY;
    const int lp = a.logprobs ? a.logprobs[row] : -1;
    const bool pen = a.apply_penalties && (fl & FIE_FLAG_PENALTY);
    const int topk = greedy ? 0 : a.top_k[row];
    const bool need_mass = lp >= 0 || (!greedy && topk == 0);
    const bool need_cand = !greedy || lp > 0;
    const float s = a.scale[row];
    const char* rowp = (const char*)a.logits + (size_t)row * (size_t)a.row_stride * SZ;

    // 1. Issue every load of the tile before anything else.
    uint4 raw[NL];
#pragma unroll
    for (int j = 0; j < NL; ++j) raw[j] = load_group<DT, VEC>(rowp, lo + (j * kScanThreads + tid) * EPL, V);

    // 2. Penalty counts of the tile's ids while the loads are in flight.
    float rep = 1.0f, pres = 0.0f, freq = 0.0f;
    if (pen) {
        rep = a.repetition[row];
        pres = a.presence[row];
        freq = a.frequency[row];
        for (int i = tid; i < CW; i += kScanThreads) cnt[i] = 0;
        if (tid == 0) { zc = 0; badc = 0; }
        __syncthreads();
        const int64_t h0 = a.hist_offsets[row], h1 = a.hist_offsets[row + 1];
        for (int64_t h = h0 + tid; h < h1; h += kScanThreads) {
            const uint32_t id = (uint32_t)a.hist_ids[h];
            if (id >= (uint32_t)lo && id < (uint32_t)hi) {
                const uint32_t o = id - lo;
                if (id == 0) atomicAdd(&zc, 1u);
                else if (LONGH) atomicAdd(&cnt[o], 1u);
                else atomicAdd(&cnt[o >> 1], 1u << ((o & 1) * 16));
            } else if (id >= (uint32_t)V && tile == NT - 1) {
                atomicAdd(&badc, 1u);
            }
        }
        __syncthreads();
        uint32_t u = 0;
        for (int i = tid; i < CW; i += kScanThreads) {
            const uint32_t wv = cnt[i];
            if (LONGH) u += wv != 0;
            else u += ((wv & 0xFFFFu) != 0) + ((wv >> 16) != 0);
        }
        u = block_sum_u32<kScanThreads>(u, scr);
        if (tid == 0) {
            P.w.nu[slot] = u;
            if (tile == 0) P.w.tok0c[row] = zc;
            if (tile == NT - 1) P.w.bad[row] = badc;
        }
    } else if (tid == 0) {
        P.w.nu[slot] = 0;
        if (tile == 0) P.w.tok0c[row] = 0;
        if (tile == NT - 1) P.w.bad[row] = 0;
    }

    // 3. Penalised values and their order keys; token 0 and tokens past V get key 0
    //    (token 0 is a tile of its own, settled by the finish kernel).
    uint32_t key[kEPT];
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        const int e0 = lo + (j * kScanThreads + tid) * EPL;
        uint32_t c[EPL];
        if (pen) {
            const int o = e0 - lo;
            if (LONGH) {
#pragma unroll
                for (int e = 0; e < EPL; ++e) c[e] = (o + e < kTile) ? cnt[o + e] : 0u;
            } else if constexpr (EPL == 8) {
                const uint4 q = *(const uint4*)&cnt[o >> 1];
                const uint32_t qq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) c[e] = (qq[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu;
            } else {
                const uint2 q = *(const uint2*)&cnt[o >> 1];
                const uint32_t qq[2] = {q.x, q.y};
#pragma unroll
                for (int e = 0; e < 4; ++e) c[e] = (qq[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu;
            }
        }
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const int idx = e0 + e;
            float x = lane_get<DT>(raw[j], e);
            if (idx == 0) P.w.tok0x[row] = x;
            if (pen && c[e]) x = penalize(x, rep, pres, freq, c[e]);
            key[j * EPL + e] = (idx < V && idx != 0) ? fkey(x + 0.0f) : 0u;
        }
    }

    // 4. Tile maximum and its first index.
    uint32_t tm = 0;
#pragma unroll
    for (int i = 0; i < kEPT; ++i) tm = key[i] > tm ? key[i] : tm;
    const uint32_t km = block_max_u32<kScanThreads>(tm, scr);
    uint32_t fi = 0xFFFFFFFFu;
#pragma unroll
    for (int i = 0; i < kEPT; ++i) {
        const uint32_t idx = (uint32_t)(lo + ((i / EPL) * kScanThreads + tid) * EPL + (i % EPL));
        if (km != 0 && key[i] == km && idx < fi) fi = idx;
    }
    fi = block_min_u32<kScanThreads>(fi, scr);
    if (tid == 0) P.w.maxc[slot] = km ? comp_key(km, fi) : 0ull;

    // 5. Tile mass relative to the tile maximum (rule R1).
    if (need_mass) {
        uint64_t sum = 0;
        if (km != 0) {
            const float m = y_of_xkey(km, s);
#pragma unroll
            for (int i = 0; i < kEPT; ++i)
                if (key[i]) sum += tok_weight(y_of_xkey(key[i], s), m);
        }
        sum = block_sum_u64<kScanThreads>(sum, (uint64_t*)scr);
        if (tid == 0) P.w.sw[slot] = sum;
    }

    // 6. The tile's top tokens.  A floor first: the bin of the c-th largest
    //    per-thread maximum, so at least c tokens lie above it and the histogram
    //    sees only about c tokens instead of the whole tile.
    if (need_cand) {
        const uint32_t c = cand_target(topk, NT);
        for (int i = tid; i < 2048; i += kScanThreads) hist[i] = 0;
        if (tid == 0) nc = 0;
        __syncthreads();
        if (tm) atomicAdd(&hist[tm >> 21], 1u);
        __syncthreads();
        const Pick p0 = pick_desc<2048, kScanThreads>(hist, c, scr, &pick);
        const uint32_t floor_key = p0.bin < 0 ? 1u : ((uint32_t)p0.bin << 21);
        for (int i = tid; i < 2048; i += kScanThreads) hist[i] = 0;
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kEPT; ++i)
            if (key[i] >= floor_key && key[i]) atomicAdd(&hist[key[i] >> 21], 1u);
        __syncthreads();
        const Pick p1 = pick_desc<2048, kScanThreads>(hist, c, scr, &pick);
        uint32_t bound;
        if (p1.bin < 0) {
            bound = 1u;                                       // every token of the tile
        } else if (p1.above + p1.inbin <= (uint32_t)kCap) {
            bound = (uint32_t)p1.bin << 21;
        } else {
            for (int i = tid; i < 2048; i += kScanThreads) hist[i] = 0;
            __syncthreads();
#pragma unroll
            for (int i = 0; i < kEPT; ++i)
                if ((key[i] >> 21) == (uint32_t)p1.bin) atomicAdd(&hist[(key[i] >> 10) & 0x7FFu], 1u);
            __syncthreads();
            const Pick p2 = pick_desc<2048, kScanThreads>(hist, c - p1.above, scr, &pick);
            const uint32_t above2 = p1.above + p2.above;
            const uint32_t pre2 = ((uint32_t)p1.bin << 11) | (uint32_t)p2.bin;
            if (above2 + p2.inbin <= (uint32_t)kCap) {
                bound = pre2 << 10;
            } else {
                for (int i = tid; i < 1024; i += kScanThreads) hist[i] = 0;
                __syncthreads();
#pragma unroll
                for (int i = 0; i < kEPT; ++i)
                    if ((key[i] >> 10) == pre2) atomicAdd(&hist[key[i] & 0x3FFu], 1u);
                __syncthreads();
                const Pick p3 = pick_desc<1024, kScanThreads>(hist, c - above2, scr, &pick);
                const uint32_t K = (pre2 << 10) | (uint32_t)p3.bin;
                bound = (above2 + p3.above + p3.inbin <= (uint32_t)kCap) ? K : K + 1u;
            }
        }
        uint64_t* out = P.w.cand + slot * kCap;
#pragma unroll
        for (int i = 0; i < kEPT; ++i) {
            if (key[i] && key[i] >= bound) {
                const uint32_t idx = (uint32_t)(lo + ((i / EPL) * kScanThreads + tid) * EPL + (i % EPL));
                const uint32_t at = atomicAdd(&nc, 1u);
                out[at] = comp_key(key[i], idx);
            }
        }
        __syncthreads();
        if (tid == 0) {
            P.w.ncand[slot] = nc;
            P.w.bound[slot] = bound;
        }
    }
}

}  // namespace fie
