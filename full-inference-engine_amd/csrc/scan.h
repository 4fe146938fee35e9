// The streaming pass of the sampler (k_scan): one read of the logits.
//
// A tile is 2048 tokens, handled by one wave64 (32 tokens per lane, coalesced
// 128-bit loads); a workgroup is four waves on four consecutive tiles of a row,
// which share only the penalty-history count of their 8192-token span.  Per tile it
// writes:
//   maxc   (key << 32 | ~index) of the tile's largest penalised logit
//   sw     sum of token weights floor(cexp(y - m_t) * 2^40) over the tile
//          (rows that need the whole-row mass)
//   cand   the tile's top tokens as (key, index) composites: every token whose key
//          is >= bound, at least min(c, tile size) of them, at most kCapW
//   nu     distinct penalised ids inside the tile (the penalty scatter width)
// Keys here are of the penalised logit x before temperature scaling: y = x / s is
// non-decreasing in x, so the order, the maxima and the top tokens carry over and
// the finish kernel converts the few values it needs.  Within a tile everything is
// wave-local (DPP reductions, ballots); there is no barrier on rows without
// penalties.
#pragma once

#include "common.h"
#include "fie_sampler.h"

namespace fie {

constexpr int kScanThreads = 256;                // four waves, four tiles
constexpr int kWavesPerWG = kScanThreads / 64;
constexpr int kSpan = kTile * kWavesPerWG;       // tokens per workgroup (8192)
constexpr int kEPT = kTile / 64;                 // tokens per lane (32)
constexpr int kCapW = 64;                        // candidates per tile, at most
constexpr int kStageW = 256;                     // tokens at or above a tile's floor, staged
constexpr int kCandMin = 16;                     // candidates per tile of greedy rows
constexpr int kCandWide = kStageW / 8;           // ... of sampled rows without top-k (8 tokens a group)
constexpr int kCandRow = 4000;                   // ... times the tiles of a row, at most
constexpr int kMaxTiles = 256;                   // vocab <= 256 * 2048
constexpr int kBucketCap = 512;                  // history ids of one span held by k_prep
constexpr int kMaxSpans = kMaxTiles / kWavesPerWG;
constexpr int kPrepThreads = 256;
constexpr int kPS = 4;
constexpr int kHelpRows = 16;                    // batches up to this many rows get span helpers
constexpr int kHBins = 1024;                     // d-bins of a helper's histogram
constexpr int kHOffs = kHBins + 4;               // bin offsets per helper (kHBins + 1, padded)                           // penalised tokens per lane held in slots

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

// A row k_finish hands to k_deep: what the full-row passes need beyond what k_deep
// recomputes from the partials (mode kDeferDraw), or that the candidates settled
// the draw and only the top-L logprobs need a pass over the row (kDeferLogprobs).
constexpr uint32_t kDeferDraw = 1, kDeferLogprobs = 2;
struct DeferRec {
    uint64_t tok_comp, cut, tlo, thi;
    int64_t token;
    uint32_t tau, mode;
};

// Device pointers into the caller's workspace.
struct Ws {
    uint64_t* maxc;      // [rows * NT]
    uint64_t* sw;        // [rows * NT]
    uint32_t* bound;     // [rows * NT]
    uint32_t* ncand;     // [rows * NT]
    uint32_t* nu;        // [rows * NT]
    uint32_t* nb;        // [rows * NS] history ids (other than 0) falling in each span
    uint16_t* bk;        // [rows * NS * kBucketCap] their offsets in the span (first kBucketCap)
    uint64_t* cand;      // [rows * NT * kCapW]
    float* tok0x;        // [rows] token 0's logit (fp32, unpenalised)
    uint32_t* tok0c;     // [rows] occurrences of token 0 in the row's history
    uint32_t* bad;       // [rows] history ids >= vocab seen
    RowRes* res;         // [rows]
    float* mt;           // [rows * (NT + 1)] tile maxima of y, slot 0 = token 0
    uint64_t* ct;        // [rows * (NT + 1)] tile scales C_t
    uint32_t* dq;        // [2] rows queued for k_deep, and taken; k_scan clears both
    uint32_t* dqrows;    // [rows] the queued rows
    DeferRec* dfr;       // [rows]
    // Span helpers of k_finish (batches of at most kHelpRows rows; NULL otherwise),
    // per (row, span): the span's d-bin histogram (counts and the two 41-bit mass
    // limbs), the bins' offsets and the span's composites in bin order, and the
    // row-maximum key the helper binned against.
    uint32_t* harr;      // [rows] arrivals at a row (helpers and its finishing workgroup)
    uint32_t* hmk;       // [rows * NS]
    uint32_t* hpc;       // [rows * NS * kHBins]
    uint64_t* hlo;       // [rows * NS * kHBins]
    uint64_t* hhi;       // [rows * NS * kHBins]
    uint32_t* hoff;      // [rows * NS * kHOffs]
    uint64_t* hcomp;     // [rows * NS * kSpan]
};

struct KParams {
    fie_sampler_args a;
    Ws w;
    int NT;
    int NS;              // spans of kSpan tokens per row
    int helpers;         // 1: k_finish runs one helper workgroup per span of each sampled row
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

// End of row `row`'s history in hist_ids: explicit ends (a device-resident history,
// rows anywhere in one array) or the next CSR offset.
FIE_DEV int64_t hist_end(const fie_sampler_args& a, int row)
{
    return a.hist_ends ? a.hist_ends[row] : a.hist_offsets[row + 1];
}

// Token idx of a row, as fp32.
template <int DT>
FIE_DEV float load_elem(const char* rowp, uint32_t idx)
{
    if constexpr (DT == FIE_F32) {
        return ((const float*)rowp)[idx];
    } else {
        const uint32_t h = ((const uint16_t*)rowp)[idx];
        return lane_get<DT>(make_uint4(h, 0, 0, 0), 0);
    }
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
// row's top-k when the top tokens spread about evenly, at least kCandMin.
FIE_DEV uint32_t cand_target(int topk, int NT, bool greedy)
{
    int c = kCandMin;                              // greedy rows: their top logprobs
    if (topk > 0) {
        // a tile's share of the row's top k is about Poisson(lambda = k / tiles):
        // lambda + 4 sqrt(lambda) + 4 leaves a tile holding more of them than its
        // candidates (the row then takes the full-row path) below 1e-5 per tile
        const float lam = (float)topk / (float)NT;
        c = (int)__builtin_ceilf(lam + 4.0f * __builtin_sqrtf(lam)) + 4;
    } else if (!greedy) {
        // a top-p cut, min-p or a plain draw: as deep as the finish kernel can sort
        // (penalties on the chosen tokens flatten a row step after step)
        c = kCandWide;
        if (c * NT > kCandRow) c = kCandRow / NT;
    }
    return (uint32_t)(c < 8 ? 8 : (c < kCapW ? c : kCapW));
}

// Token index of lane element i of the wave's tile (group i / EPL is one 16-byte
// load; groups are 64 * EPL tokens apart).
template <int EPL>
FIE_DEV int elem_index(int lo, int lane, int i) { return lo + ((i / EPL) * 64 + lane) * EPL + (i % EPL); }

// (m & a) | (~m & b) in one instruction, opaque to the optimizer (a select tree
// written in plain C++ is folded back into a runtime-indexed array in memory).
FIE_DEV uint32_t bit_select(uint32_t m, uint32_t a, uint32_t b)
{
    uint32_t r;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(m), "v"(a), "v"(b));
    return r;
}

// x[i] for a lane-varying i < 32 as a five-level select tree: five lane masks and
// 31 bitfield selects, where a plain runtime index into registers becomes a
// 31-step compare and select chain.
FIE_DEV float pick32(const float (&x)[32], uint32_t i)
{
    uint32_t v[16];
    const uint32_t m0 = 0u - (i & 1u);
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = bit_select(m0, __float_as_uint(x[2 * k + 1]), __float_as_uint(x[2 * k]));
#pragma unroll
    for (int lvl = 1; lvl < 5; ++lvl) {
        const uint32_t m = 0u - ((i >> lvl) & 1u);
#pragma unroll
        for (int k = 0; k < (16 >> lvl); ++k) v[k] = bit_select(m, v[2 * k + 1], v[2 * k]);
    }
    return __uint_as_float(v[0]);
}

// Largest t (refining `pre` over bits hi..lo) with at least `target` of the keys
// k[0..N) of the wave's lanes at or above t: a radix select by ballot counts.
template <int N>
FIE_DEV uint32_t ballot_select(const uint32_t (&k)[N], uint32_t target, uint32_t pre, int hi, int lo)
{
    for (int b = hi; b >= lo; --b) {
        const uint32_t t = pre | (1u << b);
        uint32_t cnt = 0;
#pragma unroll
        for (int g = 0; g < N; ++g) cnt += popc64(__ballot(k[g] >= t));
        if (cnt >= target) pre = t;
    }
    return pre;
}

// LDS of k_scan.
template <bool LONGH>
struct ScanSmem {
    // penalty counts of the span's tokens: u16 halves (u32 words for long histories)
    uint32_t cnt[LONGH ? kSpan : kSpan / 2];
    uint32_t pbits[kSpan / 32];        // penalised tokens of the span, one bit each
    uint64_t stage[kWavesPerWG][kStageW];
    uint32_t uniq[kWavesPerWG];
};

// Per-row settings the tile pass reads (sampler.py:182 leaves greedy rows unscaled).
struct RowCfg {
    bool greedy, pen, need_mass, need_cand;
    int lp, topk;
    float s, rep, pres, freq;
};

FIE_DEV RowCfg row_cfg(const fie_sampler_args& a, int row)
{
    RowCfg c;
    const int32_t fl = a.flags[row];
    c.greedy = fl & FIE_FLAG_GREEDY;
    c.lp = a.logprobs ? a.logprobs[row] : -1;
    c.pen = a.apply_penalties && (fl & FIE_FLAG_PENALTY);
    c.topk = c.greedy ? 0 : a.top_k[row];
    c.need_mass = c.lp >= 0 || (!c.greedy && c.topk == 0);
    c.need_cand = !c.greedy || c.lp > 0;
    c.s = c.greedy ? 1.0f : a.scale[row];
    c.rep = 1.0f;
    c.pres = 0.0f;
    c.freq = 0.0f;
    if (c.pen) {
        c.rep = a.repetition[row];
        c.pres = a.presence[row];
        c.freq = a.frequency[row];
    }
    return c;
}

// One wave's pass over one 2048-token tile of one row, its tokens already in
// registers (raw, the lane layout of load_group): penalties, the tile maximum,
// the tile mass and the candidates, written to the tile's partials.  `rowp` is
// the row's token 0 for the re-read of penalised tokens (global memory, or a
// producer's staging copy); pbits/cnt hold the penalty marks and counts of tokens
// pbase.. (u16 halves, u32 words when LONGH); `stage` is kStageW words of the
// wave's own LDS.
template <int DT, bool LONGH>
FIE_DEV void scan_tile(const KParams& P, const RowCfg& rc, int row, int tile,
                       uint4 (&raw)[kEPT / DTy<DT>::EPL], const char* rowp,
                       const uint32_t* pbits, const uint32_t* cnt, int pbase, uint64_t* stage)
{
    constexpr int EPL = DTy<DT>::EPL, NL = kEPT / EPL;
    const fie_sampler_args& a = P.a;
    const int lane = threadIdx.x & 63;
    const int NT = P.NT, V = a.vocab;
    const int lo = tile * kTile;
    const size_t slot = (size_t)row * NT + tile;
    const bool greedy = rc.greedy, pen = rc.pen, need_mass = rc.need_mass, need_cand = rc.need_cand;
    const int topk = rc.topk;
    const float s = rc.s, rep = rc.rep, pres = rc.pres, freq = rc.freq;

    // 3. The penalised logits (sampler.py:169-175).  Registers are indexed only
    //    statically (a runtime index into x[] turns into a select per element):
    //    the lane's penalised tokens read NaN in x[] and are re-read from memory
    //    (the lines were just fetched) into up to kPS slots, penalised there, and
    //    join the maximum, the mass and the staging as extra elements.  A wave
    //    with a lane holding more than kPS penalised tokens patches x[] in place.
    float x[kEPT];
#pragma unroll
    for (int j = 0; j < NL; ++j) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) x[j * EPL + e] = lane_get<DT>(raw[j], e);
    }
    float pv[kPS];           // penalised values of the slots (NaN = empty)
    uint32_t pidx[kPS];      // their token indices
#pragma unroll
    for (int q = 0; q < kPS; ++q) { pv[q] = __builtin_nanf(""); pidx[q] = 0xFFFFFFFFu; }
    bool odd = false;        // a patched value outside the unchecked divide's range
    if (pen) {
        uint32_t mine = 0;   // bit i: the lane's token i is penalised
#pragma unroll
        for (int j = 0; j < NL; ++j) {
            const int o = lo - pbase + (j * 64 + lane) * EPL;
            mine |= ((pbits[o >> 5] >> (o & 31)) & ((1u << EPL) - 1)) << (j * EPL);
        }
        auto count_of = [&](int o) -> uint32_t {
            return LONGH ? cnt[o] : ((cnt[o >> 1] >> ((o & 1) * 16)) & 0xFFFFu);
        };
        if (__ballot(__builtin_popcount(mine) > kPS) != 0) {
            for (uint32_t b = mine; b; b &= b - 1) {
                const int i = __builtin_ctz(b);
                const int o = lo - pbase + ((i / EPL) * 64 + lane) * EPL + (i % EPL);
                x[i] = penalize(x[i], rep, pres, freq, count_of(o));
                // a finite, nonzero value outside Markstein's range (extreme penalty
                // parameters) sends the wave's fp16 mass loop to the checked divide
                if (!(markstein_ok(x[i]) || x[i] == 0.0f || !__builtin_isfinite(x[i]))) odd = true;
            }
        } else if (__ballot(mine != 0) != 0) {
            // a set bit ORs a quiet NaN's exponent and quiet bit into the value
#pragma unroll
            for (int i = 0; i < kEPT; ++i)
                x[i] = __int_as_float(__float_as_int(x[i]) |
                                      (__builtin_amdgcn_sbfe((int)mine, (unsigned)i, 1u) & 0x7FC00000));
            uint32_t b = mine;
#pragma unroll
            for (int q = 0; q < kPS; ++q) {
                if (b) {
                    pidx[q] = (uint32_t)elem_index<EPL>(lo, lane, __builtin_ctz(b));
                    b &= b - 1;
                }
            }
#pragma unroll
            for (int q = 0; q < kPS; ++q)
                if (pidx[q] != 0xFFFFFFFFu) pv[q] = load_elem<DT>(rowp, pidx[q]);
#pragma unroll
            for (int q = 0; q < kPS; ++q)
                if (pidx[q] != 0xFFFFFFFFu) pv[q] = penalize(pv[q], rep, pres, freq, count_of((int)pidx[q] - pbase));
        }
    }
    // Tokens outside the tile read NaN from here on: token 0 (a tile of its own,
    // settled by the finish kernel) and tokens past the end of the row.  Every
    // step below ignores NaN: fmax skips it, it equals nothing, cexp(NaN) is 0 and
    // the staging test rejects it (NaN logits are outside the sampler's contract).
    if (tile == 0 && lane == 0) {
        P.w.tok0x[row] = lane_get<DT>(raw[0], 0);
        x[0] = __builtin_nanf("");
    }
    if (lo + kTile > V) {
#pragma unroll
        for (int i = 0; i < kEPT; ++i)
            if (elem_index<EPL>(lo, lane, i) >= V) x[i] = __builtin_nanf("");
    }

    // 4. Group and lane maxima (float max: -0 and +0 compare equal, as their folded
    //    keys do), the tile maximum's key, its first index.
    constexpr int NG = NL;
    float gm[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        float v = x[g * EPL];
#pragma unroll
        for (int e = 1; e < EPL; ++e) v = __builtin_fmaxf(v, x[g * EPL + e]);
        gm[g] = v;
    }
    float m = gm[0];
#pragma unroll
    for (int g = 1; g < NG; ++g) m = __builtin_fmaxf(m, gm[g]);
    const float mx = m;      // the lane's maximum over its own tokens (slots aside)
#pragma unroll
    for (int q = 0; q < kPS; ++q) m = __builtin_fmaxf(m, pv[q]);
    const uint32_t lkey = m == m ? fkey(m + 0.0f) : 0u;
    const uint32_t km = dwave_max_u32(lkey);
    uint32_t first = 0xFFFFFFFFu;
    if (km != 0 && lkey == km) {
        // groups lie in index order; the first group holding m, then its first token
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            if (first == 0xFFFFFFFFu && gm[g] == m) {
#pragma unroll
                for (int e = EPL - 1; e >= 0; --e)
                    if (x[g * EPL + e] == m) first = (uint32_t)elem_index<EPL>(lo, lane, g * EPL + e);
            }
        }
#pragma unroll
        for (int q = 0; q < kPS; ++q)
            if (pv[q] == m && pidx[q] < first) first = pidx[q];
    }
    const uint32_t fi = dwave_min_u32(first);
    if (lane == 0) P.w.maxc[slot] = km ? comp_key(km, fi) : 0ull;

    // 5. Tile mass relative to the tile maximum (rule R1): the integer weights
    //    floor(cexp(y - m_t) 2^40) < 2^41 as integer-valued floats, summed in fp64,
    //    which is exact (a lane's 32 weights stay below 2^46).  y - m_t needs no
    //    folding of -0: both zeros give the same difference.  The temperature
    //    divide is Markstein's corrected product, equal to the IEEE quotient while
    //    2^-96 <= |x| <= 2^96 and 2^-30 <= s <= 2^30: always so for finite,
    //    nonzero fp16 logits; 0 gives 0; +-inf and NaN give NaN there and weight 0
    //    through cexp's clamp, as the IEEE quotient's weight does.  Only penalised
    //    values can leave the range, and the patch step flags them.
    if (need_mass) {
        double acc = 0.0;
        if (km != 0) {
            const float mt = y_of_xkey(km, s);
            if (s == 1.0f) {
#pragma unroll
                for (int i = 0; i < kEPT; ++i) acc += (double)weight40(x[i] - mt);
            } else if (s >= 0x1p-30f && s <= 0x1p30f) {
                const float rs = 1.0f / s;
                if (DT == FIE_F16 && __ballot(odd) == 0) {
#pragma unroll
                    for (int i = 0; i < kEPT; ++i) acc += (double)weight40(div_markstein(x[i], s, rs) - mt);
                } else {
#pragma unroll
                    for (int i = 0; i < kEPT; ++i) {
                        const float y = markstein_ok(x[i]) ? div_markstein(x[i], s, rs) : x[i] / s;
                        acc += (double)weight40(y - mt);
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < kEPT; ++i) acc += (double)weight40(scaled(x[i], s) - mt);
            }
        }
        if (km != 0) {
            const float mt = y_of_xkey(km, s);
#pragma unroll
            for (int q = 0; q < kPS; ++q)
                if (__ballot(pidx[q] != 0xFFFFFFFFu) != 0)
                    acc += (double)weight40((s == 1.0f ? pv[q] : scaled(pv[q], s)) - mt);
        }
        const uint64_t tot = dwave_sum_u64((uint64_t)acc);
        if (lane == 0) P.w.sw[slot] = tot;
    }

    // 6. The tile's top tokens.  The floor is the largest 20-bit key prefix with at
    //    least c lane or group maxima at or above it, so at least c tokens are; tokens
    //    at or above it are staged in LDS, and when more than kCapW are, the c-th
    //    largest staged key is found by a full-width ballot select.
    if (need_cand) {
        // a partial last tile asks for at most half its groups: every group at or
        // above the floor may stage all its EPL tokens
        uint32_t c = cand_target(topk, NT, greedy);
        const int valid = V - lo < kTile ? V - lo : kTile;
        const uint32_t half = (uint32_t)((valid + EPL - 1) / EPL / 2);
        if (c > half) c = half > 8u ? half : 8u;
        c = __builtin_amdgcn_readfirstlane(c);               // uniform in the wave
        // Small c: a 20-bit prefix over the 64 lane maxima (c lanes hold a token at
        // or above it; one ballot per bit).  Wide rows: a 20-bit prefix over the 256
        // group maxima, which keeps the tokens at or above it within staging.
        uint32_t floor_key;
        if (c > (uint32_t)kCandMin) {
            uint32_t gk[NG];
#pragma unroll
            for (int g = 0; g < NG; ++g) gk[g] = gm[g] == gm[g] ? fkey(gm[g] + 0.0f) : 0u;
            floor_key = ballot_select(gk, c, 0u, 31, 12);
        } else {
            const uint32_t lk[1] = {mx == mx ? fkey(mx + 0.0f) : 0u};
            floor_key = ballot_select(lk, c, 0u, 31, 12);
        }
        // stage: per lane, its tokens at or above the floor, by a float compare
        // against the floor's value (NaN fails it); a floor whose value is not a
        // number (a key of the NaN range) or 0 (all tokens) compares by key instead
        // (the floor is wave-uniform: one branch for the wave, straight-line compares)
        const uint32_t fk = __builtin_amdgcn_readfirstlane(floor_key);
        const float fv = key_to_float(fk);
        uint32_t mask = 0, pmask = 0;      // tokens and slots at or above the floor
        if (fk > kKeyNegInf && fk <= kKeyPosInf) {
#pragma unroll
            for (int i = 0; i < kEPT; ++i) mask |= (x[i] >= fv) ? (1u << i) : 0u;
#pragma unroll
            for (int q = 0; q < kPS; ++q) pmask |= (pv[q] >= fv) ? (1u << q) : 0u;
        } else {
#pragma unroll
            for (int i = 0; i < kEPT; ++i)
                mask |= ((x[i] == x[i]) & (fkey(x[i] + 0.0f) >= fk)) ? (1u << i) : 0u;
#pragma unroll
            for (int q = 0; q < kPS; ++q)
                pmask |= ((pv[q] == pv[q]) & (fkey(pv[q] + 0.0f) >= fk)) ? (1u << q) : 0u;
        }
        uint32_t E;
        uint32_t at = dwave_excl_scan_u32((uint32_t)(__builtin_popcount(mask) + __builtin_popcount(pmask)), &E);
        uint64_t* st = stage;
        for (uint32_t b = mask; b; b &= b - 1) {
            const int i = __builtin_ctz(b);
            if (at < (uint32_t)kStageW)
                st[at] = comp_key(fkey(pick32(x, (uint32_t)i) + 0.0f), (uint32_t)elem_index<EPL>(lo, lane, i));
            ++at;
        }
        if (__ballot(pmask != 0) != 0) {
#pragma unroll
            for (int q = 0; q < kPS; ++q) {
                if ((pmask >> q) & 1u) {
                    if (at < (uint32_t)kStageW) st[at] = comp_key(fkey(pv[q] + 0.0f), pidx[q]);
                    ++at;
                }
            }
        }
        wave_lds_sync();
        // at most `cap` emitted per tile (ties at the c-th key beyond it stay
        // below the bound)
        const uint32_t cap = (uint32_t)kCapW;
        uint32_t bound = fk ? fk : 1u;
        if (E > (uint32_t)kStageW) {
            // more than kStageW tokens in the floor's bin (massive ties): emit
            // nothing and mark the tile incomplete; the row takes the full-row path
            bound = 0xFFFFFFFFu;
            E = 0;
        } else if (E > cap) {
            constexpr int SPL = kStageW / 64;
            uint32_t sk[SPL];
#pragma unroll
            for (int q = 0; q < SPL; ++q) {
                const uint32_t idx = (uint32_t)(q * 64 + lane);
                sk[q] = idx < E ? comp_k(st[idx]) : 0u;
            }
            // the c-th largest staged key, searched over all 32 bits: the floor
            // bounds it from below only (a group may hold several tokens above
            // the floor's bucket, so the answer can lie above that bucket)
            const uint32_t K = ballot_select(sk, c, 0u, 31, 0);
            uint32_t ge = 0;
#pragma unroll
            for (int q = 0; q < SPL; ++q) ge += popc64(__ballot(sk[q] >= K));
            bound = ge <= cap ? K : K + 1u;                   // ties beyond cap dropped
        }
        // emit the staged tokens with key >= bound (at most cap)
        uint64_t* out = P.w.cand + slot * kCapW;
        uint32_t nout = 0;
        for (uint32_t q0 = 0; q0 < E; q0 += 64) {
            const uint32_t idx = q0 + lane;
            const uint64_t cc = idx < E ? st[idx] : 0ull;
            const bool keep = idx < E && comp_k(cc) >= bound;
            const uint64_t bal = __ballot(keep);
            const uint32_t pos = nout + popc64(bal & ((1ull << lane) - 1));
            if (keep && pos < cap) out[pos] = cc;                // bound keeps pos < cap
            nout += popc64(bal);
        }
        if (lane == 0) {
            // more than cap at or above the bound cannot happen (the bound is the
            // c-th largest staged key, c <= cap); should it, the tile reports
            // itself incomplete and the row takes the full-row path
            const bool over = nout > cap;
            P.w.ncand[slot] = over ? 0u : nout;
            P.w.bound[slot] = over ? 0xFFFFFFFFu : bound;
        }
    }
}

// ---------------------------------------------------------------- k_scan
template <int DT, bool VEC, bool LONGH>
__global__ __launch_bounds__(kScanThreads) void k_scan(const KParams P)
{
    constexpr int EPL = DTy<DT>::EPL, SZ = DTy<DT>::SZ, NL = kEPT / EPL;
    constexpr int CW = LONGH ? kSpan : kSpan / 2;
    __shared__ ScanSmem<LONGH> L;

    const fie_sampler_args& a = P.a;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int row = blockIdx.y;
    const int NT = P.NT, V = a.vocab;
    const int slo = blockIdx.x * kSpan;                 // first token of the span
    const int shi = min(slo + kSpan, V);
    const int tile = blockIdx.x * kWavesPerWG + wv;     // this wave's tile
    const int lo = tile * kTile;
    const bool live = tile < NT;                        // waves past the row's end idle
    const RowCfg rc = row_cfg(a, row);
    const bool pen = rc.pen;
    const char* rowp = (const char*)a.logits + (size_t)row * (size_t)a.row_stride * SZ;
    const size_t slot = (size_t)row * NT + tile;
    if (blockIdx.x == 0 && blockIdx.y == 0 && tid < 2) P.w.dq[tid] = 0u;   // k_deep's queue, filled by k_finish
    if (P.helpers && blockIdx.x == 0 && tid == 0) P.w.harr[row] = 0u;     // k_finish's arrivals at the row

    // 1. The span's history bucket (k_prep), then every load of the tile: the
    //    history is counted while the logits are in flight.
    const size_t rs = (size_t)row * P.NS + blockIdx.x;
    uint32_t nb = 0, e0 = 0;
    if (pen) {
        nb = P.w.nb[rs];
        e0 = P.w.bk[rs * kBucketCap + tid];
    }
    uint4 raw[NL];
#pragma unroll
    for (int j = 0; j < NL; ++j)
        raw[j] = live ? load_group<DT, VEC>(rowp, lo + (j * 64 + lane) * EPL, V) : make_uint4(0, 0, 0, 0);

    // 2. Penalty counts of the span's ids (sampler.py:134-144), shared by the four
    //    waves.  A token's first count sets its bit in pbits and counts it as a
    //    distinct id of its tile.  A bucket that overflowed (more than kBucketCap
    //    ids in the span) is replaced by a scan of the row's whole history.
    if (pen) {
        for (int i = tid; i < CW / 4; i += kScanThreads) ((uint4*)L.cnt)[i] = make_uint4(0, 0, 0, 0);
        for (int i = tid; i < kSpan / 32; i += kScanThreads) L.pbits[i] = 0;
        if (tid < kWavesPerWG) L.uniq[tid] = 0;
        __syncthreads();
        auto count = [&](uint32_t o) {
            uint32_t was;
            if (LONGH) {
                was = atomicAdd(&L.cnt[o], 1u);
            } else {
                const uint32_t sh = (o & 1) * 16;
                was = (atomicAdd(&L.cnt[o >> 1], 1u << sh) >> sh) & 0xFFFFu;
            }
            if (was == 0) {
                atomicOr(&L.pbits[o >> 5], 1u << (o & 31));
                atomicAdd(&L.uniq[o / kTile], 1u);
            }
        };
        if (nb <= (uint32_t)kBucketCap) {
            if ((uint32_t)tid < nb) count(e0);
            for (uint32_t i = tid + kScanThreads; i < nb; i += kScanThreads) count(P.w.bk[rs * kBucketCap + i]);
        } else {
            const int64_t h0 = a.hist_offsets[row], h1 = hist_end(a, row);
            for (int64_t h = h0 + tid; h < h1; h += kScanThreads) {
                const uint32_t id = (uint32_t)a.hist_ids[h];
                if (id != 0 && id >= (uint32_t)slo && id < (uint32_t)shi) count(id - (uint32_t)slo);
            }
        }
        __syncthreads();
        if (live && lane == 0) P.w.nu[slot] = L.uniq[wv];
    } else {
        if (live && lane == 0) P.w.nu[slot] = 0;
    }
    if (!live) return;

    scan_tile<DT, LONGH>(P, rc, row, tile, raw, rowp, L.pbits, L.cnt, slo, L.stage[wv]);
}

}  // namespace fie
