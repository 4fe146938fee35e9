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
constexpr int kCandMin = 16;                     // candidates per tile for rows without top-k
constexpr int kStageW = 256;                     // tokens at or above a tile's floor, staged
constexpr int kMaxTiles = 256;                   // vocab <= 256 * 2048
constexpr int kHistPer = 8;                      // history ids per thread per batch

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
    uint64_t* cand;      // [rows * NT * kCapW]
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
// row's top-k when the top tokens spread about evenly, at least kCandMin.
FIE_DEV uint32_t cand_target(int topk, int NT)
{
    int c = kCandMin;
    if (topk > 0) c = 2 * ((topk + NT - 1) / NT) + 4;
    return (uint32_t)(c < 8 ? 8 : (c < kCapW ? c : kCapW));
}

// Token index of lane element i of the wave's tile (group i / EPL is one 16-byte
// load; groups are 64 * EPL tokens apart).
template <int EPL>
FIE_DEV int elem_index(int lo, int lane, int i) { return lo + ((i / EPL) * 64 + lane) * EPL + (i % EPL); }

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
    uint32_t zc, badc;
    uint32_t uniq[kWavesPerWG];
};

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
    const int32_t fl = a.flags[row];
    const bool greedy = fl & FIE_FLAG_GREEDY;
    const int lp = a.logprobs ? a.logprobs[row] : -1;
    const bool pen = a.apply_penalties && (fl & FIE_FLAG_PENALTY);
    const int topk = greedy ? 0 : a.top_k[row];
    const bool need_mass = lp >= 0 || (!greedy && topk == 0);
    const bool need_cand = !greedy || lp > 0;
    const float s = greedy ? 1.0f : a.scale[row];       // greedy rows stay unscaled (sampler.py:182)
    const char* rowp = (const char*)a.logits + (size_t)row * (size_t)a.row_stride * SZ;
    const size_t slot = (size_t)row * NT + tile;

    // 1. The first history batch, then every load of the tile: the history is
    //    counted while the logits are in flight.
    uint32_t hid[kHistPer];
    int64_t h0 = 0, h1 = 0;
    if (pen) {
        h0 = a.hist_offsets[row];
        h1 = a.hist_offsets[row + 1];
#pragma unroll
        for (int q = 0; q < kHistPer; ++q) {
            const int64_t h = h0 + q * kScanThreads + tid;
            hid[q] = h < h1 ? (uint32_t)a.hist_ids[h] : 0xFFFFFFFFu;
        }
    }
    uint4 raw[NL];
#pragma unroll
    for (int j = 0; j < NL; ++j)
        raw[j] = live ? load_group<DT, VEC>(rowp, lo + (j * 64 + lane) * EPL, V) : make_uint4(0, 0, 0, 0);

    // 2. Penalty counts of the span's ids (sampler.py:134-144), shared by the four
    //    waves.  A token's first count sets its bit in pbits and counts it as a
    //    distinct id of its tile.
    float rep = 1.0f, pres = 0.0f, freq = 0.0f;
    if (pen) {
        rep = a.repetition[row];
        pres = a.presence[row];
        freq = a.frequency[row];
        for (int i = tid; i < CW / 4; i += kScanThreads) ((uint4*)L.cnt)[i] = make_uint4(0, 0, 0, 0);
        for (int i = tid; i < kSpan / 32; i += kScanThreads) L.pbits[i] = 0;
        if (tid < kWavesPerWG) L.uniq[tid] = 0;
        if (tid == 0) { L.zc = 0; L.badc = 0; }
        __syncthreads();
        for (int64_t base = h0; base < h1; base += (int64_t)kHistPer * kScanThreads) {
            uint32_t ids[kHistPer];
#pragma unroll
            for (int q = 0; q < kHistPer; ++q) {
                const int64_t h = base + q * kScanThreads + tid;
                ids[q] = base == h0 ? hid[q] : (h < h1 ? (uint32_t)a.hist_ids[h] : 0xFFFFFFFFu);
            }
#pragma unroll
            for (int q = 0; q < kHistPer; ++q) {
                const uint32_t id = ids[q];
                const int64_t h = base + q * kScanThreads + tid;
                if (id >= (uint32_t)slo && id < (uint32_t)shi) {
                    const uint32_t o = id - slo;
                    if (id == 0) {
                        atomicAdd(&L.zc, 1u);
                    } else {
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
                    }
                } else if (h < h1 && id >= (uint32_t)V && slo + kSpan >= V) {
                    atomicAdd(&L.badc, 1u);
                }
            }
        }
        __syncthreads();
        if (tid == 0) {
            if (blockIdx.x == 0) P.w.tok0c[row] = L.zc;
            if (slo + kSpan >= V) P.w.bad[row] = L.badc;
        }
        if (live && lane == 0) P.w.nu[slot] = L.uniq[wv];
    } else {
        if (tid == 0) {
            if (blockIdx.x == 0) P.w.tok0c[row] = 0;
            if (slo + kSpan >= V) P.w.bad[row] = 0;
        }
        if (live && lane == 0) P.w.nu[slot] = 0;
    }
    if (!live) return;

    // 3. The penalised logits (sampler.py:169-175) of the lane's tokens; the
    //    group's bits of pbits say which tokens need their count looked up.
    float x[kEPT];
#pragma unroll
    for (int j = 0; j < NL; ++j) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) x[j * EPL + e] = lane_get<DT>(raw[j], e);
    }
    if (pen) {
        uint32_t mine = 0;   // bit i: the lane's token i is penalised
#pragma unroll
        for (int j = 0; j < NL; ++j) {
            const int o = lo - slo + (j * 64 + lane) * EPL;
            mine |= ((L.pbits[o >> 5] >> (o & 31)) & ((1u << EPL) - 1)) << (j * EPL);
        }
        for (uint32_t b = mine; b; b &= b - 1) {
            const int i = __builtin_ctz(b);
            const int o = lo - slo + ((i / EPL) * 64 + lane) * EPL + (i % EPL);
            const uint32_t cc = LONGH ? L.cnt[o] : ((L.cnt[o >> 1] >> ((o & 1) * 16)) & 0xFFFFu);
            x[i] = penalize(x[i], rep, pres, freq, cc);
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
    }
    const uint32_t fi = dwave_min_u32(first);
    if (lane == 0) P.w.maxc[slot] = km ? comp_key(km, fi) : 0ull;

    // 5. Tile mass relative to the tile maximum (rule R1): the integer weights
    //    floor(cexp(y - m_t) 2^40) < 2^41 as integer-valued floats, summed in fp64,
    //    which is exact (a lane's 32 weights stay below 2^46).
    if (need_mass) {
        double acc = 0.0;
        if (km != 0) {
            const float mt = y_of_xkey(km, s);
            if (s == 1.0f) {
#pragma unroll
                for (int i = 0; i < kEPT; ++i) acc += (double)weight40((x[i] + 0.0f) - mt);
            } else if (s >= 0x1p-30f && s <= 0x1p30f) {
                const float rs = 1.0f / s;
#pragma unroll
                for (int i = 0; i < kEPT; ++i) {
                    const float y = markstein_ok(x[i]) ? div_markstein(x[i], s, rs) : x[i] / s;
                    acc += (double)weight40((y + 0.0f) - mt);
                }
            } else {
#pragma unroll
                for (int i = 0; i < kEPT; ++i) acc += (double)weight40(scaled(x[i], s) - mt);
            }
        }
        const uint64_t tot = dwave_sum_u64((uint64_t)acc);
        if (lane == 0) P.w.sw[slot] = tot;
    }

    // 6. The tile's top tokens.  The floor is the largest 12-bit key prefix with
    //    at least c group maxima at or above it, so at least c tokens are; tokens
    //    at or above it are staged in LDS, and when more than kCapW are, the c-th
    //    largest staged key is found by a full-width ballot select.
    if (need_cand) {
        const uint32_t c = cand_target(topk, NT);
        uint32_t gk[NG];
#pragma unroll
        for (int g = 0; g < NG; ++g) gk[g] = gm[g] == gm[g] ? fkey(gm[g] + 0.0f) : 0u;
        const uint32_t floor_key = ballot_select(gk, c, 0u, 31, 20);
        // stage: per lane, its tokens at or above the floor, by a float compare
        // against the floor's value (NaN fails it); a floor whose value is not a
        // number (a key of the NaN range) or 0 (all tokens) compares by key instead
        const float fv = key_to_float(floor_key);
        const bool fv_ok = floor_key > kKeyNegInf && floor_key <= kKeyPosInf;
        uint32_t mask = 0;
#pragma unroll
        for (int i = 0; i < kEPT; ++i) {
            const bool ge = fv_ok ? (x[i] >= fv) : (x[i] == x[i] && fkey(x[i] + 0.0f) >= floor_key);
            mask |= ge ? (1u << i) : 0u;
        }
        uint32_t E;
        uint32_t at = dwave_excl_scan_u32((uint32_t)__builtin_popcount(mask), &E);
        uint64_t* st = L.stage[wv];
        for (uint32_t b = mask; b; b &= b - 1) {
            const int i = __builtin_ctz(b);
            if (at < (uint32_t)kStageW)
                st[at] = comp_key(fkey(x[i] + 0.0f), (uint32_t)elem_index<EPL>(lo, lane, i));
            ++at;
        }
        wave_lds_sync();
        uint32_t bound = floor_key ? floor_key : 1u;
        if (E > (uint32_t)kStageW) {
            // more than kStageW tokens in the floor's bin (massive ties): emit
            // nothing and mark the tile incomplete; the row takes the full-row path
            bound = 0xFFFFFFFFu;
            E = 0;
        } else if (E > (uint32_t)kCapW) {
            constexpr int SPL = kStageW / 64;
            uint32_t sk[SPL];
#pragma unroll
            for (int q = 0; q < SPL; ++q) {
                const uint32_t idx = (uint32_t)(q * 64 + lane);
                sk[q] = idx < E ? comp_k(st[idx]) : 0u;
            }
            // the floor fixed the top 12 bits unless it stayed at 0 (fewer than c
            // groups in the tile, all of them staged)
            const uint32_t K = floor_key ? ballot_select(sk, c, floor_key & 0xFFF00000u, 19, 0)
                                         : ballot_select(sk, c, 0u, 31, 0);
            uint32_t ge = 0;
#pragma unroll
            for (int q = 0; q < SPL; ++q) ge += popc64(__ballot(sk[q] >= K));
            bound = ge <= (uint32_t)kCapW ? K : K + 1u;       // ties beyond kCapW dropped
        }
        // emit the staged tokens with key >= bound (at most kCapW)
        uint64_t* out = P.w.cand + slot * kCapW;
        uint32_t nout = 0;
        for (uint32_t q0 = 0; q0 < E; q0 += 64) {
            const uint32_t idx = q0 + lane;
            const uint64_t cc = idx < E ? st[idx] : 0ull;
            const bool keep = idx < E && comp_k(cc) >= bound;
            const uint64_t bal = __ballot(keep);
            const uint32_t pos = nout + popc64(bal & ((1ull << lane) - 1));
            if (keep && pos < (uint32_t)kCapW) out[pos] = cc;   // bound keeps pos < kCapW
            nout += popc64(bal);
        }
        if (lane == 0) {
            P.w.ncand[slot] = nout;
            P.w.bound[slot] = bound;
        }
    }
}

}  // namespace fie
