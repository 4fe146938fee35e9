// The per-row kernel of the sampler (k_finish): one workgroup of 512 threads per row.
//
// It merges the tile partials of k_scan (maxima, masses, top tokens), settles token
// 0's penalty, and decides the row exactly on the candidate set whenever the
// decision provably lies among the candidates: every token whose scaled key is
// above the largest tile bound was streamed out, so a threshold, a cut or a draw
// that lands above that key is final.  Otherwise the row takes the full-row path
// in the same workgroup: radix passes that re-read the row from memory, narrowing a
// key range until it fits in LDS, then the same LDS selection.
#pragma once

#include "scan.h"

namespace fie {


constexpr int kFinThreads = 512;
constexpr int kGCap = 4096;        // composites held in LDS (candidates / a gathered bin)
constexpr int kPassBins = 1024;    // bins of a full-row radix pass / of the d-bin histogram
constexpr int kChunk = 4096;       // tokens per step of a full-row pass

// Radix digits over the 64-bit rank composite (key << 32 | ~index): three over the
// key, then three over the index (bits 31..24 of ~index are constant for V < 2^24).
struct Digit {
    int shift, bits;
};
constexpr int kLevels = 7;
__device__ constexpr Digit kDigits[kLevels] = {{54, 10}, {44, 10}, {34, 10}, {24, 10}, {14, 10}, {4, 10}, {0, 4}};

struct SelResult {
    uint64_t comp;       // the element where the running measure crosses the target
    u128 excl;           // measure of the selected set ranked before it
    u128 meas;           // its own measure
    int found;
};

struct FinSmem {
    uint64_t cand[kGCap];                       // candidates or a gathered key range
    uint32_t pc[kPassBins];                     // full-row pass: counts per bin
    union {
        uint64_t pm_lo[kPassBins];              // full-row pass: mass per bin (low limb)
        float pmf[kPassBins];                   // candidate narrowing: float mass per bin
    };
    uint64_t pm_hi[kPassBins];                  // full-row pass: mass per bin (high limb)
    uint32_t cnt[kChunk];                       // penalty counts of one chunk
    uint32_t snb[kMaxSpans];                    // history ids per span (k_prep), of a pass's row
    uint32_t hc[256];                           // LDS selection: counts per digit
    uint64_t hm_lo[256], hm_hi[256];            // LDS selection: mass per digit
    float mt[kMaxTiles + 1];                    // tile maxima of y (slot 0 = token 0)
    uint64_t ct[kMaxTiles + 1];                 // tile scales C_t
    uint32_t nc[kMaxTiles];                     // candidates per tile
    uint64_t red64[16];
    u128 red128[16];
    uint32_t red32[32];
    uint32_t n, zc, bad;
    int ibin, flag;
    uint64_t bcomp[2];
    u128 bex, bme;
    uint32_t bcnt;
    uint64_t cmax;
    SelResult sel;
    DeferRec dfr;                               // a row deferred to the full-row path in place
    uint32_t dmode;                             // its mode (0: not deferred)
};

// Weight of a y-domain composite under rule R1: floor(cexp(y - m_t) 2^40) * C_t.
// Both factors are at most 2^40; split at bit 24 they give four products of operands
// below 2^24, which the 24-bit multiplier forms at full rate (a 64 x 64-bit product
// takes eight quarter-rate 32-bit multiplies).  The sum is the exact product.
FIE_DEV u128 weight_of(const FinSmem& S, float y, uint32_t idx)
{
    const int slot = idx == 0 ? 0 : 1 + (int)(idx / kTile);
    const float w = weight40(y - S.mt[slot]);              // an integer below 2^41, as a float
    const float wh = __builtin_floorf(w * 0x1p-24f);       // exact: w has 24 significant bits
    const uint32_t w1 = (uint32_t)wh & 0x1FFFFu;
    const uint32_t w0 = (uint32_t)(w - wh * 0x1p24f) & 0xFFFFFFu;
    const uint64_t c = S.ct[slot];
    const uint32_t c0 = (uint32_t)c & 0xFFFFFFu, c1 = (uint32_t)(c >> 24) & 0x1FFFFu;
    const uint64_t p00 = (uint64_t)w0 * c0, p01 = (uint64_t)w0 * c1;
    const uint64_t p10 = (uint64_t)w1 * c0, p11 = (uint64_t)w1 * c1;
    return (u128)p00 + ((u128)(p01 + p10) << 24) + ((u128)p11 << 48);
}

FIE_DEV u128 comp_weight(const FinSmem& S, uint64_t c)
{
    return weight_of(S, key_to_float(comp_k(c)), comp_idx(c));
}

// Predicate shared by every selection: the element survives top-k / min-p (key >=
// tau), lies above the safety key (key > safe), and is kept by the top-p cut
// (composite >= cut, cut = 0 for none).
struct Pred {
    uint32_t tau;
    uint32_t safe;   // 0 = no restriction (keys are never 0)
    uint64_t cut;
    uint64_t hi = ~0ull;   // composites above hi excluded (none by default)
    FIE_DEV bool operator()(uint64_t c) const
    {
        const uint32_t k = comp_k(c);
        return k >= tau && k > safe && c >= cut && c <= hi;
    }
};

// ---------------------------------------------------------------- LDS selection
// Radix selection over S.cand[0, n): among elements satisfying `pr`, in descending
// composite order, the element where the running measure (count, or weight when
// MASS) first exceeds g: excl <= g < excl + meas.  Digits are 8-bit windows placed
// just below the common prefix of the remaining range, so few levels are needed.
template <bool MASS>
FIE_DEV SelResult lds_select(FinSmem& S, int n, const Pred pr, u128 g)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint64_t prefix = 0, pmask = 0;
    u128 excl = 0;
    for (int level = 0; level < 64; ++level) {
        // range of the remaining elements (one barrier), and a cleared histogram
        uint64_t mn = ~0ull, mx = 0;
        for (int i = tid; i < n; i += kFinThreads) {
            const uint64_t c = S.cand[i];
            if ((c & pmask) == prefix && pr(c)) {
                mn = c < mn ? c : mn;
                mx = c > mx ? c : mx;
            }
        }
        for (int i = tid; i < 256; i += kFinThreads) {
            S.hc[i] = 0;
            if (MASS) { S.hm_lo[i] = 0; S.hm_hi[i] = 0; }
        }
        mx = wave_max_u64(mx);
        mn = ~wave_max_u64(~mn);
        if (lane == 0) { S.red64[wave] = mx; S.red64[8 + wave] = mn; }
        __syncthreads();
        mx = 0;
        mn = ~0ull;
#pragma unroll
        for (int w = 0; w < kFinThreads / 64; ++w) {
            mx = S.red64[w] > mx ? S.red64[w] : mx;
            mn = S.red64[8 + w] < mn ? S.red64[8 + w] : mn;
        }
        if (mn >= mx) {
            __syncthreads();   // S.red64 is read above: no thread may reuse it yet
            if (mx == 0) return SelResult{0, 0, 0, 0};
            const u128 m = MASS ? comp_weight(S, mx) : (u128)1;
            return SelResult{mx, excl, m, g < m ? 1 : 0};
        }
        const int hb = 63 - __builtin_clzll(mn ^ mx);
        const int shift = hb >= 7 ? hb - 7 : 0;
        const uint64_t hmask = (hb >= 63) ? 0ull : ~((2ull << hb) - 1);
        for (int i = tid; i < n; i += kFinThreads) {
            const uint64_t c = S.cand[i];
            if ((c & pmask) == prefix && pr(c)) {
                const int d = (int)((c >> shift) & 0xFFu);
                if (MASS) {
                    const u128 w = comp_weight(S, c);
                    const uint64_t lo = (uint64_t)w;
                    const uint64_t old = atomicAdd((unsigned long long*)&S.hm_lo[d], (unsigned long long)lo);
                    const uint64_t hi = (uint64_t)(w >> 64) + ((old + lo < old) ? 1ull : 0ull);
                    if (hi) atomicAdd((unsigned long long*)&S.hm_hi[d], (unsigned long long)hi);
                } else {
                    atomicAdd(&S.hc[d], 1u);
                }
            }
        }
        __syncthreads();
        // wave 0 scans the 256 digits from the top
        if (tid < 64) {
            u128 loc[4];
            u128 sum = 0;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int d = 255 - (tid * 4 + q);
                loc[q] = MASS ? (((u128)S.hm_hi[d] << 64) | S.hm_lo[d]) : (u128)S.hc[d];
                sum += loc[q];
            }
            const u128 incl = wave_incl_scan_u128(sum);
            u128 run = incl - sum;
            if (run <= g && g < incl) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if (run <= g && g < run + loc[q]) {
                        S.ibin = 255 - (tid * 4 + q);
                        S.bex = run;
                    }
                    run += loc[q];
                }
            }
            if (tid == 63 && !(g < incl)) { S.ibin = -1; S.bex = incl; }
        }
        __syncthreads();
        const int d = S.ibin;
        const u128 above = S.bex;
        if (d < 0) {
            __syncthreads();
            return SelResult{0, excl + above, 0, 0};
        }
        g -= above;
        excl += above;
        prefix = (mn & hmask) | ((uint64_t)d << shift);
        pmask = shift == 0 ? ~0ull : (~((1ull << shift) - 1) | hmask);
    }
    return SelResult{0, 0, 0, 0};
}

// ---------------------------------------------------------------- full-row passes
// Visit every token of the row once, re-reading it from memory: f(y, idx) with each
// token's scaled (penalised) logit, token 0 with its settled value.  The row streams
// in kChunk-token chunks through a ring of kPassDepth register buffers, the next
// chunks' loads in flight while one is processed.  A pass is bound by its per-token
// instructions: the third buffer gains 3% on many full-row rows at once and nothing
// on a single one.  A penalised row's counts come
// from k_prep's span bucket, loaded with the chunk (one id per thread: kBucketCap ==
// kFinThreads), so counting never waits on a dependent load; a span whose bucket
// overflowed is counted from the whole history instead.
constexpr int kPassDepth = 3;
static_assert(kBucketCap == kFinThreads && kSpan == 2 * kChunk, "bucket entries per thread, chunks per span");

template <int DT, bool VEC, class F>
FIE_DEV void row_pass(FinSmem& S, const KParams& P, int row, float s, bool pen, float rep,
                      float pres, float freq, uint32_t k0, F&& f)
{
    constexpr int EPL = DTy<DT>::EPL, SZ = DTy<DT>::SZ;
    constexpr int NL = kChunk / kFinThreads / EPL;
    constexpr int D = kPassDepth;
    const fie_sampler_args& a = P.a;
    const int V = a.vocab, tid = threadIdx.x;
    const int nch = (V + kChunk - 1) / kChunk;
    const char* rowp = (const char*)a.logits + (size_t)row * (size_t)a.row_stride * SZ;
    const bool mark = s != 1.0f && s >= 0x1p-30f && s <= 0x1p30f;
    const float rs = 1.0f / s;
    if (tid == 0 && k0) f(key_to_float(k0), 0u);
    uint4 buf[D][NL];
    uint32_t bof[D];
    bool overflow = false;
    if (pen) {
        for (int i = tid; i < P.NS; i += kFinThreads) {
            const uint32_t nb = P.w.nb[(size_t)row * P.NS + i];
            S.snb[i] = nb;
            overflow |= nb > (uint32_t)kBucketCap;
        }
    }
    if (VEC && !__syncthreads_or(overflow)) {
        // The common case, as straight-line streaming: whole chunks, one vector load
        // per group, every span's bucket complete.  Every step of the ring issues the
        // same loads (past the last whole chunk it reloads that chunk, unused), so the
        // compiler's wait counts see the D - 1 chunks still in flight; the partial
        // last chunk follows the ring.
        const int nfull = V / kChunk;
        auto issue_full = [&](uint4 (&b)[NL], uint32_t& of, int c) {
            const int lo = (c < nfull ? c : nfull - 1) * kChunk;
#pragma unroll
            for (int j = 0; j < NL; ++j) b[j] = *(const uint4*)(rowp + (size_t)(lo + (j * kFinThreads + tid) * EPL) * SZ);
            of = P.w.bk[((size_t)row * P.NS + lo / kSpan) * kBucketCap + tid];
        };
        auto count_bucket = [&](uint32_t of, int lo) {
            for (int i = tid; i < kChunk / 4; i += kFinThreads) ((uint4*)S.cnt)[i] = make_uint4(0, 0, 0, 0);
            __syncthreads();
            const uint32_t o = of - (uint32_t)(lo % kSpan);
            if ((uint32_t)tid < S.snb[lo / kSpan] && o < (uint32_t)kChunk) atomicAdd(&S.cnt[o], 1u);
            __syncthreads();
        };
        auto visit = [&](const uint4 (&b)[NL], int lo) {
#pragma unroll
            for (int j = 0; j < NL; ++j) {
                const int e0 = lo + (j * kFinThreads + tid) * EPL;
#pragma unroll
                for (int e = 0; e < EPL; ++e) {
                    const int idx = e0 + e;
                    if (idx >= V || idx == 0) continue;
                    float x = lane_get<DT>(b[j], e);
                    if (pen) {
                        const uint32_t cc = S.cnt[idx - lo];
                        if (cc) x = penalize(x, rep, pres, freq, cc);
                    }
                    float y;
                    if (s == 1.0f) y = x + 0.0f;
                    else if (mark && markstein_ok(x)) y = div_markstein(x, s, rs) + 0.0f;
                    else y = scaled(x, s);
                    f(y, (uint32_t)idx);
                }
            }
        };
        if (nfull > 0) {
#pragma unroll
            for (int q = 0; q < D; ++q) issue_full(buf[q], bof[q], q);
            for (int c0 = 0; c0 < nfull; c0 += D) {
#pragma unroll
                for (int q = 0; q < D; ++q) {
                    const int c = c0 + q;
                    if (c < nfull) {
                        if (pen) count_bucket(bof[q], c * kChunk);
                        visit(buf[q], c * kChunk);
                        if (pen) __syncthreads();
                    }
                    issue_full(buf[q], bof[q], c + D);
                }
            }
        }
        const int lo = nfull * kChunk;
        if (lo < V) {
#pragma unroll
            for (int j = 0; j < NL; ++j) buf[0][j] = load_group<DT, VEC>(rowp, lo + (j * kFinThreads + tid) * EPL, V);
            if (pen) count_bucket(P.w.bk[((size_t)row * P.NS + lo / kSpan) * kBucketCap + tid], lo);
            visit(buf[0], lo);
        }
        __syncthreads();
        return;
    }
    auto issue = [&](uint4 (&b)[NL], uint32_t& of, int c) {
        const int lo = c * kChunk;
#pragma unroll
        for (int j = 0; j < NL; ++j) b[j] = load_group<DT, VEC>(rowp, lo + (j * kFinThreads + tid) * EPL, V);
        if (pen) {
            // a chunk past the row's end (the ring's tail) reads the last span's entry, unused
            const int sp = lo / kSpan < P.NS ? lo / kSpan : P.NS - 1;
            of = P.w.bk[((size_t)row * P.NS + sp) * kBucketCap + tid];
        }
    };
    auto count = [&](uint32_t of, int lo, int hi) {
        if (lo >= V) return;                                     // uniform: no token to count
        for (int i = tid; i < kChunk / 4; i += kFinThreads) ((uint4*)S.cnt)[i] = make_uint4(0, 0, 0, 0);
        __syncthreads();
        const uint32_t nb = S.snb[lo / kSpan];
        if (nb <= (uint32_t)kBucketCap) {
            const uint32_t o = of - (uint32_t)(lo % kSpan);
            if ((uint32_t)tid < nb && o < (uint32_t)kChunk) atomicAdd(&S.cnt[o], 1u);
        } else {
            const int64_t h0 = a.hist_offsets[row], h1 = hist_end(a, row);
            for (int64_t h = h0 + tid; h < h1; h += kFinThreads) {
                const uint32_t id = (uint32_t)a.hist_ids[h];
                if (id >= (uint32_t)lo && id < (uint32_t)hi && id != 0) atomicAdd(&S.cnt[id - lo], 1u);
            }
        }
        __syncthreads();
    };
#pragma unroll
    for (int q = 0; q < D; ++q)
        if (q < nch) issue(buf[q], bof[q], q);
    // a ring of D buffers in fixed roles (no register copies, which would wait on
    // loads still in flight): buffer q holds chunk c0 + q while the others load.
    // Past the row's end the loads read nothing and every token fails idx < V.
    for (int c0 = 0; c0 < nch; c0 += D) {
#pragma unroll
        for (int q = 0; q < D; ++q) {
            const int c = c0 + q;
            const int lo = c * kChunk, hi = min(lo + kChunk, V);
            if (pen) count(bof[q], lo, hi);
#pragma unroll
            for (int j = 0; j < NL; ++j) {
                const int e0 = lo + (j * kFinThreads + tid) * EPL;
#pragma unroll
                for (int e = 0; e < EPL; ++e) {
                    const int idx = e0 + e;
                    if (idx >= V || idx == 0) continue;
                    float x = lane_get<DT>(buf[q][j], e);
                    if (pen) {
                        const uint32_t cc = S.cnt[idx - lo];
                        if (cc) x = penalize(x, rep, pres, freq, cc);
                    }
                    float y;
                    if (s == 1.0f) y = x + 0.0f;
                    else if (mark && markstein_ok(x)) y = div_markstein(x, s, rs) + 0.0f;
                    else y = scaled(x, s);
                    f(y, (uint32_t)idx);
                }
            }
            if (pen) __syncthreads();
            issue(buf[q], bof[q], c + D);
        }
    }
    __syncthreads();
}

// Count (and mass) histogram of one digit level over the elements satisfying pr
// whose composite bits above the digit equal `hiprefix`.
template <int DT, bool VEC, bool MASS>
FIE_DEV void pass_hist(FinSmem& S, const KParams& P, int row, float s, bool pen, float rep,
                       float pres, float freq, uint32_t k0, const Pred pr, int level,
                       uint64_t hiprefix)
{
    const Digit dg = kDigits[level];
    const int top = dg.shift + dg.bits;
    const uint32_t dmask = (1u << dg.bits) - 1;
    for (int i = threadIdx.x; i < kPassBins; i += kFinThreads) {
        S.pc[i] = 0;
        if (MASS) { S.pm_lo[i] = 0; S.pm_hi[i] = 0; }
    }
    __syncthreads();
    row_pass<DT, VEC>(S, P, row, s, pen, rep, pres, freq, k0, [&](float y, uint32_t idx) {
        const uint64_t c = comp_key(fkey(y), idx);
        if ((top >= 64 || (c >> top) == hiprefix) && pr(c)) {
            const uint32_t d = (uint32_t)(c >> dg.shift) & dmask;
            atomicAdd(&S.pc[d], 1u);
            if (MASS) {
                const u128 w = comp_weight(S, c);
                const uint64_t lo = (uint64_t)w;
                const uint64_t old = atomicAdd((unsigned long long*)&S.pm_lo[d], (unsigned long long)lo);
                const uint64_t hi = (uint64_t)(w >> 64) + ((old + lo < old) ? 1ull : 0ull);
                if (hi) atomicAdd((unsigned long long*)&S.pm_hi[d], (unsigned long long)hi);
            }
        }
    });
}

// Descending scan of the pass histogram for the bin where the running measure
// crosses g.  Returns the bin (-1 if the total is <= g) with S.bex = measure above
// it and S.bcnt = its count.
template <bool MASS>
FIE_DEV int pass_pick(FinSmem& S, int nbins, u128 g)
{
    const int tid = threadIdx.x;
    const int per = (nbins + kFinThreads - 1) / kFinThreads;   // 1..4
    u128 sum = 0;
    for (int q = 0; q < per; ++q) {
        const int b = nbins - 1 - (tid * per + q);
        if (b >= 0) sum += MASS ? (((u128)S.pm_hi[b] << 64) | S.pm_lo[b]) : (u128)S.pc[b];
    }
    // block exclusive scan of u128 in thread order
    const int lane = tid & 63, wave = tid >> 6;
    const u128 incl = wave_incl_scan_u128(sum);
    if (lane == 63) S.red128[wave] = incl;
    if (tid == 0) S.ibin = -1;
    __syncthreads();
    u128 before = 0, all = 0;
    for (int w = 0; w < kFinThreads / 64; ++w) {
        if (w < wave) before += S.red128[w];
        all += S.red128[w];
    }
    before += incl - sum;
    if (before <= g && g < before + sum) {
        u128 run = before;
        for (int q = 0; q < per; ++q) {
            const int b = nbins - 1 - (tid * per + q);
            if (b < 0) break;
            const u128 m = MASS ? (((u128)S.pm_hi[b] << 64) | S.pm_lo[b]) : (u128)S.pc[b];
            if (run <= g && g < run + m) {
                S.ibin = b;
                S.bex = run;
                S.bcnt = S.pc[b];
            }
            run += m;
        }
    }
    if (tid == 0 && !(g < all)) S.bex = all;
    __syncthreads();
    const int b = S.ibin;
    __syncthreads();
    return b;
}

// Gather the elements satisfying pr whose composite bits from `top` up equal
// `hiprefix` into S.cand; returns their number (the caller ensures <= kGCap).
template <int DT, bool VEC>
FIE_DEV int pass_gather(FinSmem& S, const KParams& P, int row, float s, bool pen, float rep,
                        float pres, float freq, uint32_t k0, const Pred pr, int top,
                        uint64_t hiprefix)
{
    if (threadIdx.x == 0) S.n = 0;
    __syncthreads();
    row_pass<DT, VEC>(S, P, row, s, pen, rep, pres, freq, k0, [&](float y, uint32_t idx) {
        const uint64_t c = comp_key(fkey(y), idx);
        if ((top >= 64 || (c >> top) == hiprefix) && pr(c)) {
            const uint32_t at = atomicAdd(&S.n, 1u);
            if (at < (uint32_t)kGCap) S.cand[at] = c;
        }
    });
    const int n = (int)S.n;
    __syncthreads();
    return n;
}

// Full-row selection: radix levels over re-read passes until the selected key
// range fits in LDS, then the LDS selection.  When `have_l1` the level-0 pass
// histogram for the same predicate is already in S (and `l1_adjust` has been
// applied by the caller).
template <int DT, bool VEC, bool MASS>
FIE_DEV SelResult row_select(FinSmem& S, const KParams& P, int row, float s, bool pen, float rep,
                             float pres, float freq, uint32_t k0, const Pred pr, u128 g,
                             bool have_l1)
{
    uint64_t hiprefix = 0;
    u128 excl = 0;
    for (int level = 0; level < kLevels; ++level) {
        const Digit dg = kDigits[level];
        if (!(level == 0 && have_l1))
            pass_hist<DT, VEC, MASS>(S, P, row, s, pen, rep, pres, freq, k0, pr, level, hiprefix);
        const int b = pass_pick<MASS>(S, 1 << dg.bits, g);
        if (b < 0) return SelResult{0, excl + S.bex, 0, 0};
        const u128 above = S.bex;
        const uint32_t cnt = S.bcnt;
        __syncthreads();
        g -= above;
        excl += above;
        hiprefix = (hiprefix << dg.bits) | (uint64_t)b;
        if (cnt <= (uint32_t)kGCap) {
            const int n = pass_gather<DT, VEC>(S, P, row, s, pen, rep, pres, freq, k0, pr,
                                               dg.shift, hiprefix);
            SelResult r = lds_select<MASS>(S, n, pr, g);
            r.excl += excl;
            return r;
        }
    }
    return SelResult{0, 0, 0, 0};
}

// Rule R5 as a threshold: L = the bound a 32-step bisection over the order keys of
// d in [-80, 0] finds for cexp(d) >= mp, then the smallest y-key K with
// fl(key_to_float(K) - M) >= L (monotone in K).  0 when mp <= 0.
FIE_DEV float minp_bound(float mp)
{
    uint32_t lo = fkey(-80.0f), hi = fkey(0.0f);
    if (cexp(key_to_float(lo)) >= mp) return -__builtin_inff();
    while (hi - lo > 1) {
        const uint32_t mid = lo + (hi - lo) / 2;
        if (cexp(key_to_float(mid)) >= mp) hi = mid;
        else lo = mid;
    }
    return key_to_float(hi);
}

FIE_DEV uint32_t minp_key(float M, float mp)
{
    if (!(mp > 0.0f)) return 0;
    const float L = minp_bound(mp);
    uint32_t lo = kKeyNegInf, hi = fkey(M);
    if ((key_to_float(lo) - M) >= L) return lo;          // every value passes
    if (!((key_to_float(hi) - M) >= L)) return hi;       // degenerate rows (M not finite)
    while (hi - lo > 1) {
        const uint32_t mid = lo + (hi - lo) / 2;
        if ((key_to_float(mid) - M) >= L) hi = mid;
        else lo = mid;
    }
    return hi;
}

// ---------------------------------------------------------------- binned full-row path
// Bins of a row by d = fl(M - y) at kDQ bins per unit (the last bin takes
// d >= (kPassBins - 1) / kDQ and NaN).  fl(M - y) and the scaling by a power of two are monotone, so bins lie
// in rule R2 order: a lower bin holds only larger values, and ties share a bin.
constexpr float kDQ = 64.0f;

FIE_DEV int dbin_y(float M, float y)
{
    const float q = (M - y) * kDQ;
    return q < (float)(kPassBins - 1) ? (int)q : kPassBins - 1;
}

FIE_DEV int dbin_key(float M, uint32_t key) { return dbin_y(M, key_to_float(key)); }

// Bin masses of the d-bins are kept as two 41-bit limbs (w < 2^82): each limb sum
// over at most 2^19 tokens stays below 2^60, so plain non-returning 64-bit LDS
// atomics add them exactly, with no carry to detect.
FIE_DEV u128 bin_mass(const FinSmem& S, int b) { return ((u128)S.pm_hi[b] << 41) + S.pm_lo[b]; }

FIE_DEV void bin_add(FinSmem& S, int b, u128 w)
{
    constexpr uint64_t kLimb = (1ull << 41) - 1;
    const uint64_t lo = (uint64_t)w & kLimb, hi = (uint64_t)(w >> 41);
    if (lo) atomicAdd((unsigned long long*)&S.pm_lo[b], (unsigned long long)lo);
    if (hi) atomicAdd((unsigned long long*)&S.pm_hi[b], (unsigned long long)hi);
}

// Ascending scan of bins [0, bmax], bin bmax measuring `last` instead of its own
// total, for the bin where the running measure (count, or mass when MASS) first
// exceeds g; -1 when the total is <= g.  *above receives the measure before it
// (the total when -1).
template <bool MASS>
FIE_DEV int dbin_pick(FinSmem& S, int bmax, u128 last, u128 g, u128* above)
{
    constexpr int per = kPassBins / kFinThreads;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    auto meas = [&](int b) -> u128 {
        if (b > bmax) return 0;
        if (b == bmax) return last;
        return MASS ? bin_mass(S, b) : (u128)S.pc[b];
    };
    u128 sum = 0;
#pragma unroll
    for (int q = 0; q < per; ++q) sum += meas(tid * per + q);
    const u128 incl = wave_incl_scan_u128(sum);
    if (lane == 63) S.red128[wave] = incl;
    if (tid == 0) S.ibin = -1;
    __syncthreads();
    u128 before = 0, all = 0;
    for (int w = 0; w < kFinThreads / 64; ++w) {
        if (w < wave) before += S.red128[w];
        all += S.red128[w];
    }
    before += incl - sum;
    if (before <= g && g < before + sum) {
        u128 run = before;
#pragma unroll
        for (int q = 0; q < per; ++q) {
            const u128 m = meas(tid * per + q);
            if (run <= g && g < run + m) {
                S.ibin = tid * per + q;
                S.bex = run;
            }
            run += m;
        }
    }
    if (tid == 0 && !(g < all)) S.bex = all;
    __syncthreads();
    const int b = S.ibin;
    *above = S.bex;
    __syncthreads();
    return b;
}

// The full-row path on the bin histogram: one pass for the counts and masses of
// every bin, then each crossing (top-k rank, top-p cut, draw) is found on the bins
// and settled exactly among the elements of its one bin, gathered by a pass that
// needs no weights.  Returns false (nothing decided) when a bin to be gathered
// holds more than kGCap elements.
template <int DT, bool VEC>
FIE_DEV bool binned_deep(FinSmem& S, const KParams& P, int row, float s, bool pen, float rep,
                         float pres, float freq, uint32_t k0, float M, int topk, float mp, float tp,
                         double u, u128 sall, uint32_t* tk_out, uint32_t* tau_out, uint64_t* cut_out,
                         u128* T_out, uint64_t* tok_out, bool hd)
{
    const int tid = threadIdx.x;
    // The span helpers' histograms and bucketed composites stand in for the passes
    // when every helper binned against this row maximum (token 0 is not the
    // maximum); otherwise the row is re-read.
    bool use_h = false;
    if (hd) {
        bool ok = true;
        for (int i = tid; i < P.NS; i += kFinThreads) ok &= P.w.hmk[(size_t)row * P.NS + i] == fkey(M);
        use_h = __syncthreads_and(ok);
    }
    if (use_h) {
        // two adjacent bins per thread, one vector load per span and array, and the
        // loads of up to kMerge spans issued together (a span at a time waits on each
        // round trip: ~12 us for a row of 19 spans)
        constexpr int kMerge = 20;
        const int b0 = 2 * tid;
        uint32_t c0 = 0, c1 = 0;
        uint64_t l0 = 0, l1 = 0, h0 = 0, h1 = 0;
        for (int sp0 = 0; sp0 < P.NS; sp0 += kMerge) {
            uint2 vc[kMerge];
            ulonglong2 vl[kMerge], vh[kMerge];
#pragma unroll
            for (int q = 0; q < kMerge; ++q) {
                if (sp0 + q < P.NS) {
                    const size_t o = ((size_t)row * P.NS + sp0 + q) * kHBins + b0;
                    vc[q] = *(const uint2*)(P.w.hpc + o);
                    vl[q] = *(const ulonglong2*)(P.w.hlo + o);
                    vh[q] = *(const ulonglong2*)(P.w.hhi + o);
                } else {
                    vc[q] = make_uint2(0, 0);
                    vl[q] = make_ulonglong2(0, 0);
                    vh[q] = make_ulonglong2(0, 0);
                }
            }
#pragma unroll
            for (int q = 0; q < kMerge; ++q) {
                c0 += vc[q].x;
                c1 += vc[q].y;
                l0 += vl[q].x;
                l1 += vl[q].y;
                h0 += vh[q].x;
                h1 += vh[q].y;
            }
        }
        S.pc[b0] = c0;
        S.pc[b0 + 1] = c1;
        S.pm_lo[b0] = l0;
        S.pm_lo[b0 + 1] = l1;
        S.pm_hi[b0] = h0;
        S.pm_hi[b0 + 1] = h1;
        __syncthreads();
        if (tid == 0 && k0) {
            const float y = key_to_float(k0);
            const int b = dbin_y(M, y);
            S.pc[b] += 1u;
            bin_add(S, b, weight_of(S, y, 0u));
        }
        __syncthreads();
    } else {
        for (int i = tid; i < kPassBins; i += kFinThreads) {
            S.pc[i] = 0;
            S.pm_lo[i] = 0;
            S.pm_hi[i] = 0;
        }
        __syncthreads();
        row_pass<DT, VEC>(S, P, row, s, pen, rep, pres, freq, k0, [&](float y, uint32_t idx) {
            const int b = dbin_y(M, y);
            atomicAdd(&S.pc[b], 1u);
            bin_add(S, b, weight_of(S, y, idx));
        });
    }
    // S.cand holds the elements (ncur of them) of bins [cur_lo, cur_hi] and, when
    // cur2_lo >= 0, of bins [cur2_lo, cur2_hi] as well.
    int cur_lo = -1, cur_hi = -1, cur2_lo = -1, cur2_hi = -1, ncur = 0;
    auto gather2 = [&](int bl, int bh, int b2l, int b2h) -> bool {
        if (bl == cur_lo && bh == cur_hi && b2l == cur2_lo && b2h == cur2_hi) return true;
        uint32_t cnt = 0;
        for (int b = bl; b <= bh; ++b) cnt += S.pc[b];
        for (int b = b2l; b2l >= 0 && b <= b2h; ++b) cnt += S.pc[b];
        if (cnt > (uint32_t)kGCap) return false;
        if (use_h) {
            // the bins' segments of every span's bucketed composites, concatenated
            __syncthreads();
            const int nseg = 2 * P.NS;
            uint32_t st = 0, len = 0;
            if (tid < nseg) {
                const int sp = tid >> 1, l = (tid & 1) ? b2l : bl, h = (tid & 1) ? b2h : bh;
                if (l >= 0) {
                    const uint32_t* off = P.w.hoff + ((size_t)row * P.NS + sp) * kHOffs;
                    st = off[l];
                    len = off[h + 1] - st;
                }
            }
            uint32_t total;
            const uint32_t pre = block_excl_scan_u32<kFinThreads>(len, S.red32, &total);
            if (tid < nseg) {
                S.hc[tid] = pre;
                S.cnt[tid] = st;
            }
            __syncthreads();
            const uint32_t n = total < (uint32_t)kGCap ? total : (uint32_t)kGCap;
            for (uint32_t i = tid; i < n; i += kFinThreads) {
                int lo = 0, hi = nseg - 1;            // the last segment starting at or before i
                while (lo < hi) {
                    const int mid = (lo + hi + 1) >> 1;
                    if (S.hc[mid] <= i) lo = mid;
                    else hi = mid - 1;
                }
                const size_t src = ((size_t)row * P.NS + (lo >> 1)) * kSpan + S.cnt[lo] + (i - S.hc[lo]);
                S.cand[i] = P.w.hcomp[src];
            }
            uint32_t m = n;
            if (k0) {
                const int b = dbin_y(M, key_to_float(k0));
                if (((b >= bl && b <= bh) || (b2l >= 0 && b >= b2l && b <= b2h)) && m < (uint32_t)kGCap) {
                    if (tid == 0) S.cand[m] = comp_key(k0, 0);
                    ++m;
                }
            }
            ncur = (int)m;
        } else {
        if (tid == 0) S.n = 0;
        __syncthreads();
        row_pass<DT, VEC>(S, P, row, s, pen, rep, pres, freq, k0, [&](float y, uint32_t idx) {
            const int b = dbin_y(M, y);
            if ((b >= bl && b <= bh) || (b2l >= 0 && b >= b2l && b <= b2h)) {
                const uint32_t at = atomicAdd(&S.n, 1u);
                if (at < (uint32_t)kGCap) S.cand[at] = comp_key(fkey(y), idx);
            }
        });
        ncur = (int)S.n;
        }
        cur_lo = bl;
        cur_hi = bh;
        cur2_lo = b2l;
        cur2_hi = b2h;
        __syncthreads();
        return true;
    };
    auto gather = [&](int bl, int bh) -> bool { return gather2(bl, bh, -1, -1); };

    // top-k threshold: the element of rank topk - 1
    uint32_t tk = 0;
    if (topk > 0) {
        u128 above;
        const int b = dbin_pick<false>(S, kPassBins - 1, (u128)S.pc[kPassBins - 1], (u128)(topk - 1), &above);
        if (b < 0 || !gather(b, b)) return false;
        const SelResult r = lds_select<false>(S, ncur, Pred{0, 0, 0}, (u128)(topk - 1) - above);
        if (!r.found) return false;
        tk = comp_k(r.comp);
    }
    const uint32_t tmp = minp_key(M, mp);
    const uint32_t tau = tk > tmp ? tk : tmp;

    // survivors (key >= tau): whole bins before tau's bin, part of that bin
    int bt = kPassBins - 1;
    u128 lastt = bin_mass(S, kPassBins - 1);
    u128 Sv = sall;
    if (tau != 0) {
        bt = dbin_key(M, tau);
        if (!gather(bt, bt)) return false;
        u128 part = 0;
        for (int i = tid; i < ncur; i += kFinThreads)
            if (comp_k(S.cand[i]) >= tau) part += comp_weight(S, S.cand[i]);
        lastt = block_sum_u128<kFinThreads>(part, S.red128);
        u128 before = 0;
        for (int b = tid; b < bt; b += kFinThreads) before += bin_mass(S, b);
        Sv = lastt + block_sum_u128<kFinThreads>(before, S.red128);
    }

    // top-p cut among the survivors.  The cut's bin b fixes T to (above, above +
    // m_b], hence the draw t = floor(u T) to a short run of bins [dl, dh]; the pass
    // that gathers b gathers that run too when it fits.
    uint64_t cut = 0;
    u128 T = Sv;
    int bc = bt;
    u128 lastc = lastt;
    int dl = -1, dh = -1;     // the draw's run of bins, gathered with the cut's
    u128 above_dl = 0;        // survivors' mass before bin dl
    if (tp < 1.0f) {
        const u128 thr = ceil_mul_f32(tp, Sv);
        u128 above;
        const int b = dbin_pick<true>(S, bt, lastt, thr - 1, &above);
        if (b < 0) {
            T = above;                            // every survivor; no cut (Sv == 0)
        } else {
            const u128 mb = b == bt ? lastt : bin_mass(S, b);
            u128 a2, a3;
            dl = dbin_pick<true>(S, b, mb, floor_mul_f64(u, above + 1), &a2);
            dh = dbin_pick<true>(S, b, mb, floor_mul_f64(u, above + mb), &a3);
            above_dl = a2;
            if (dl < 0 || dh < 0 || dh >= b || !gather2(b, b, dl, dh)) {
                dl = dh = -1;
                if (!gather(b, b)) return false;
            }
            // within bin b only: composites of the lower bins (the draw's run) are larger
            uint64_t chi = ~0ull;
            if (dl >= 0) {
                uint64_t mn = ~0ull;
                for (int i = tid; i < ncur; i += kFinThreads)
                    if (dbin_key(M, comp_k(S.cand[i])) < b) mn = S.cand[i] < mn ? S.cand[i] : mn;
                mn = ~wave_max_u64(~mn);
                if ((tid & 63) == 0) S.red64[tid >> 6] = mn;
                __syncthreads();
                for (int w = 0; w < kFinThreads / 64; ++w) mn = S.red64[w] < mn ? S.red64[w] : mn;
                __syncthreads();
                chi = mn - 1;
            }
            Pred pc{tau, 0, 0};
            pc.hi = chi;
            const SelResult r = lds_select<true>(S, ncur, pc, thr - 1 - above);
            if (!r.found) return false;
            cut = r.comp;
            T = above + r.excl + r.meas;
            bc = b;
            lastc = T - above;
        }
    }

    // the draw among the kept tokens (the largest token when their mass is 0)
    uint64_t tok = 0;
    if (T == 0) {
        u128 above;
        const int b = dbin_pick<false>(S, kPassBins - 1, (u128)S.pc[kPassBins - 1], 0, &above);
        if (b < 0 || !gather(b, b)) return false;
        const SelResult r = lds_select<false>(S, ncur, Pred{0, 0, 0}, 0);
        if (!r.found) return false;
        tok = r.comp;
    } else {
        const u128 g = floor_mul_f64(u, T);
        u128 above;
        const int b = dbin_pick<true>(S, bc, lastc, g, &above);
        if (b < 0) return false;
        Pred pd{tau, 0, cut};
        u128 base = above;
        if (dl >= 0 && b >= dl && b <= dh) {
            base = above_dl;                      // the held run [dl, dh]: its elements rank first
        } else {
            if (!(b == cur_lo && b == cur_hi) && !gather(b, b)) return false;
            if (cur2_lo >= 0) {
                // bin b held below the run: skip the run's (larger) composites
                uint64_t mn = ~0ull;
                for (int i = tid; i < ncur; i += kFinThreads)
                    if (dbin_key(M, comp_k(S.cand[i])) < b) mn = S.cand[i] < mn ? S.cand[i] : mn;
                mn = ~wave_max_u64(~mn);
                if ((tid & 63) == 0) S.red64[tid >> 6] = mn;
                __syncthreads();
                for (int w = 0; w < kFinThreads / 64; ++w) mn = S.red64[w] < mn ? S.red64[w] : mn;
                __syncthreads();
                pd.hi = mn - 1;
            }
        }
        const SelResult r = lds_select<true>(S, ncur, pd, g - base);
        if (!r.found) return false;
        tok = r.comp;
    }
    *tk_out = tk;
    *tau_out = tau;
    *cut_out = cut;
    *T_out = T;
    *tok_out = tok;
    return true;
}

// The shortest R2 prefix of the complete candidates S.cand[0, nv) holding at least
// `cnt` elements and, when use_mass, mass above g, moved to S.cand[0, m); returns m
// (nv, untouched, when no shorter prefix qualifies or it would not fit the staging
// area).  The prefix is a union of d-bins (dbin_key), located on a count and mass
// histogram of the candidates, so the sort that follows handles only the elements a
// top-k threshold, a top-p cut, a draw or top-L logprobs can reach.
FIE_DEV int narrow_candidates(FinSmem& S, int nv, float M, int cnt, bool use_mass, u128 g)
{
    const int tid = threadIdx.x;
    for (int i = tid; i < kPassBins; i += kFinThreads) {
        S.pc[i] = 0;
        S.pm_lo[i] = 0;
        S.pm_hi[i] = 0;
    }
    __syncthreads();
    for (int i = tid; i < nv; i += kFinThreads) {
        const uint64_t c = S.cand[i];
        const int b = dbin_key(M, comp_k(c));
        atomicAdd(&S.pc[b], 1u);
        if (use_mass) bin_add(S, b, comp_weight(S, c));
    }
    __syncthreads();
    u128 above;
    int bs = 0;
    if (cnt > 0) {
        bs = dbin_pick<false>(S, kPassBins - 1, (u128)S.pc[kPassBins - 1], (u128)(cnt - 1), &above);
        if (bs < 0) return nv;
    }
    if (use_mass) {
        const int b2 = dbin_pick<true>(S, kPassBins - 1, bin_mass(S, kPassBins - 1), g, &above);
        if (b2 < 0) return nv;
        bs = b2 > bs ? b2 : bs;
    }
    constexpr int kStage = kChunk / 2;           // S.cnt holds this many composites
    uint64_t* tmp = (uint64_t*)S.cnt;
    if (tid == 0) S.n = 0;
    __syncthreads();
    for (int i = tid; i < nv; i += kFinThreads) {
        const uint64_t c = S.cand[i];
        if (dbin_key(M, comp_k(c)) <= bs) {
            const uint32_t at = atomicAdd(&S.n, 1u);
            if (at < (uint32_t)kStage) tmp[at] = c;
        }
    }
    __syncthreads();
    const int m = (int)S.n;
    __syncthreads();
    if (m > kStage || m >= nv) return nv;
    for (int i = tid; i < m; i += kFinThreads) S.cand[i] = tmp[i];
    __syncthreads();
    return m;
}

// Token 0 keeps its penalty iff the row is the widest of the batch (no pad entry
// rewrites index 0 after it) and no id >= vocab first occurs after it
// (sampler.py:148,156-157,174-175 with a sequential scatter).
FIE_DEV bool q1_keeps(FinSmem& S, const KParams& P, int row)
{
    const fie_sampler_args& a = P.a;
    const int NT = P.NT, B = a.rows, tid = threadIdx.x;
    auto nu_of = [&](int r) -> uint32_t {
        if (!(a.flags[r] & FIE_FLAG_PENALTY)) return 0u;
        uint32_t u = P.w.tok0c[r] ? 1u : 0u;
        if (a.hist_invalid) u += (uint32_t)a.hist_invalid[r] & 0x3FFFFFFFu;
        return u;
    };
    uint32_t mine = 0, wmax = 0;
    for (int r = tid; r < B; r += kFinThreads) {
        uint32_t u = nu_of(r);
        for (int t = 0; t < NT; ++t) u += P.w.nu[(size_t)r * NT + t];
        wmax = u > wmax ? u : wmax;
        if (r == row) S.red32[31] = u;
    }
    wmax = block_max_u32<kFinThreads>(wmax, S.red32);
    mine = S.red32[31];
    __syncthreads();
    const bool late = a.hist_invalid && (((uint32_t)a.hist_invalid[row] >> 30) & 1u);
    return mine == wmax && !late;
}

// ---------------------------------------------------------------- candidates
// A tile's candidates sit in kCapW (= one wave) slots of the partials, the first
// S.nc[t] of them valid: wave w reads tile t = t0 + w + kFinWaves q with one 512-byte
// load, Q tiles per wave held at once (Q = 10: rows of up to 80 tiles in one round
// trip; kReloadQ where registers are short).
constexpr int kFinWaves = kFinThreads / 64;
constexpr int kReloadQ = 5;
static_assert(kCapW == 64, "one tile's candidate slots per wave");
static_assert(kMaxTiles < kFinThreads, "the last thread is free for token 0");

// Float mass of a token y relative to the row maximum M: rule R1's weight / 2^80 up
// to the floors of R1 and the exponentials' rounding (used only to narrow).
FIE_DEV float approx_mass(float y, float M) { return __expf(y - M); }

// The x-domain candidate slot as a y-domain composite.  rs = 1/s when s lies in
// Markstein's range (cand_rs), else 0: inside the range the corrected product is
// the IEEE quotient, three operations instead of the divide's sequence.
FIE_DEV uint64_t cand_y(uint64_t xc, float s, float rs)
{
    const float x = key_to_float(comp_k(xc));
    float y;
    if (s == 1.0f) y = x;
    else if (rs != 0.0f && markstein_ok(x)) y = div_markstein(x, s, rs) + 0.0f;
    else y = scaled(x, s);
    return comp_key(fkey(y), comp_idx(xc));
}

FIE_DEV float cand_rs(float s) { return (s != 1.0f && s >= 0x1p-30f && s <= 0x1p30f) ? 1.0f / s : 0.0f; }

// Q held y-domain composites per thread (those with ok set): the largest is tracked;
// those whose key exceeds `safe` join S.cand (at most kGCap stored, all counted in
// S.n: one LDS atomic per wave) and, with `bins`, the count and float mass of their
// d-bin.  Called by whole waves.
template <int Q>
FIE_DEV void cand_commit(FinSmem& S, const uint64_t (&cv)[Q], const bool (&ok)[Q], uint32_t safe,
                         uint64_t& best, bool bins, float M)
{
    uint32_t keep = 0, k = 0;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        if (ok[q]) best = cv[q] > best ? cv[q] : best;
        if (ok[q] && comp_k(cv[q]) > safe) {
            keep |= 1u << q;
            ++k;
        }
    }
    uint32_t wt;
    uint32_t at = dwave_excl_scan_u32(k, &wt);
    if (wt == 0) return;                          // uniform
    uint32_t base = 0;
    if ((threadIdx.x & 63) == 0) base = atomicAdd(&S.n, wt);
    at += (uint32_t)__shfl((int)base, 0, 64);
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        if (!((keep >> q) & 1u)) continue;
        if (at < (uint32_t)kGCap) S.cand[at] = cv[q];
        ++at;
        if (bins) {
            const float y = key_to_float(comp_k(cv[q]));
            const int b = dbin_y(M, y);
            atomicAdd(&S.pc[b], 1u);
            atomicAdd(&S.pmf[b], approx_mass(y, M));
        }
    }
}

// The first sweep of a two-sweep commit: the held composites above `safe` are
// counted (S.n, one LDS atomic per wave) and binned by d-bin (count, and float mass
// when `mass`), the largest tracked; nothing is stored.  Called by whole waves.
template <int Q>
FIE_DEV void cand_count(FinSmem& S, const uint64_t (&cv)[Q], const bool (&ok)[Q], uint32_t safe,
                        uint64_t& best, bool mass, float M)
{
    uint32_t k = 0;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        if (!ok[q]) continue;
        best = cv[q] > best ? cv[q] : best;
        if (comp_k(cv[q]) > safe) {
            ++k;
            const float y = key_to_float(comp_k(cv[q]));
            const int b = dbin_y(M, y);
            atomicAdd(&S.pc[b], 1u);
            if (mass) atomicAdd(&S.pmf[b], approx_mass(y, M));
        }
    }
    const uint32_t wk = wave_sum_u32(k);
    if ((threadIdx.x & 63) == 0 && wk) atomicAdd(&S.n, wk);
}

// Tiles t0 + w + kFinWaves q (q < Q) of the row, and token 0 (composite z0) on the
// last thread when `with0`: load, convert, commit.
template <int Q>
FIE_DEV void cand_batch(FinSmem& S, const KParams& P, int row, int NT, int t0, float s, uint32_t safe,
                        uint64_t& best, bool bins, float M, bool with0, uint64_t z0)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint64_t cv[Q + 1];
    bool ok[Q + 1];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        const int t = t0 + wave + kFinWaves * q;
        ok[q] = t < NT && (uint32_t)lane < S.nc[t];
        cv[q] = ok[q] ? P.w.cand[((size_t)row * NT + t) * kCapW + lane] : 0ull;
    }
    const float rs = cand_rs(s);
#pragma unroll
    for (int q = 0; q < Q; ++q) cv[q] = ok[q] ? cand_y(cv[q], s, rs) : 0ull;
    ok[Q] = with0 && tid == kFinThreads - 1;
    cv[Q] = z0;
    cand_commit(S, cv, ok, safe, best, bins, M);
}

// The row's candidates from every tile, token 0 (the last thread) included: those
// whose key exceeds `safe` into S.cand in any order, at most kGCap of them.  Returns
// how many there are (possibly more than were stored); S.cmax receives the largest
// composite of all.  Needs S.nc.
FIE_DEV int load_candidates(FinSmem& S, const KParams& P, int row, int NT, float s, uint32_t k0, uint32_t safe)
{
    const int tid = threadIdx.x;
    if (tid == 0) { S.n = 0; S.cmax = 0; }
    __syncthreads();
    uint64_t best = 0;
    for (int t0 = 0; t0 < NT; t0 += kFinWaves * kReloadQ)
        cand_batch<kReloadQ>(S, P, row, NT, t0, s, safe, best, false, 0.0f, t0 == 0, comp_key(k0, 0));
    best = wave_max_u64(best);
    if ((tid & 63) == 0 && best) atomicMax((unsigned long long*)&S.cmax, (unsigned long long)best);
    __syncthreads();
    const int m = (int)S.n;
    __syncthreads();
    return m;
}

FIE_DEV float wave_incl_scan_f32(float v)
{
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const float u = __shfl_up(v, d, 64);
        if (lane >= d) v += u;
    }
    return v;
}

// narrow_candidates for a row binned as its candidates were taken (S.pc counts,
// S.pmf float masses): the count criterion is exact; the mass criterion asks the
// float prefix to exceed g by a margin (2^-9 relative, 2^-26 absolute, in units of
// 2^80) that covers the float sums' rounding and the floors of rule R1, so the
// prefix it picks holds exact mass above g.  Should a crossing still fall past the
// prefix, the exact selection finds no element there and reloads every candidate.
// The last d-bin a narrowed prefix must keep, from the bins' counts (S.pc) and,
// with use_mass, float masses (S.pmf): the bin where the running count reaches
// cnt (cnt > 0) and the bin where the float prefix first exceeds g by the margin
// described above, the later of the two; -1 when either is not found
// (no narrowing).
FIE_DEV int binned_bound(FinSmem& S, int cnt, bool use_mass, u128 g)
{
    constexpr int per = kPassBins / kFinThreads;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float target = (float)(u128_to_double(g) * 0x1p-80 * (1.0 + 0x1p-9) + 0x1p-26);
    uint32_t c[per], cs = 0;
    float m[per], ms = 0.0f;
#pragma unroll
    for (int q = 0; q < per; ++q) {
        c[q] = S.pc[tid * per + q];
        m[q] = use_mass ? S.pmf[tid * per + q] : 0.0f;
        cs += c[q];
        ms += m[q];
    }
    const uint32_t ci = wave_incl_scan_u32(cs);
    const float mi = wave_incl_scan_f32(ms);
    if (lane == 63) {
        S.red32[wave] = ci;
        S.red32[kFinWaves + wave] = __float_as_uint(mi);
    }
    if (tid == 0) {
        S.ibin = cnt > 0 ? -1 : 0;
        S.flag = use_mass ? -1 : 0;
        S.bcnt = 0;
    }
    __syncthreads();
    uint32_t cb = ci - cs;
    float mb = mi - ms;
    float mall = 0.0f;
    for (int w = 0; w < kFinWaves; ++w) {
        if (w < wave) {
            cb += S.red32[w];
            mb += __uint_as_float(S.red32[kFinWaves + w]);
        }
        mall += __uint_as_float(S.red32[kFinWaves + w]);
    }
    // every candidate's mass together is below g, beyond the float sums' error: the
    // crossing lies past the candidates
    const bool beyond = use_mass &&
        (double)mall * (1.0 + 0x1p-9) + 0x1p-26 < u128_to_double(g) * 0x1p-80 * (1.0 - 0x1p-40);
    uint32_t crun = cb;
    float mrun = mb;
#pragma unroll
    for (int q = 0; q < per; ++q) {
        const int b = tid * per + q;
        if (cnt > 0 && crun < (uint32_t)cnt && crun + c[q] >= (uint32_t)cnt) S.ibin = b;
        if (use_mass && !(mrun > target) && mrun + m[q] > target) atomicMax(&S.flag, b);
        crun += c[q];
        mrun += m[q];
    }
    __syncthreads();
    const int bc = S.ibin, bm = S.flag;
    __syncthreads();
    if (beyond) return -2;
    return (bc < 0 || bm < 0) ? -1 : (bc > bm ? bc : bm);
}

FIE_DEV int narrow_binned(FinSmem& S, int nv, float M, int cnt, u128 g)
{
    const int tid = threadIdx.x;
    const int bs = binned_bound(S, cnt, true, g);
    if (bs == -2) return -1;                     // the crossing lies past every candidate
    if (bs < 0) return nv;
    constexpr int kStage = kChunk / 2;           // S.cnt holds this many composites
    uint64_t* tmp = (uint64_t*)S.cnt;
    for (int i = tid; i < nv; i += kFinThreads) {
        const uint64_t x = S.cand[i];
        if (dbin_key(M, comp_k(x)) <= bs) {
            const uint32_t at = atomicAdd(&S.bcnt, 1u);
            if (at < (uint32_t)kStage) tmp[at] = x;
        }
    }
    __syncthreads();
    const int k = (int)S.bcnt;
    if (k > kStage || k >= nv) return nv;
    for (int i = tid; i < k; i += kFinThreads) S.cand[i] = tmp[i];
    __syncthreads();
    return k;
}

// ---------------------------------------------------------------- sorted candidates
constexpr int kSortMax = kGCap;    // candidates sorted in LDS, at most
constexpr int kNarrowRegs = 128;   // two-sweep commits narrow from this many candidates on
constexpr int kRankSort = 256;     // up to this many sort by rank (two or more threads each), more by bitonic merges

// v of lane (lane ^ J): DPP moves inside rows of 16 lanes (quad permutes for 1 and
// 2, row shifts by 4 and 8 selected by the lane's bit), a swizzle inside 32 lanes
// for 16, a permute for 32.
template <int J>
FIE_DEV uint32_t lane_xor_u32(uint32_t v)
{
    const int lane = threadIdx.x & 63;
    if constexpr (J == 1) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);
    } else if constexpr (J == 2) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);
    } else if constexpr (J == 4 || J == 8) {
        const uint32_t up = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x100 | J, 0xF, 0xF, false);
        const uint32_t dn = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x110 | J, 0xF, 0xF, false);
        return (lane & J) ? dn : up;
    } else if constexpr (J == 16) {
        return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x401F);
    } else {
        return (uint32_t)__shfl_xor((int)v, 32, 64);
    }
}

// One compare-exchange stage of stride J < 64 for block size k over a lane's two
// elements e0 = base + lane, e1 = e0 + 64 (descending: the lower index of a pair
// keeps the larger value where (index & k) == 0).
template <int J>
FIE_DEV void bitonic_stage(uint64_t& v0, uint64_t& v1, int e0, int e1, int k)
{
    const int lane = threadIdx.x & 63;
    const uint32_t a = lane_xor_u32<J>((uint32_t)v0), b = lane_xor_u32<J>((uint32_t)(v0 >> 32));
    const uint32_t c = lane_xor_u32<J>((uint32_t)v1), d = lane_xor_u32<J>((uint32_t)(v1 >> 32));
    const uint64_t p0 = ((uint64_t)b << 32) | a, p1 = ((uint64_t)d << 32) | c;
    const bool lower = (lane & J) == 0;
    const bool max0 = lower == ((e0 & k) == 0), max1 = lower == ((e1 & k) == 0);
    v0 = max0 ? (v0 > p0 ? v0 : p0) : (v0 < p0 ? v0 : p0);
    v1 = max1 ? (v1 > p1 ? v1 : p1) : (v1 < p1 ? v1 : p1);
}

// One 128-element block of a descending bitonic sort inside one wave (lane holds
// elements base + lane and base + 64 + lane): for each block size k in [k0, k1],
// the compare-exchange stages of stride min(k / 2, 64) down to 1.  Stride 64 pairs
// a lane's own two elements; smaller strides pair lanes (bitonic_stage).
FIE_DEV void wave_bitonic(uint64_t* c, int base, int k0, int k1)
{
    const int lane = threadIdx.x & 63;
    const int e0 = base + lane, e1 = base + 64 + lane;
    uint64_t v0 = c[e0], v1 = c[e1];
    for (int k = k0; k <= k1; k <<= 1) {
        const int jm = k >> 1 < 64 ? k >> 1 : 64;
        if (jm >= 64) {
            const bool desc = (e0 & k) == 0;
            const uint64_t hi = v0 > v1 ? v0 : v1, lo = v0 > v1 ? v1 : v0;
            v0 = desc ? hi : lo;
            v1 = desc ? lo : hi;
        }
        if (jm >= 32) bitonic_stage<32>(v0, v1, e0, e1, k);
        if (jm >= 16) bitonic_stage<16>(v0, v1, e0, e1, k);
        if (jm >= 8) bitonic_stage<8>(v0, v1, e0, e1, k);
        if (jm >= 4) bitonic_stage<4>(v0, v1, e0, e1, k);
        if (jm >= 2) bitonic_stage<2>(v0, v1, e0, e1, k);
        bitonic_stage<1>(v0, v1, e0, e1, k);
    }
    c[e0] = v0;
    c[e1] = v1;
}

// Sorts S.cand[0, n) descending (n <= kSortMax; composites are distinct), padding
// with 0 to a power of two of at least 128.  Strides below 128 run inside waves;
// only the larger strides of the merges take a barrier each.
FIE_DEV void sort_desc(FinSmem& S, int n)
{
    const int tid = threadIdx.x, wave = tid >> 6;
    if (n <= kRankSort) {
        // a rank sort: each composite's place is the number of larger ones (they are
        // distinct), counted over broadcast LDS reads by F threads per composite, each
        // over one F-th of the list; partial counts meet in S.pc
        int np = 64;
        while (np < n) np <<= 1;
        const int F = kFinThreads / np;
        const int i = tid & (np - 1), h = tid / np;
        const bool have = i < n;
        const uint64_t e = have ? S.cand[i] : 0ull;
        const int part = ((n + F - 1) / F + 1) & ~1;          // even: 16-byte reads stay aligned
        const int jlo = min(h * part, n), jhi = min(jlo + part, n);
        uint32_t r = 0;
        if (have) {
            int j = jlo;
            for (; j + 8 <= jhi; j += 8) {
                ulonglong2 p[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) p[u] = *(const ulonglong2*)&S.cand[j + 2 * u];
#pragma unroll
                for (int u = 0; u < 4; ++u) r += (p[u].x > e ? 1u : 0u) + (p[u].y > e ? 1u : 0u);
            }
            for (; j < jhi; ++j) r += S.cand[j] > e ? 1u : 0u;
            if (h) S.pc[tid] = r;
        }
        __syncthreads();
        if (have && !h) {
            for (int k = 1; k < F; ++k) r += S.pc[k * np + i];
            S.cand[r] = e;
        }
        for (int k = n + tid; k < 128; k += kFinThreads) S.cand[k] = 0;   // as the merge sort pads
        __syncthreads();
        return;
    }
    int N = 128;
    while (N < n) N <<= 1;
    for (int i = n + tid; i < N; i += kFinThreads) S.cand[i] = 0;
    __syncthreads();
    for (int b = wave * 128; b < N; b += kFinThreads * 2) wave_bitonic(S.cand, b, 2, 128);
    for (int k = 256; k <= N; k <<= 1) {
        for (int j = k >> 1; j >= 128; j >>= 1) {
            __syncthreads();
            for (int i = tid; i < N / 2; i += kFinThreads) {
                const int a0 = ((i & ~(j - 1)) << 1) | (i & (j - 1)), b0 = a0 + j;
                const uint64_t x = S.cand[a0], y = S.cand[b0];
                if ((x < y) == ((a0 & k) == 0)) {
                    S.cand[a0] = y;
                    S.cand[b0] = x;
                }
            }
        }
        __syncthreads();
        for (int b = wave * 128; b < N; b += kFinThreads * 2) wave_bitonic(S.cand, b, k, k);
    }
    __syncthreads();
}

// One thread's chunk [lo, hi) of the sorted candidates S.cand[0, nv): the mass
// before it (base) and of it (sum), and over the whole list the survivors' (key >=
// tau, a prefix) count and mass.  One barrier; it also sets S.ibin and S.flag to -1
// for the sorted_find calls that follow.
struct SortedScan {
    int lo, hi;
    u128 base, sum;
    u128 Sv;
    int ns;
};

FIE_DEV SortedScan sorted_scan(FinSmem& S, int nv, uint32_t tau)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int E = (nv + kFinThreads - 1) / kFinThreads;
    SortedScan r;
    r.lo = min(tid * E, nv);
    r.hi = min(r.lo + E, nv);
    u128 sum = 0, vsum = 0;
    uint32_t vcnt = 0;
    for (int i = r.lo; i < r.hi; ++i) {
        const uint64_t c = S.cand[i];
        const u128 w = comp_weight(S, c);
        sum += w;
        if (comp_k(c) >= tau) {
            vsum += w;
            ++vcnt;
        }
    }
    const u128 incl = wave_incl_scan_u128(sum);
    if (tau != 0) {                                   // uniform; tau == 0: every candidate survives
        const u128 vw = wave_sum_u128(vsum);
        const uint32_t vc = wave_sum_u32(vcnt);
        if (lane == 63) {
            S.red128[kFinWaves + wave] = vw;
            S.red32[wave] = vc;
        }
    }
    if (lane == 63) S.red128[wave] = incl;
    if (tid == 0) {
        S.ibin = -1;
        S.flag = -1;
    }
    __syncthreads();
    u128 before = 0, sv = 0;
    uint32_t ns = 0;
    for (int w = 0; w < kFinWaves; ++w) {
        if (w < wave) before += S.red128[w];
        if (tau != 0) {
            sv += S.red128[kFinWaves + w];
            ns += S.red32[w];
        } else {
            sv += S.red128[w];
        }
    }
    if (tau == 0) ns = (uint32_t)nv;
    r.base = before + incl - sum;
    r.sum = sum;
    r.Sv = sv;
    r.ns = (int)ns;
    return r;
}

// The first sorted candidate whose inclusive prefix mass exceeds g, published by
// the thread whose chunk holds it into *slot_i (left at -1 when none does) and its
// prefix into *slot_m; read them after a barrier.
FIE_DEV void sorted_find(FinSmem& S, const SortedScan& sc, u128 g, int* slot_i, u128* slot_m)
{
    if (sc.lo < sc.hi && sc.base <= g && g < sc.base + sc.sum) {
        u128 run = sc.base;
        for (int i = sc.lo; i < sc.hi; ++i) {
            run += comp_weight(S, S.cand[i]);
            if (run > g) {
                *slot_i = i;
                *slot_m = run;
                break;
            }
        }
    }
}

// ---------------------------------------------------------------- k_finish, k_deep
// One row's finish.  PH 0 (k_finish) settles every row its candidates can settle
// and queues the others for PH 1 (k_deep), which runs the passes over the whole
// row: the full-row draw, and top-L logprobs deeper than the candidates.  Both
// phases compute the same prologue (row maximum, tile table, row mass) from the
// partials; a queued row's DeferRec carries what PH 1 cannot recompute cheaply.
template <int DT, bool VEC, int PH, int Q>
FIE_DEV void finish_row(FinSmem& S, const KParams& P, const int row, const bool inl, const bool hd = false)
{
    const fie_sampler_args& a = P.a;
    const int tid = threadIdx.x, NT = P.NT;
    const int32_t fl = a.flags[row];
    const bool greedy = fl & FIE_FLAG_GREEDY;
    const int lp = a.logprobs ? a.logprobs[row] : -1;
    const bool pen = a.apply_penalties && (fl & FIE_FLAG_PENALTY);
    const int topk = greedy ? 0 : a.top_k[row];
    const float tp = greedy ? 1.0f : a.top_p[row];
    const float mp = greedy ? 0.0f : a.min_p[row];
    const float s = greedy ? 1.0f : a.scale[row];
    const bool need_mass = lp >= 0 || (!greedy && topk == 0);
    float rep = 1.0f, pres = 0.0f, freq = 0.0f;
    if (pen) { rep = a.repetition[row]; pres = a.presence[row]; freq = a.frequency[row]; }
    // the row's draw: on-device counter-based, or the caller's
    const double urow = greedy ? 0.0 : (a.rng ? philox_uniform(a.rng + 3 * (size_t)row) : a.uniform[row]);
    int32_t status = 0;
    if (pen && P.w.bad[row] && !a.hist_invalid) status |= FIE_ROW_UNCOUNTED_IDS;

    // Every per-tile partial this row reads, loaded together up front: the tile
    // maxima, sums, candidate counts and bounds, token 0's logit and count, and in
    // PH 0 the candidate slots of the first kFinWaves * Q tiles (a tile's count
    // arrives with them, so all its slots are read and the invalid ones dropped).
    const bool need_cand = !greedy || lp > 0;
    const int lane = tid & 63, wave = tid >> 6;
    const size_t tbase = (size_t)row * NT + tid;
    const uint64_t pf_max = tid < NT ? P.w.maxc[tbase] : 0ull;
    const uint64_t pf_sw = (need_mass && tid < NT) ? P.w.sw[tbase] : 0ull;
    const uint32_t pf_nc = (need_cand && tid < NT) ? P.w.ncand[tbase] : 0u;
    const uint32_t pf_bd = (need_cand && tid < NT) ? P.w.bound[tbase] : 0u;
    const float x0 = P.w.tok0x[row];
    const uint32_t c0 = pen ? P.w.tok0c[row] : 0u;
    const bool spec = PH == 0 && need_cand;
    // rows narrowed by mass (no top-k, no min-p) bin their candidates as they are taken
    const bool bins = spec && !greedy && topk == 0 && !(mp > 0.0f);
    // rows narrowed by count (top-k, top-L) whose every tile's slots are held in
    // registers commit their candidates in two sweeps: count and bin them, then
    // store only the narrowed prefix (for rows narrowed by mass, committing all and
    // compacting measured faster)
    const bool regs = spec && !bins && NT <= kFinWaves * Q;
    if (bins || regs) {
        for (int i = tid; i < kPassBins; i += kFinThreads) {
            S.pc[i] = 0;
            S.pmf[i] = 0.0f;
        }
    }
    uint64_t xs[Q + 1];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        const int t = wave + kFinWaves * q;
        xs[q] = spec && t < NT ? P.w.cand[((size_t)row * NT + t) * kCapW + lane] : 0ull;
    }
    // Round 1: the row maximum, the safety bound and the candidate count, per wave.
    {
        const uint64_t wm = wave_max_u64(pf_max);
        const uint32_t wb = wave_max_u32(pf_bd);
        const uint32_t wn = wave_sum_u32(pf_nc);
        if (tid < NT) S.nc[tid] = pf_nc;
        if (lane == 0) {
            S.red64[wave] = wm;
            S.red64[kFinWaves + wave] = ((uint64_t)wb << 32) | wn;
        }
        if (tid == 0) {
            S.n = 0;
            S.cmax = 0;
            if (PH == 0) S.dmode = 0;            // PH 1 in place: the caller has read it
        }
    }
    __syncthreads();
    uint64_t xm = 0;
    uint32_t kx = 0, ncall = 0;
    for (int w = 0; w < kFinWaves; ++w) {
        xm = S.red64[w] > xm ? S.red64[w] : xm;
        const uint64_t bn = S.red64[kFinWaves + w];
        kx = (uint32_t)(bn >> 32) > kx ? (uint32_t)(bn >> 32) : kx;
        ncall += (uint32_t)bn;
    }

    // Token 0 (a tile of its own).
    float w0 = x0;
    if (c0 && q1_keeps(S, P, row)) w0 = penalize(x0, rep, pres, freq, c0);
    const float y0 = s == 1.0f ? w0 + 0.0f : scaled(w0, s);
    const uint32_t k0 = fkey(y0);

    // Row maximum M of y and the tile table of rule R1: thread t for tile t (slot
    // t + 1), the last thread for token 0 (slot 0); each slot's share of the row
    // mass (rule R1: C_t times the tile sum of weights) summed per wave.
    const uint32_t kxm = xm ? fkey(y_of_xkey(comp_k(xm), s)) : 0u;
    const uint32_t Mkey = kxm > k0 ? kxm : k0;
    const float M = key_to_float(Mkey);
    {
        u128 part = 0;
        const bool z = tid == kFinThreads - 1;
        if (tid < NT || z) {
            float mt;
            uint64_t ct;
            if (z) {
                mt = y0;
                ct = fixed40(cexp(y0 - M));
            } else {
                mt = pf_max ? y_of_xkey(comp_k(pf_max), s) : 0.0f;
                ct = pf_max ? fixed40(cexp(mt - M)) : 0ull;
            }
            const int slot = z ? 0 : tid + 1;
            S.mt[slot] = mt;
            S.ct[slot] = ct;
            P.w.mt[(size_t)row * (NT + 1) + slot] = mt;
            P.w.ct[(size_t)row * (NT + 1) + slot] = ct;
            if (need_mass) part = z ? (u128)tok_weight(y0, y0) * ct : (u128)ct * pf_sw;
        }
        if (need_mass) {
            part = wave_sum_u128(part);
            if (lane == 0) S.red128[wave] = part;
        }
    }

    // The safety key: every token whose scaled key exceeds it is a candidate.
    uint32_t safe = 0;
    if (kx <= 1u || kx <= kKeyNegInf) safe = 0;
    else if (kx > kKeyPosInf) safe = 0xFFFFFFFFu;
    else safe = fkey(y_of_xkey(kx, s));

    // PH 0: the candidates as y-domain composites, those above the safety key into
    // S.cand (binned when narrowed by mass); tiles past the held ones load now.
    bool okr[Q + 1];             // the held slots, for the second sweep
    if (spec) {
        uint64_t best = 0;
        {
            const float rs = cand_rs(s);
#pragma unroll
            for (int q = 0; q < Q; ++q) {
                const int t = wave + kFinWaves * q;
                okr[q] = t < NT && (uint32_t)lane < S.nc[t];
                xs[q] = okr[q] ? cand_y(xs[q], s, rs) : 0ull;
            }
            okr[Q] = tid == kFinThreads - 1;
            xs[Q] = comp_key(k0, 0);
            if (regs) cand_count(S, xs, okr, safe, best, bins, M);
            else cand_commit(S, xs, okr, safe, best, bins, M);
        }
        if (!regs)
            for (int t0 = kFinWaves * Q; t0 < NT; t0 += kFinWaves * Q)
                cand_batch<Q>(S, P, row, NT, t0, s, safe, best, bins, M, false, 0ull);
        best = wave_max_u64(best);
        if (lane == 0 && best) atomicMax((unsigned long long*)&S.cmax, (unsigned long long)best);
    }
    // Round 2: the row mass and the candidates.
    __syncthreads();
    u128 sall = 0;
    if (need_mass)
        for (int w = 0; w < kFinWaves; ++w) sall += S.red128[w];

    int64_t token = -1;
    uint64_t tok_comp = 0;   // y-domain composite of the chosen token
    uint32_t tau = 0;
    uint64_t cut = 0;
    u128 T = 0;
    bool deep = false;
    double lse = 0.0;
    DeferRec dr{};
    if (PH == 1) dr = inl ? S.dfr : P.w.dfr[row];
    // PH 0: hand the row to the full-row path with what is settled so far: in place
    // (inl: the caller runs PH 1 next, the record in LDS) or queued for k_deep
    auto defer = [&](uint32_t mode) {
        if (tid == 0) {
            DeferRec d;
            d.tok_comp = tok_comp;
            d.cut = cut;
            d.tlo = (uint64_t)T;
            d.thi = (uint64_t)(T >> 64);
            d.token = token;
            d.tau = tau;
            d.mode = mode;
            S.dmode = mode;
            if (inl) {
                S.dfr = d;
            } else {
                P.w.dfr[row] = d;
                const uint32_t at = atomicAdd(&P.w.dq[0], 1u);
                if (at < (uint32_t)a.rows) P.w.dqrows[at] = (uint32_t)row;
            }
        }
    };
    if (lp >= 0) lse = log(u128_to_double(sall)) - 80.0 * 0.69314718055994530942;

    // Greedy rows: argmax, first index on ties (sampler.py:106,236-238).
    if (greedy) {
        const uint64_t best = xm > comp_key(k0, 0) ? xm : comp_key(k0, 0);
        token = comp_idx(best);
        tok_comp = best;
        T = comp_weight(S, best);
    }

    // Candidates as y-domain composites, sorted: every token whose scaled key
    // exceeds `safe` is among them.
    int n = need_cand ? (int)ncall + 1 : 0;   // candidates, token 0 included
    int nv = 0;              // those above the safety key (sorted)
    int nvall = 0;           // nv before narrowing to a prefix
    uint64_t cmax = 0;       // the largest candidate composite
    bool sorted = false;
    if (need_cand) {
        if (PH == 1) {
            // the row was queued: its candidates are reloaded below only for logprobs
            deep = dr.mode == kDeferDraw;
        } else {
        nv = (int)S.n;
        cmax = S.cmax;


        if (nv > kSortMax) {
            deep = true;
        } else {
            // what the selections below can reach: top-k and top-L by count; a
            // top-p cut (over the whole row: no top-k, no min-p) or a plain draw by
            // mass; min-p rows sort every candidate
            const int L = lp > 0 ? (lp < a.lp_cols ? lp : a.lp_cols) : 0;
            int cnt = L;
            bool by_mass = false;
            u128 g = 0;
            bool narrow = nv > 384;
            if (!greedy) {
                if (mp > 0.0f) narrow = false;
                else if (topk > 0) cnt = topk > cnt ? topk : cnt;
                else if (tp < 1.0f) { by_mass = true; g = ceil_mul_f32(tp, sall) - 1; }
                else { by_mass = true; g = floor_mul_f64(urow, sall); }
                if (by_mass && sall == 0) narrow = false;
            }
            nvall = nv;
            if (regs) {
                // second sweep: only the composites in bins up to the bound the
                // selections can reach go to S.cand (narrowing is cheap here, so
                // rows narrow from kNarrowRegs candidates on)
                int bs = kPassBins;
                if (nv > kNarrowRegs && (cnt > 0 || by_mass) && !(mp > 0.0f) && !(by_mass && sall == 0)) {
                    const int b = binned_bound(S, cnt, by_mass, g);
                    if (b >= 0) bs = b;
                }
                if (tid == 0) S.n = 0;
                __syncthreads();
                bool ok2[Q + 1];
#pragma unroll
                for (int q = 0; q <= Q; ++q)
                    ok2[q] = okr[q] && (bs >= kPassBins || dbin_key(M, comp_k(xs[q])) <= bs);
                uint64_t unused = 0;
                cand_commit(S, xs, ok2, safe, unused, false, M);
                __syncthreads();
                nv = (int)S.n;
                __syncthreads();
            } else if (narrow && (cnt > 0 || by_mass)) {
                nv = by_mass ? narrow_binned(S, nv, M, cnt, g) : narrow_candidates(S, nv, M, cnt, false, g);
            }

            if (nv < 0) {
                deep = true;                     // no need to sort what cannot settle the row
                nv = 0;
            } else {
                sort_desc(S, nv);
                sorted = true;
            }
        }
        }
    }
    if (PH == 1 && dr.mode == kDeferLogprobs) {
        token = dr.token;
        tok_comp = dr.tok_comp;
        tau = dr.tau;
        cut = dr.cut;
        T = ((u128)dr.thi << 64) | dr.tlo;
    }

    // Sampled rows on the sorted candidates: top-k, min-p, S, top-p cut, draw.  The
    // narrowed prefix holds every crossing by construction; should a cut or draw
    // still miss it, that is not a verdict: every candidate is then loaded and
    // sorted and the selection runs again.
    if (PH == 0 && !greedy && !deep) {
        for (;;) {
            const bool partial = nv < nvall;
            bool miss = false;
            uint32_t tk = 0;
            if (topk > 0) {
                // the top-k threshold lies in the complete region iff it holds topk
                if (nv < topk) deep = true;
                else tk = comp_k(S.cand[topk - 1]);
            }
            const uint32_t tmp = minp_key(M, mp);
            tau = tk > tmp ? tk : tmp;
            if (!deep && tau != 0 && tau <= safe) deep = true;
            if (!deep) {
                // survivors (key >= tau) and the complete region (key > safe) are
                // prefixes of the sorted candidates; with tau != 0 the survivors lie in it
                const SortedScan sc = sorted_scan(S, nv, tau);
                const int ns = tau != 0 ? sc.ns : nv;
                const u128 Sv = tau != 0 ? sc.Sv : sall;
                int lim = ns;
                cut = 0;
                if (tp < 1.0f) {
                    const u128 thr = ceil_mul_f32(tp, Sv);
                    sorted_find(S, sc, thr - 1, &S.ibin, &S.bex);
                    __syncthreads();
                    const int i = S.ibin;
                    if (i < 0 || i >= lim) (partial ? miss : deep) = true;
                    else { cut = S.cand[i]; T = S.bex; lim = i + 1; }
                } else {
                    T = Sv;
                }
                if (!deep && !miss) {
                    if (T == 0) {
                        token = comp_idx(cmax);
                        tok_comp = cmax;
                    } else {
                        const u128 g = floor_mul_f64(urow, T);
                        sorted_find(S, sc, g, &S.flag, &S.bme);
                        __syncthreads();
                        const int i = S.flag;
                        if (i < 0 || i >= lim) (partial ? miss : deep) = true;
                        else { token = comp_idx(S.cand[i]); tok_comp = S.cand[i]; }
                    }
                }
            }
            if (!deep && !miss && a.tk_key && tid == 0) a.tk_key[row] = tk;
            if (!miss) break;
            nv = load_candidates(S, P, row, NT, s, k0, safe);
            nvall = nv;
            sort_desc(S, nv);
        }
    }

    // Full-row path for sampled rows the candidates could not settle.
    if (PH == 0 && !greedy && deep) {
        defer(kDeferDraw);
        return;
    }
    if (PH == 1 && !greedy && deep) {
        status |= FIE_ROW_EXACT_PATH;
        cut = 0;
        uint32_t tk = 0;
        const bool binned = binned_deep<DT, VEC>(S, P, row, s, pen, rep, pres, freq, k0, M, topk, mp, tp,
                                                 urow, sall, &tk, &tau, &cut, &T, &tok_comp, hd);
        if (!binned) {
        // radix levels over the composite, re-reading the row per level
        cut = 0;
        tk = 0;
        if (topk > 0) {
            const SelResult r = row_select<DT, VEC, false>(S, P, row, s, pen, rep, pres, freq, k0,
                                                           Pred{0, 0, 0}, (u128)(topk - 1), false);
            tk = comp_k(r.comp);
        }
        const uint32_t tmp = minp_key(M, mp);
        tau = tk > tmp ? tk : tmp;
        const Pred surv{tau, 0, 0};
        pass_hist<DT, VEC, true>(S, P, row, s, pen, rep, pres, freq, k0, surv, 0, 0);
        u128 part = 0;
        for (int b = tid; b < kPassBins; b += kFinThreads)
            part += ((u128)S.pm_hi[b] << 64) | S.pm_lo[b];
        const u128 Sv = block_sum_u128<kFinThreads>(part, S.red128);
        bool l1 = true;
        if (tp < 1.0f) {
            const u128 thr = ceil_mul_f32(tp, Sv);
            const SelResult r = row_select<DT, VEC, true>(S, P, row, s, pen, rep, pres, freq, k0,
                                                          surv, thr - 1, true);
            cut = r.comp;
            T = r.excl + r.meas;
            l1 = false;
        } else {
            T = Sv;
        }
        if (T == 0) {
            const SelResult r = row_select<DT, VEC, false>(S, P, row, s, pen, rep, pres, freq, k0,
                                                           Pred{0, 0, 0}, 0, false);
            tok_comp = r.comp;
        } else {
            const u128 g = floor_mul_f64(urow, T);
            const SelResult r = row_select<DT, VEC, true>(S, P, row, s, pen, rep, pres, freq, k0,
                                                          Pred{tau, 0, cut}, g, l1);
            tok_comp = r.comp;
        }
        }
        token = comp_idx(tok_comp);
        if (a.tk_key && tid == 0) a.tk_key[row] = tk;
        // the LDS candidates were overwritten: reload them for the logprobs below
        sorted = false;
        if (lp > 0 && n > 0) {
            nv = load_candidates(S, P, row, NT, s, k0, safe);
            if (nv <= kSortMax) {
                sort_desc(S, nv);
                sorted = true;
            }
        }
    }

    // Logprobs (sampler.py:262-291, rule R7): chosen token, then the row's best L,
    // all from the penalised, scaled distribution before filtering.
    if (lp >= 0) {
        if (tid == 0 && a.chosen_logprob)
            a.chosen_logprob[row] = (float)(((double)key_to_float(comp_k(tok_comp)) - (double)M) - lse);
        const int L = lp < a.lp_cols ? lp : a.lp_cols;
        if (L > 0) {
            if (sorted && nv >= L) {
                // the first L sorted candidates
                for (int j = tid; j < a.lp_cols; j += kFinThreads) {
                    const size_t o = (size_t)row * a.lp_cols + j;
                    const bool have = j < L;
                    const uint64_t c = have ? S.cand[j] : 0ull;
                    if (a.top_ids) a.top_ids[o] = have ? (int64_t)comp_idx(c) : -1;
                    if (a.top_logprobs)
                        a.top_logprobs[o] = have ? (float)(((double)key_to_float(comp_k(c)) - (double)M) - lse) : 0.0f;
                }
            } else if (PH == 0) {
                defer(kDeferLogprobs);
                return;
            } else {
                // the L-th largest composite over the row, the L composites >= it
                // gathered, then sorted by one thread
                const SelResult r = row_select<DT, VEC, false>(S, P, row, s, pen, rep, pres, freq, k0,
                                                               Pred{0, 0, 0}, (u128)(L - 1), false);
                n = pass_gather<DT, VEC>(S, P, row, s, pen, rep, pres, freq, k0, Pred{0, 0, r.comp}, 64, 0);
                if (tid == 0) {
                    const int m = n < 32 ? n : 32;
                    uint64_t* top = S.cand;
                    for (int i = 1; i < m; ++i) {
                        const uint64_t c = top[i];
                        int j = i;
                        while (j > 0 && top[j - 1] < c) { top[j] = top[j - 1]; --j; }
                        top[j] = c;
                    }
                    for (int j = 0; j < a.lp_cols; ++j) {
                        const size_t o = (size_t)row * a.lp_cols + j;
                        const bool have = j < m && j < L;
                        if (a.top_ids) a.top_ids[o] = have ? (int64_t)comp_idx(top[j]) : -1;
                        if (a.top_logprobs)
                            a.top_logprobs[o] = have ? (float)(((double)key_to_float(comp_k(top[j])) - (double)M) - lse) : 0.0f;
                    }
                }
            }
        } else if (tid == 0) {
            for (int j = 0; j < a.lp_cols; ++j) {
                const size_t o = (size_t)row * a.lp_cols + j;
                if (a.top_ids) a.top_ids[o] = -1;
                if (a.top_logprobs) a.top_logprobs[o] = 0.0f;
            }
        }
    }

    if (tid == 0) {
        a.tokens[row] = token;
        if (a.status) a.status[row] = status;
        if (a.row_max) a.row_max[row] = M;
        if (a.cut_comp) a.cut_comp[row] = cut;
        if (greedy && a.tk_key) a.tk_key[row] = 0;
        if (a.kept_mass) { a.kept_mass[2 * row] = (uint64_t)T; a.kept_mass[2 * row + 1] = (uint64_t)(T >> 64); }
        if (a.row_mass) { a.row_mass[2 * row] = (uint64_t)sall; a.row_mass[2 * row + 1] = (uint64_t)(sall >> 64); }
        RowRes rr;
        rr.cut = cut;
        rr.klo = (uint64_t)T;
        rr.khi = (uint64_t)(T >> 64);
        rr.tau = tau;
        rr.greedy = greedy ? 1u : 0u;
        rr.token = token;
        rr.M = M;
        rr.s = s;
        P.w.res[row] = rr;
    }
}

// ---------------------------------------------------------------- span helpers
// Batches of at most kHelpRows rows leave most CUs idle, and a row the candidates
// cannot settle would stream all of its tokens through one workgroup.  There,
// k_finish runs one helper workgroup per span of each sampled row beside the
// row's own workgroup.  A helper bins its span's tokens by d = fl(M - y) exactly as
// the full-row pass does (counts and R1 masses per bin) and stores the span's
// composites ordered by bin, so the full-row selection reads one histogram per
// span and gathers a bin from the spans' segments instead of re-reading the row.
// Nobody waits: each of the row's workgroups counts itself in (harr) after its
// stores, and the last to arrive finishes the row if its own workgroup handed it
// to the full-row path.  Rows with a small top-k never take that path.
constexpr int kHelpTopK = 1024;
static_assert(kHBins == kPassBins && kHBins == 2 * kFinThreads, "two bins per thread");

FIE_DEV bool helped_row(const KParams& P, int row)
{
    if (P.a.flags[row] & FIE_FLAG_GREEDY) return false;
    const int k = P.a.top_k[row];
    return k == 0 || k > kHelpTopK;
}

// Counts the workgroup in at the row: `add` is 1, plus kArrDeep from the row's own
// workgroup when it hands the row to the full-row path.  Returns -1, or for the
// last of the row's NS + 1 workgroups whether the row is to be finished (0 / 1).
// A workgroup that publishes (every helper; the row's own one only with a record
// for the full-row path) has each wave wait for its own stores, then one thread
// fences for the workgroup: a device-scope fence per wave costs ~0.2 us each,
// serialised across the helpers, and one that writes back nothing the others need
// only delays the step.  The last one acquires only when the row is to be finished.
constexpr uint32_t kArrDeep = 1u << 16;

FIE_DEV int arrive(FinSmem& S, const KParams& P, int row, uint32_t add, bool publish)
{
    if (publish) __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        if (publish) __threadfence();
        const uint32_t now = atomicAdd(&P.w.harr[row], add) + add;
        const bool last = (now & (kArrDeep - 1)) == (uint32_t)P.NS + 1;
        if (last) {
            P.w.harr[row] = 0u;              // ready for the next call
            if (now >> 16) __threadfence();
        }
        S.ibin = last ? (int)(now >> 16) : -1;
    }
    __syncthreads();
    const int r = S.ibin;
    __syncthreads();
    return r;
}

// Returns true when this workgroup is to finish the row through the full-row path.
template <int DT, bool VEC>
FIE_DEV bool span_helper(FinSmem& S, const KParams& P, const int row, const int sp)
{
    constexpr int EPL = DTy<DT>::EPL, SZ = DTy<DT>::SZ;
    constexpr int NL = kSpan / kFinThreads / EPL;
    const fie_sampler_args& a = P.a;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int NT = P.NT, NS = P.NS, V = a.vocab;
    if (!helped_row(P, row)) return false;
    const int32_t fl = a.flags[row];
    const bool pen = a.apply_penalties && (fl & FIE_FLAG_PENALTY);
    const float s = a.scale[row];
    float rep = 1.0f, pres = 0.0f, freq = 0.0f;
    if (pen) { rep = a.repetition[row]; pres = a.presence[row]; freq = a.frequency[row]; }
    const int lo = sp * kSpan;
    const char* rowp = (const char*)a.logits + (size_t)row * (size_t)a.row_stride * SZ;
    uint4 raw[NL];
#pragma unroll
    for (int j = 0; j < NL; ++j) raw[j] = load_group<DT, VEC>(rowp, lo + (j * kFinThreads + tid) * EPL, V);
    const uint64_t pf_max = tid < NT ? P.w.maxc[(size_t)row * NT + tid] : 0ull;
    const size_t hs = (size_t)row * NS + sp;
    uint32_t nb = 0, of = 0;
    if (pen) {
        nb = P.w.nb[hs];
        of = P.w.bk[hs * kBucketCap + tid];
    }
    uint32_t* cnt = (uint32_t*)S.cand;       // penalty counts of the span's tokens
    for (int i = tid; i < kPassBins; i += kFinThreads) {
        S.pc[i] = 0;
        S.pm_lo[i] = 0;
        S.pm_hi[i] = 0;
    }
    if (pen)
        for (int i = tid; i < kSpan / 4; i += kFinThreads) ((uint4*)cnt)[i] = make_uint4(0, 0, 0, 0);
    {
        const uint64_t wm = wave_max_u64(pf_max);
        if (lane == 0) S.red64[wave] = wm;
    }
    __syncthreads();
    // the row maximum and the span's tiles of the R1 tile table, as the row's own
    // workgroup computes them (token 0 left out: the row's workgroup checks it)
    uint64_t xm = 0;
    for (int w = 0; w < kFinWaves; ++w) xm = S.red64[w] > xm ? S.red64[w] : xm;
    const uint32_t kxm = xm ? fkey(y_of_xkey(comp_k(xm), s)) : 0u;
    const float M = key_to_float(kxm);
    if (tid < NT && tid / kWavesPerWG == sp) {
        const float mt = pf_max ? y_of_xkey(comp_k(pf_max), s) : 0.0f;
        S.mt[tid + 1] = mt;
        S.ct[tid + 1] = pf_max ? fixed40(cexp(mt - M)) : 0ull;
    }
    if (pen) {
        if (nb <= (uint32_t)kBucketCap) {
            if ((uint32_t)tid < nb) atomicAdd(&cnt[of], 1u);
        } else {
            const int64_t h0 = a.hist_offsets[row], h1 = hist_end(a, row);
            const int hi = min(lo + kSpan, V);
            for (int64_t h = h0 + tid; h < h1; h += kFinThreads) {
                const uint32_t id = (uint32_t)a.hist_ids[h];
                if (id >= (uint32_t)lo && id < (uint32_t)hi && id != 0) atomicAdd(&cnt[id - lo], 1u);
            }
        }
    }
    __syncthreads();
    // every token of the span: its bin, count and mass (row_pass's arithmetic)
    const bool mark = s != 1.0f && s >= 0x1p-30f && s <= 0x1p30f;
    const float rs = 1.0f / s;
    uint64_t cv[NL * EPL];
    int bv[NL * EPL];
    // the last bin (d >= 16 and NaN) holds most tokens of a flat or long-tailed row:
    // summed per thread and per wave first, not by same-address LDS atomics
    uint32_t tail_n = 0;
    u128 tail_w = 0;
#pragma unroll
    for (int j = 0; j < NL; ++j) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const int k = j * EPL + e;
            const int idx = lo + (j * kFinThreads + tid) * EPL + e;
            bv[k] = -1;
            cv[k] = 0;
            if (idx >= V || idx == 0) continue;
            float x = lane_get<DT>(raw[j], e);
            if (pen) {
                const uint32_t cc = cnt[idx - lo];
                if (cc) x = penalize(x, rep, pres, freq, cc);
            }
            float y;
            if (s == 1.0f) y = x + 0.0f;
            else if (mark && markstein_ok(x)) y = div_markstein(x, s, rs) + 0.0f;
            else y = scaled(x, s);
            const int b = dbin_y(M, y);
            const u128 w = weight_of(S, y, (uint32_t)idx);
            if (b == kPassBins - 1) {
                ++tail_n;
                tail_w += w;
            } else {
                atomicAdd(&S.pc[b], 1u);
                bin_add(S, b, w);
            }
            bv[k] = b;
            cv[k] = comp_key(fkey(y), (uint32_t)idx);
        }
    }
    tail_n = wave_sum_u32(tail_n);
    tail_w = wave_sum_u128(tail_w);
    if (lane == 0 && tail_n) {
        atomicAdd(&S.pc[kPassBins - 1], tail_n);
        bin_add(S, kPassBins - 1, tail_w);
    }
    __syncthreads();
    // the histogram and the bins' offsets, then the composites in bin order
    const uint32_t ca = S.pc[2 * tid], cb = S.pc[2 * tid + 1];
    {
        const size_t o = hs * kHBins + 2 * tid;
        P.w.hpc[o] = ca;
        P.w.hpc[o + 1] = cb;
        P.w.hlo[o] = S.pm_lo[2 * tid];
        P.w.hlo[o + 1] = S.pm_lo[2 * tid + 1];
        P.w.hhi[o] = S.pm_hi[2 * tid];
        P.w.hhi[o + 1] = S.pm_hi[2 * tid + 1];
    }
    uint32_t total;
    const uint32_t ex = block_excl_scan_u32<kFinThreads>(ca + cb, S.red32, &total);
    S.cnt[2 * tid] = ex;
    S.cnt[2 * tid + 1] = ex + ca;
    {
        uint32_t* off = P.w.hoff + hs * kHOffs;
        off[2 * tid] = ex;
        off[2 * tid + 1] = ex + ca;
        if (tid == 0) {
            off[kHBins] = total;
            P.w.hmk[hs] = fkey(M);
        }
    }
    __syncthreads();
    const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;   // lanes before this one
#pragma unroll
    for (int k = 0; k < NL * EPL; ++k) {
        const bool tail = bv[k] == kPassBins - 1;
        const uint64_t m = __ballot(tail);
        if (m) {
            // the last bin's slots: one LDS atomic per wave, ranks by lane
            const int first = __ffsll((unsigned long long)m) - 1;
            uint32_t base = 0;
            if (lane == first) base = atomicAdd(&S.cnt[kPassBins - 1], (uint32_t)__popcll(m));
            base = (uint32_t)__shfl((int)base, first);
            if (tail) P.w.hcomp[hs * kSpan + base + (uint32_t)__popcll(m & below)] = cv[k];
        }
        if (bv[k] >= 0 && !tail) {
            const uint32_t at = atomicAdd(&S.cnt[bv[k]], 1u);
            P.w.hcomp[hs * kSpan + at] = cv[k];
        }
    }
    return arrive(S, P, row, 1u, true) > 0;
}

// One workgroup per row.  A row's finish is a chain of dependent steps, so its
// latency is the kernel's: with no more rows than CUs (one workgroup each) the WIDE
// variant takes up to 256 registers a lane and spills nothing; larger batches take
// 128 (two workgroups a CU).
template <int DT, bool VEC, bool WIDE>
__global__ __launch_bounds__(kFinThreads, WIDE ? 2 : 4) void k_finish(const KParams P)
{
    __shared__ FinSmem S;
    if constexpr (WIDE) {
        // a row the candidates could not settle takes the full-row path here, at once;
        // with span helpers, in whichever of the row's workgroups arrives last
        bool deep, inl = true, hd = false;
        if (blockIdx.y > 0) {
            deep = span_helper<DT, VEC>(S, P, blockIdx.x, blockIdx.y - 1);
            inl = false;
            hd = true;
        } else {
            finish_row<DT, VEC, 0, 10>(S, P, blockIdx.x, true);
            __syncthreads();
            deep = S.dmode != 0;
            if (P.helpers && helped_row(P, blockIdx.x)) {
                // the record goes out only with a row for the full-row path
                if (deep && threadIdx.x == 0) P.w.dfr[blockIdx.x] = S.dfr;
                deep = arrive(S, P, blockIdx.x, deep ? 1u + kArrDeep : 1u, deep) > 0;
                hd = true;
            }
        }
        if (deep) finish_row<DT, VEC, 1, kReloadQ>(S, P, blockIdx.x, inl, hd);
    } else {
        finish_row<DT, VEC, 0, kReloadQ>(S, P, blockIdx.x, false);
    }
}

// A fixed grid taking queued rows one at a time; every workgroup leaves once the
// queue is drained (the count is final: k_finish has completed).  The queue is
// short in decode (a few rows a step) but holds every row of a flat batch.
template <int DT, bool VEC>
__global__ __launch_bounds__(kFinThreads, 4) void k_deep(const KParams P)
{
    __shared__ FinSmem S;
    const uint32_t queued = P.w.dq[0];
    const uint32_t total = queued < (uint32_t)P.a.rows ? queued : (uint32_t)P.a.rows;
    if (blockIdx.x >= total) return;
    finish_row<DT, VEC, 1, kReloadQ>(S, P, (int)P.w.dqrows[blockIdx.x], false);
}

}  // namespace fie
