// MI355X fused token sampler: kernels and the C ABI (include/fie_sampler.h).
//
// One sampler step for [rows, vocab] logits is at most two launches on the
// caller's stream, with no host synchronisation:
//
//   k_penalty  (rows with penalties)  sampler.py:120-175: per-row distinct history
//              ids, counts and penalised values, sorted by token id, cut into one
//              segment per slice of the row.
//   k_sample   one workgroup per (row, slice).  The slice is read from HBM once
//              into registers, with the slice's penalty patches applied from LDS.
//              Greedy rows need only the row max.  Top-k rows count the keys that
//              can reach the top k into a histogram, agree on the bin of the k-th
//              value and gather every token from that bin up.  Wide rows (sampled,
//              no top-k) agree on the row max, weigh every token exactly, agree on
//              the top-p cut and draw windows from the survivor mass histogram,
//              and gather the tokens in those windows.  The row's last workgroup
//              sorts the candidates and applies the filters and the draw.
//
// All mass sums are 64-bit integer sums of floor(cexp(y - M) * 2^40), so results
// do not depend on how the row is split into workgroups or on atomic order.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <stdlib.h>

#include "common.h"
#include "layout.h"
#include "fie_sampler.h"

namespace fie {

// ============================================================== element access
template <int DT> struct Dt;
template <> struct Dt<FIE_F32> { static constexpr int EPC = 4, ES = 4; };
template <> struct Dt<FIE_F16> { static constexpr int EPC = 8, ES = 2; };
template <> struct Dt<FIE_BF16> { static constexpr int EPC = 8, ES = 2; };

FIE_DEV float half_bits_to_float(uint32_t h)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

template <int DT>
FIE_DEV float load_one(const char* row, int64_t i)
{
    if constexpr (DT == FIE_F32) {
        return ((const float*)row)[i];
    } else if constexpr (DT == FIE_F16) {
        return half_bits_to_float(((const uint16_t*)row)[i]);
    } else {
        return __uint_as_float((uint32_t)((const uint16_t*)row)[i] << 16);
    }
}

// Loads the 16-byte chunk starting at element e0 (fully inside the row).
template <int DT>
FIE_DEV void load_chunk(const char* row, int64_t e0, bool vec_ok, float* v)
{
    constexpr int EPC = Dt<DT>::EPC;
    if (vec_ok) {
        const uint4 raw = *(const uint4*)(row + e0 * Dt<DT>::ES);
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
        if constexpr (DT == FIE_F32) {
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = __uint_as_float(w[j]);
        } else if constexpr (DT == FIE_F16) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[2 * j] = half_bits_to_float(w[j] & 0xFFFFu);
                v[2 * j + 1] = half_bits_to_float(w[j] >> 16);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[2 * j] = __uint_as_float(w[j] << 16);
                v[2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < EPC; ++j) v[j] = load_one<DT>(row, e0 + j);
    }
}

FIE_DEV const char* row_ptr(const Params& P, int r)
{
    return P.logits + (int64_t)r * P.row_stride_bytes;
}

// Slice s of a row covers chunks [s*cps, (s+1)*cps) clipped to the row.
FIE_DEV int64_t slice_begin(const Params& P, int s)
{
    int64_t e = (int64_t)s * P.cps * P.epc;
    return e < P.vocab ? e : P.vocab;
}

// ============================================================== penalty patches
// Penalised values of one slice, staged in LDS: a bitmap over the slice's
// elements and the (sorted) patch list, so the streaming loop tests one LDS word
// per chunk and looks values up only on a hit.
struct PatchLds {
    uint32_t bitmap[kMaxSlice / 32];
    int32_t ids[kPatchLds];    // offsets inside the slice, ascending
    float vals[kPatchLds];
};

struct PatchView {
    int n;                     // patches in this slice
    bool in_lds;
    int64_t e0;                // first element of the slice
    const int32_t* gids;       // global fallback when n > kPatchLds
    const float* gvals;
};

// Whether the row's token-0 patch is undone by the reference's pad writes
// (sampler.py:148,156-157,174-175: index 0 receives the original logit from every
// pad or out-of-vocab entry that comes after the real entry).
FIE_DEV bool token0_patch_dropped(const Params& P, int r)
{
    const PenMeta pm = P.pen[r];
    if (!pm.has0) return false;
    const unsigned long long wb = __hip_atomic_load(P.wbatch, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
    const int width = ((int64_t)(wb >> 32) == (P.epoch & 0xFFFFFFFF)) ? (int)(wb & 0xFFFFFFFFu) : 0;
    return pm.nuniq < width || pm.inval_after0;
}

FIE_DEV PatchView stage_patches(const Params& P, int r, int s, PatchLds& L)
{
    PatchView pv{0, true, slice_begin(P, s), nullptr, nullptr};
    if (!P.apply_pen) return pv;
    const int* seg = P.seg + (int64_t)r * (kMaxSlices + 1);
    const int a = seg[s], b = seg[s + 1];
    pv.n = b - a;
    if (pv.n <= 0) { pv.n = 0; return pv; }
    const int64_t base = P.hist_off[r] + a;
    pv.gids = P.pen_ids + base;
    pv.gvals = P.pen_vals + base;
    pv.in_lds = pv.n <= kPatchLds;
    const int64_t e1 = slice_begin(P, s + 1);
    const int words = (int)((e1 - pv.e0 + 31) / 32);
    for (int i = threadIdx.x; i < words; i += kThreads) L.bitmap[i] = 0;
    __syncthreads();
    const bool drop0 = (s == 0) && token0_patch_dropped(P, r);
    for (int i = threadIdx.x; i < pv.n; i += kThreads) {
        const int id = pv.gids[i];
        const int off = (int)(id - pv.e0);
        if (pv.in_lds) {
            L.ids[i] = off;
            L.vals[i] = pv.gvals[i];
        }
        if (!(drop0 && id == 0)) atomicOr(&L.bitmap[off >> 5], 1u << (off & 31));
    }
    __syncthreads();
    return pv;
}

FIE_DEV float patch_value(const PatchView& pv, const PatchLds& L, int off)
{
    int lo = 0, hi = pv.n - 1;
    if (pv.in_lds) {
        while (lo < hi) {
            int mid = (lo + hi) >> 1;
            if (L.ids[mid] < off) lo = mid + 1; else hi = mid;
        }
        return L.vals[lo];
    }
    const int id = (int)(pv.e0 + off);
    while (lo < hi) {
        int mid = (lo + hi) >> 1;
        if (pv.gids[mid] < id) lo = mid + 1; else hi = mid;
    }
    return pv.gvals[lo];
}

// Applies the patches of one chunk (elements e0..e0+EPC-1 of the row).
template <int EPC>
FIE_DEV void apply_patches(const PatchView& pv, const PatchLds& L, int64_t e0, float* v)
{
    if (pv.n == 0) return;
    const int off = (int)(e0 - pv.e0);
    const uint32_t bits = (L.bitmap[off >> 5] >> (off & 31)) & ((1u << EPC) - 1u);
    if (bits == 0) return;
    // static element indices only, so v[] stays in registers
#pragma unroll
    for (int j = 0; j < EPC; ++j)
        if (bits & (1u << j)) v[j] = patch_value(pv, L, off + j);
}

// Calls f(w, index) for every element of slice s of row r, 16-byte chunks
// distributed round-robin over the workgroup, four chunks in flight per thread.
template <int DT, typename F>
FIE_DEV void for_each_element(const Params& P, int r, int s, const PatchView& pv,
                              const PatchLds& L, F&& f)
{
    constexpr int EPC = Dt<DT>::EPC;
    const char* row = row_ptr(P, r);
    const int64_t nfull = P.vocab / EPC;                 // chunks entirely in the row
    const int64_t c0 = (int64_t)s * P.cps;
    int64_t c1 = c0 + P.cps;
    const int64_t nch = (P.vocab + EPC - 1) / EPC;
    if (c1 > nch) c1 = nch;
    const int64_t cf = c1 < nfull ? c1 : nfull;          // full chunks of this slice
    const bool vec_ok = P.vec_ok;
    int64_t c = c0 + threadIdx.x;
    for (; c + 3 * kThreads < cf; c += 4 * kThreads) {
        float v[4][EPC];
#pragma unroll
        for (int u = 0; u < 4; ++u) load_chunk<DT>(row, (c + u * kThreads) * EPC, vec_ok, v[u]);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t e0 = (c + u * kThreads) * EPC;
            apply_patches<EPC>(pv, L, e0, v[u]);
#pragma unroll
            for (int j = 0; j < EPC; ++j) f(v[u][j], (uint32_t)(e0 + j));
        }
    }
    for (; c < cf; c += kThreads) {
        float v[EPC];
        load_chunk<DT>(row, c * EPC, vec_ok, v);
        apply_patches<EPC>(pv, L, c * EPC, v);
#pragma unroll
        for (int j = 0; j < EPC; ++j) f(v[j], (uint32_t)(c * EPC + j));
    }
    // the partial last chunk of the row
    if (c1 > nfull && c0 <= nfull && threadIdx.x == (int)((nfull - c0) % kThreads)) {
        const int64_t e0 = nfull * EPC;
        float v[EPC];
        for (int j = 0; j < EPC; ++j) v[j] = (e0 + j < P.vocab) ? load_one<DT>(row, e0 + j) : 0.0f;
        apply_patches<EPC>(pv, L, e0, v);
        for (int j = 0; j < EPC; ++j)
            if (e0 + j < P.vocab) f(v[j], (uint32_t)(e0 + j));
    }
}

// Wave-aggregated append of (w bits, index) to a row's candidate buffer.
FIE_DEV void append_candidate(bool pred, float w, uint32_t idx, unsigned int* counter,
                              uint64_t* buf)
{
    const uint64_t mask = __ballot(pred);
    if (mask == 0) return;
    const int lane = threadIdx.x & 63;
    const int leader = __builtin_ctzll(mask);
    unsigned int base = 0;
    if (lane == leader) base = atomicAdd(counter, (unsigned int)__popcll(mask));
    base = __shfl(base, leader, 64);
    if (pred) {
        const unsigned int pos = base + (unsigned int)__popcll(mask & ((1ull << lane) - 1ull));
        if (pos < (unsigned int)kCap)
            st_shared(&buf[pos], ((uint64_t)__float_as_uint(w) << 32) | idx);
    }
}

FIE_DEV int d_bin(float d, float dscale)
{
    float t = -d * dscale;
    t = fminf(t, (float)(kMassBins - 1));
    t = fmaxf(t, 0.0f);
    return (int)t;
}

FIE_DEV int bin_of_key(uint32_t k, float s, float M, float dscale)
{
    const float y = scaled(key_to_float(k), s);
    return d_bin(y - M, dscale);
}

// ============================================================== penalties
// One workgroup of 1024 threads per row.  Dynamic LDS: 2 * words u32.
__global__ __launch_bounds__(kPenThreads) void k_penalty(Params P)
{
    extern __shared__ uint32_t pen_lds[];
    __shared__ int s_p0, s_ninv, s_red[kPenThreads / 64];
    __shared__ int s_inv_pos[256], s_inv_id[256];
    const int r = blockIdx.x;
    const int tid = threadIdx.x;
    const int words = (P.vocab + 31) / 32;
    uint32_t* bits = pen_lds;
    uint32_t* prefix = pen_lds + words;
    int32_t* seg = P.seg + (int64_t)r * (kMaxSlices + 1);
    const int64_t off = P.hist_off[r];
    const int64_t n = P.hist_off[r + 1] - off;
    const bool active = (P.flags[r] & 2) && n > 0;
    if (!active) {
        for (int s = tid; s <= P.S; s += kPenThreads) seg[s] = 0;
        if (tid == 0) P.pen[r] = PenMeta{0, 0, 0, 0};
        return;
    }
    for (int i = tid; i < words; i += kPenThreads) bits[i] = 0;
    if (tid == 0) { s_p0 = 0x7FFFFFFF; s_ninv = 0; }
    __syncthreads();
    const int32_t* ids = P.hist_ids + off;
    for (int64_t j = tid; j < n; j += kPenThreads) {
        const int id = ids[j];
        if (id < P.vocab) {
            atomicOr(&bits[id >> 5], 1u << (id & 31));
            if (id == 0) atomicMin(&s_p0, (int)j);
        } else {
            const int k = atomicAdd(&s_ninv, 1);
            if (k < 256) { s_inv_pos[k] = (int)j; s_inv_id[k] = id; }
        }
    }
    __syncthreads();
    // exclusive rank of each bitmap word: contiguous runs of words per thread
    const int per = (words + kPenThreads - 1) / kPenThreads;
    const int w0 = tid * per;
    int local = 0;
    for (int w = w0; w < w0 + per && w < words; ++w) local += __popc(bits[w]);
    {
        // block exclusive scan of `local`
        const int lane = tid & 63, wave = tid >> 6;
        int incl = local;
        for (int d = 1; d < 64; d <<= 1) {
            int o = __shfl_up(incl, d, 64);
            if (lane >= d) incl += o;
        }
        if (lane == 63) s_red[wave] = incl;
        __syncthreads();
        if (tid == 0) {
            int run = 0;
            for (int w = 0; w < kPenThreads / 64; ++w) { int t = s_red[w]; s_red[w] = run; run += t; }
        }
        __syncthreads();
        int run = s_red[wave] + incl - local;
        for (int w = w0; w < w0 + per && w < words; ++w) { prefix[w] = run; run += __popc(bits[w]); }
    }
    __syncthreads();
    const int nvalid = (words > 0) ? (int)(prefix[words - 1] + __popc(bits[words - 1])) : 0;
    uint32_t* cnt = P.pen_cnt + off;
    for (int i = tid; i < nvalid; i += kPenThreads) cnt[i] = 0;
    drain_memory();
    __syncthreads();
    for (int64_t j = tid; j < n; j += kPenThreads) {
        const int id = ids[j];
        if (id < P.vocab) {
            const int rk = (int)prefix[id >> 5] + __popc(bits[id >> 5] & ((1u << (id & 31)) - 1u));
            atomicAdd(&cnt[rk], 1u);
        }
    }
    drain_memory();
    __syncthreads();
    // penalised values in token-id order (sampler.py:169-173)
    const char* row = row_ptr(P, r);
    const float rep = P.rep[r], pres = P.pres[r], freq = P.freq[r];
    for (int w = tid; w < words; w += kPenThreads) {
        uint32_t b = bits[w];
        int rk = (int)prefix[w];
        while (b) {
            const int bit = __builtin_ctz(b);
            b &= b - 1;
            const int id = w * 32 + bit;
            const uint32_t c = __hip_atomic_load(&cnt[rk], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            float g;
            if (P.dtype == FIE_F32) g = load_one<FIE_F32>(row, id);
            else if (P.dtype == FIE_F16) g = load_one<FIE_F16>(row, id);
            else g = load_one<FIE_BF16>(row, id);
            float pen = (g > 0.0f) ? g / rep : g * rep;
            pen = pen - pres;
            pen = pen - freq * (float)c;
            P.pen_ids[off + rk] = id;
            P.pen_vals[off + rk] = pen;
            ++rk;
        }
    }
    // segment starts: rank of the first element of each slice
    for (int s = tid; s <= P.S; s += kPenThreads) {
        const int64_t e = slice_begin(P, s);
        int rk;
        if (e >= P.vocab) rk = nvalid;
        else rk = (int)prefix[e >> 5] + __popc(bits[e >> 5] & ((1u << (e & 31)) - 1u));
        seg[s] = rk;
    }
    if (tid == 0) {
        // ids >= vocab: distinct count and whether one first appears after token 0
        int ninv = s_ninv;
        int uniq_inv = 0, after0 = 0;
        const int p0 = s_p0;
        if (ninv <= 256) {
            for (int a = 0; a < ninv; ++a) {
                bool first = true;
                for (int b2 = 0; b2 < ninv; ++b2)
                    if (s_inv_id[b2] == s_inv_id[a] && s_inv_pos[b2] < s_inv_pos[a]) { first = false; break; }
                if (first) { ++uniq_inv; if (p0 != 0x7FFFFFFF && s_inv_pos[a] > p0) after0 = 1; }
            }
        } else {
            for (int64_t a = 0; a < n; ++a) {
                const int id = ids[a];
                if (id < P.vocab) continue;
                bool first = true;
                for (int64_t b2 = 0; b2 < a; ++b2) if (ids[b2] == id) { first = false; break; }
                if (first) { ++uniq_inv; if (p0 != 0x7FFFFFFF && a > p0) after0 = 1; }
            }
        }
        const int nuniq = nvalid + uniq_inv;
        P.pen[r] = PenMeta{nvalid, nuniq, p0 != 0x7FFFFFFF ? 1 : 0, after0};
        const unsigned long long tag = ((unsigned long long)(P.epoch & 0xFFFFFFFF) << 32) | (unsigned)nuniq;
        atomicMax(P.wbatch, tag);
    }
}

// ============================================================== diagnostics
// Optional per-(row, slice) phase timestamps (wall clock, 100 MHz) for profiling.
__device__ uint64_t* g_trace = nullptr;

FIE_DEV void trace_mark(int r, int s, int S, int i)
{
    uint64_t* t = g_trace;
    if (t != nullptr && threadIdx.x == 0) t[((int64_t)r * S + s) * 8 + i] = wall_clock64();
}

// ============================================================== row hand-off
// The workgroups of one row cooperate through three arrival counters in the
// row's state.  A workgroup publishes its partial results (agent-scope atomics),
// drains its memory counters and increments the counter; the last one to arrive
// turns the merged partials into a plan, publishes it and raises kPlanReady;
// the others wait for that bit.  The wait is bounded: a workgroup that gives up
// marks the row FIE_ROW_TIMEOUT and leaves, and the host resolves such a row
// with the exact fallback.  Waiting is safe because workgroups are dispatched in
// order and one row's workgroups are consecutive, so a row never waits on a
// workgroup that cannot become resident.
constexpr unsigned int kPlanReady = 0x80000000u;
constexpr unsigned int kSpinLimit = 1u << 18;

FIE_DEV bool arrive(unsigned int* ctr, int S, int* flag)
{
    drain_memory();
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned int old = atomicAdd(ctr, 1u);
        *flag = ((old & ~kPlanReady) == (unsigned int)(S - 1));
    }
    __syncthreads();
    return *flag != 0;
}

FIE_DEV void publish_plan(unsigned int* ctr)
{
    drain_memory();
    __syncthreads();
    if (threadIdx.x == 0) atomicOr(ctr, kPlanReady);
}

FIE_DEV bool wait_plan(unsigned int* ctr, int* flag)
{
    if (threadIdx.x == 0) {
        unsigned int n = 0;
        bool ok = true;
        while (!(ld_shared(ctr) & kPlanReady)) {
            __builtin_amdgcn_s_sleep(2);
            if (++n > kSpinLimit) { ok = false; break; }
        }
        *flag = ok;
    }
    __syncthreads();
    return *flag != 0;
}

// ============================================================== per-row plans
FIE_DEV void write_row_outputs_default(const Params& P, int r)
{
    P.tk_key[r] = 0;
    P.cut_comp[r] = 0;
    P.kept_mass[r] = 0;
    P.row_mass[r] = 0;
}

struct SampleLds {
    PatchLds patch;
    union {
        uint32_t chist[kCountBins];
        struct {
            uint32_t cnt[kMassBins];
            unsigned long long mass[kMassBins];
        } mh;
        uint64_t key[kCap];
    } u;
    uint64_t red[kWaves + 1];
    uint64_t scal[4];
    uint32_t ured[kWaves];
    int flag;
    int found_bin;
};

// Rank selection of the row (top-k and logprob lists): the bin of the global
// count histogram that holds the kk-th largest w; candidates are gathered from
// that bin's lower edge (less a margin that covers values a temperature divide
// merges with the threshold value).
FIE_DEV uint32_t plan_rank(const Params& P, int r, int kk, SampleLds& L)
{
    uint32_t* gh = P.chist + (int64_t)r * kCountBins;
    constexpr int per = kCountBins / kThreads;
    const int tid = threadIdx.x;
    const int bhi = kCountBins - 1 - tid * per;
    uint32_t c[per];
    uint64_t local = 0;
#pragma unroll
    for (int i = 0; i < per; ++i) {
        c[i] = ld_shared(&gh[bhi - i]);
        if (c[i]) st_shared(&gh[bhi - i], 0u);
        local += c[i];
    }
    uint64_t total;
    const uint64_t above = block_excl_scan_u64<kThreads>(local, L.red, &total);
    if (tid == 0) L.found_bin = 0;
    __syncthreads();
    if (above < (uint64_t)kk && above + local >= (uint64_t)kk) {
        uint64_t cum = above;
        for (int i = 0; i < per; ++i) {
            cum += c[i];
            if (cum >= (uint64_t)kk) { L.found_bin = bhi - i; break; }
        }
    }
    __syncthreads();
    const int64_t lo = ((int64_t)L.found_bin << kCountShift) - 16;
    return lo > 0 ? (uint32_t)lo : 0u;
}

// Wide rows: from the survivor mass histogram, the bin holding the top-p cut
// (first bin whose inclusive mass reaches ceil(p*S)) and the bins the draw can
// land in, as at most two w-key intervals; run by the row's last workgroup.
FIE_DEV void plan_wide(const Params& P, int r, SampleLds& L)
{
    RowState& st = P.st[r];
    const int tid = threadIdx.x;
    unsigned long long* gm = P.mmass + (int64_t)r * kMassBins;
    uint32_t* gc = P.mcnt + (int64_t)r * kMassBins;
    constexpr int per = kMassBins / kThreads;
    const int b0 = tid * per;
    uint64_t m[per];
    uint64_t local = 0;
#pragma unroll
    for (int i = 0; i < per; ++i) {
        m[i] = ld_shared(&gm[b0 + i]);
        L.u.mh.cnt[b0 + i] = ld_shared(&gc[b0 + i]);
        local += m[i];
    }
    uint64_t S;
    uint64_t run = block_excl_scan_u64<kThreads>(local, L.red, &S);
    unsigned long long* A = L.u.mh.mass;   // A[b] = survivor mass of bins < b
#pragma unroll
    for (int i = 0; i < per; ++i) { A[b0 + i] = run; run += m[i]; }
    __syncthreads();
    const float p = P.top_p[r];
    const double u = P.uniform[r];
    if (tid == 0) {
        auto Aat = [&](int b) -> uint64_t { return b >= kMassBins ? S : A[b]; };
        int bc = -1, blo, bhi;
        uint64_t thr = ~0ull;
        if (p < 1.0f) {
            thr = ceil_mul_f32(p, S);
            int lo = 0, hi = kMassBins - 1;
            while (lo < hi) { int mid = (lo + hi) >> 1; if (Aat(mid + 1) >= thr) hi = mid; else lo = mid + 1; }
            bc = lo;
            const uint64_t tlo = floor_mul_f64(u, Aat(bc));
            const uint64_t thi = floor_mul_f64(u, Aat(bc + 1));
            lo = 0; hi = bc;
            while (lo < hi) { int mid = (lo + hi) >> 1; if (Aat(mid + 1) > tlo) hi = mid; else lo = mid + 1; }
            blo = lo;
            lo = 0; hi = bc;
            while (lo < hi) { int mid = (lo + hi) >> 1; if (Aat(mid + 1) > thi) hi = mid; else lo = mid + 1; }
            bhi = lo;
        } else {
            const uint64_t t = floor_mul_f64(u, S);
            int lo = 0, hi = kMassBins - 1;
            while (lo < hi) { int mid = (lo + hi) >> 1; if (Aat(mid + 1) > t) hi = mid; else lo = mid + 1; }
            blo = bhi = lo;
        }
        int wa[2] = {blo, 0}, wb[2] = {bhi, 0}, nw = 1;
        if (bc >= 0 && bc > bhi) {
            if (bc == bhi + 1) wb[0] = bc;
            else { wa[1] = bc; wb[1] = bc; nw = 2; }
        }
        uint64_t count = 0;
        for (int w = 0; w < nw; ++w)
            for (int b = wa[w]; b <= wb[w]; ++b) count += L.u.mh.cnt[b];
        const float s = P.scale[r], M = ld_shared(&st.M), ds = ld_shared(&st.dscale);
        for (int w = 0; w < nw; ++w) {
            uint32_t lo2 = kKeyNegInf, hi2 = kKeyPosInf;
            while (lo2 < hi2) {       // smallest key with bin <= wb
                const uint32_t mid = lo2 + (hi2 - lo2) / 2;
                if (bin_of_key(mid, s, M, ds) <= wb[w]) hi2 = mid; else lo2 = mid + 1;
            }
            st_shared(&st.wlo[w], lo2);
            lo2 = kKeyNegInf; hi2 = kKeyPosInf;
            while (lo2 < hi2) {       // largest key with bin >= wa
                const uint32_t mid = lo2 + (hi2 - lo2 + 1) / 2;
                if (bin_of_key(mid, s, M, ds) >= wa[w]) lo2 = mid; else hi2 = mid - 1;
            }
            st_shared(&st.whi[w], lo2);
        }
        st_shared(&st.nwin, nw);
        st_shared(&st.bc, bc);
        st_shared(&st.wb0, wb[0]);
        st_shared(&st.thr, (unsigned long long)thr);
        st_shared(&st.S, (unsigned long long)S);
        st_shared(&st.Awa, (unsigned long long)Aat(wa[0]));
        st_shared(&st.Abc, (unsigned long long)(bc >= 0 ? Aat(bc) : 0));
        if (count > (uint64_t)kCap) atomicOr(&st.overflow, 1u);
    }
    __syncthreads();
}

// ============================================================== finishing a row
// Top-L logprob entries from sorted candidates (sampler.py:273-291).
FIE_DEV void write_logprobs(const Params& P, int r, const uint64_t* key, int n, float M,
                            uint64_t sall, float ychosen)
{
    const int Lp = P.logprobs[r];
    if (Lp < 0) return;
    const double lse = log((double)sall / 1099511627776.0);
    if (threadIdx.x == 0) P.chosen_lp[r] = (float)(((double)ychosen - (double)M) - lse);
    for (int j = threadIdx.x; j < P.lp_cols; j += kThreads) {
        const int64_t o = (int64_t)r * P.lp_cols + j;
        if (j < Lp && j < n) {
            const uint64_t c = key[j];
            const float y = key_to_float((uint32_t)(c >> 32));
            P.top_ids[o] = comp_idx(c);
            P.top_lp[o] = (float)(((double)y - (double)M) - lse);
        } else {
            P.top_ids[o] = -1;
            P.top_lp[o] = 0.0f;
        }
    }
}

// Loads n candidates (w bits, index), turns them into rank keys of y and sorts
// them (value descending, index ascending).
FIE_DEV void load_sorted(const uint64_t* buf, int n, float s, uint64_t* key)
{
    const int N = pow2_at_least(n);
    for (int i = threadIdx.x; i < N; i += kThreads) {
        uint64_t c = 0;
        if (i < n) {
            const uint64_t raw = ld_shared(&buf[i]);
            const float y = scaled(__uint_as_float((uint32_t)(raw >> 32)), s);
            c = comp_key(fkey(y), (uint32_t)raw);
        }
        key[i] = c;
    }
    __syncthreads();
    bitonic_sort_desc<kThreads>(key, N);
}

FIE_DEV void set_status(const Params& P, int r, int bits)
{
    if (bits) atomicOr(&P.status[r], bits);
}

// Greedy rows with logprobs and top-k rows: the candidates hold every survivor.
// Filters sampler.py:194-228 with rules R2-R5, then the draw R4.
FIE_DEV void finalize_topk(const Params& P, int r, int kind, SampleLds& L)
{
    RowState& st = P.st[r];
    const int tid = threadIdx.x;
    const float s = P.scale[r], M = ld_shared(&st.M);
    const unsigned int nraw = ld_shared(&st.nA);
    const bool over = nraw > (unsigned int)kCap;
    const int n = over ? kCap : (int)nraw;
    const uint64_t sall = ld_shared(&st.sall);
    const uint32_t keyA = ld_shared(&st.keyA);
    uint64_t* key = L.u.key;
    if (kind == kKindGreedy) {
        const unsigned long long mp = ld_shared(&st.maxpack);
        const int argmax = (int)(0xFFFFFFFFu - (uint32_t)(mp & 0xFFFFFFFFu));
        if (P.logprobs[r] > 0) load_sorted(P.candA + (int64_t)r * kCap, n, s, key);
        write_logprobs(P, r, key, n, M, sall, M);
        if (tid == 0) {
            write_row_outputs_default(P, r);
            set_status(P, r, over ? FIE_ROW_OVERFLOW : 0);
            P.kept_mass[r] = weight_of(1.0f);
            P.row_mass[r] = sall;
            P.tokens[r] = argmax;
        }
        return;
    }
    load_sorted(P.candA + (int64_t)r * kCap, n, s, key);
    const int k = P.top_k[r];
    const float mp = P.min_p[r];
    const float p = P.top_p[r];
    const uint32_t tk = (k >= 1 && k <= n) ? (uint32_t)(key[k - 1] >> 32) : 0u;
    // A survivor outside the candidates would have w-key < keyA: check that the
    // largest such value cannot reach the threshold.
    bool unsafe = over || k > n;
    if (keyA > kKeyNegInf) {
        const float yout = scaled(key_to_float(keyA - 1), s);
        if (fkey(yout) >= tk) unsafe = true;
    }
    constexpr int per = kCap / kThreads;
    const int j0 = tid * per;
    uint64_t w[per];
    bool sv[per];
    uint64_t local = 0;
#pragma unroll
    for (int i = 0; i < per; ++i) {
        const int j = j0 + i;
        sv[i] = false;
        w[i] = 0;
        if (j < n) {
            const uint32_t yk = (uint32_t)(key[j] >> 32);
            const float e = cexp(key_to_float(yk) - M);
            sv[i] = yk >= tk && !(mp > 0.0f && e < mp);
            if (sv[i]) w[i] = weight_of(e);
        }
        local += w[i];
    }
    uint64_t S;
    const uint64_t excl0 = block_excl_scan_u64<kThreads>(local, L.red, &S);
    const uint64_t thr = (p < 1.0f) ? ceil_mul_f32(p, S) : ~0ull;
    uint64_t ex = excl0, kept_local = 0, cut = ~0ull;
    bool kept[per];
#pragma unroll
    for (int i = 0; i < per; ++i) {
        kept[i] = sv[i] && ex < thr;
        if (kept[i]) { kept_local += w[i]; cut = key[j0 + i] < cut ? key[j0 + i] : cut; }
        ex += w[i];
    }
    const uint64_t T = block_sum_u64<kThreads>(kept_local, L.red);
    cut = block_min_u64<kThreads>(cut, L.red);
    const uint64_t t = floor_mul_f64(P.uniform[r], T);
    if (tid == 0) L.scal[0] = ~0ull;
    __syncthreads();
    ex = excl0;
#pragma unroll
    for (int i = 0; i < per; ++i) {
        if (kept[i] && ex <= t && t < ex + w[i]) L.scal[0] = key[j0 + i];
        ex += w[i];
    }
    __syncthreads();
    const uint64_t chosen = L.scal[0];
    write_logprobs(P, r, key, n, M, sall, key_to_float((uint32_t)(chosen >> 32)));
    if (tid == 0) {
        set_status(P, r, (unsafe || chosen == ~0ull) ? FIE_ROW_OVERFLOW : 0);
        P.tk_key[r] = tk;
        P.cut_comp[r] = (p < 1.0f && cut != ~0ull) ? cut : 0;
        P.kept_mass[r] = T;
        P.row_mass[r] = (P.logprobs[r] >= 0) ? sall : 0;
        P.tokens[r] = (chosen == ~0ull) ? -1 : (int64_t)comp_idx(chosen);
    }
}

// Wide rows: exact cut and draw from the window candidates and the masses in
// front of the windows (rules R2-R4).
FIE_DEV void finalize_wide(const Params& P, int r, SampleLds& L)
{
    RowState& st = P.st[r];
    const int tid = threadIdx.x;
    const float s = P.scale[r], p = P.top_p[r];
    const float M = ld_shared(&st.M), ds = ld_shared(&st.dscale);
    const unsigned int nraw = ld_shared(&st.nB);
    const int n = nraw > (unsigned int)kCap ? kCap : (int)nraw;
    const int bc = ld_shared(&st.bc), wb0 = ld_shared(&st.wb0);
    const uint64_t thr = ld_shared(&st.thr), S = ld_shared(&st.S);
    const uint64_t Awa = ld_shared(&st.Awa), Abc = ld_shared(&st.Abc);
    const bool over = ld_shared(&st.overflow) || nraw > (unsigned int)kCap;
    const uint64_t sall = ld_shared(&st.sall);
    uint64_t* key = L.u.key;
    load_sorted(P.candB + (int64_t)r * kCap, n, s, key);
    constexpr int per = kCap / kThreads;
    const int j0 = tid * per;
    uint64_t w[per], w0 = 0;
    int bn[per];
    uint64_t local = 0;
#pragma unroll
    for (int i = 0; i < per; ++i) {
        const int j = j0 + i;
        w[i] = 0;
        bn[i] = kMassBins;
        if (j < n) {
            const float d = key_to_float((uint32_t)(key[j] >> 32)) - M;
            w[i] = weight_of(cexp(d));
            bn[i] = d_bin(d, ds);
            if (bn[i] <= wb0) w0 += w[i];
        }
        local += w[i];
    }
    uint64_t tot;
    uint64_t pre = block_excl_scan_u64<kThreads>(local, L.red, &tot);
    const uint64_t W0 = block_sum_u64<kThreads>(w0, L.red);   // mass gathered in window 0
    uint64_t ex[per];
    bool kept[per];
    uint64_t kept_bc = 0, cut = ~0ull;
#pragma unroll
    for (int i = 0; i < per; ++i) {
        const int j = j0 + i;
        kept[i] = false;
        ex[i] = 0;
        if (j < n) {
            const int b = bn[i];
            ex[i] = (b <= wb0) ? Awa + pre : Abc + (pre - W0);
            if (p < 1.0f) {
                kept[i] = b < bc || (b == bc && ex[i] < thr);
                if (b == bc && kept[i]) {
                    kept_bc += w[i];
                    cut = key[j] < cut ? key[j] : cut;
                }
            } else {
                kept[i] = true;
            }
        }
        pre += w[i];
    }
    kept_bc = block_sum_u64<kThreads>(kept_bc, L.red);
    cut = block_min_u64<kThreads>(cut, L.red);
    const uint64_t T = (p < 1.0f) ? Abc + kept_bc : S;
    const uint64_t t = floor_mul_f64(P.uniform[r], T);
    if (tid == 0) L.scal[0] = ~0ull;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < per; ++i)
        if (kept[i] && ex[i] <= t && t < ex[i] + w[i]) L.scal[0] = key[j0 + i];
    __syncthreads();
    const uint64_t chosen = L.scal[0];
    if (tid == 0) {
        set_status(P, r, (over || chosen == ~0ull) ? FIE_ROW_OVERFLOW : 0);
        P.tk_key[r] = 0;
        P.cut_comp[r] = (p < 1.0f && cut != ~0ull) ? cut : 0;
        P.kept_mass[r] = T;
        P.row_mass[r] = sall;
        P.tokens[r] = (chosen == ~0ull) ? -1 : (int64_t)comp_idx(chosen);
        L.scal[1] = chosen;
    }
    __syncthreads();
    // logprobs of a wide row: the top-L candidates gathered for the rank list
    if (P.logprobs[r] >= 0) {
        const unsigned int na = ld_shared(&st.nA);
        const int nA = na > (unsigned int)kCap ? kCap : (int)na;
        if (P.logprobs[r] > 0) load_sorted(P.candA + (int64_t)r * kCap, nA, s, key);
        write_logprobs(P, r, key, nA, M, sall, key_to_float((uint32_t)(L.scal[1] >> 32)));
        if (tid == 0 && na > (unsigned int)kCap) set_status(P, r, FIE_ROW_OVERFLOW);
    }
}

// Restores the row's accumulators and histograms to zero for the next call.
FIE_DEV void reset_row(const Params& P, int r, bool wide)
{
    RowState& st = P.st[r];
    if (wide) {
        unsigned long long* gm = P.mmass + (int64_t)r * kMassBins;
        uint32_t* gc = P.mcnt + (int64_t)r * kMassBins;
        for (int b = threadIdx.x; b < kMassBins; b += kThreads) {
            if (ld_shared(&gc[b])) {
                st_shared(&gc[b], 0u);
                st_shared(&gm[b], 0ull);
            }
        }
    }
    if (threadIdx.x == 0) {
        st_shared(&st.maxpack, 0ull);
        st_shared(&st.minkey_inv, 0u);
        st_shared(&st.sall, 0ull);
        st_shared(&st.nA, 0u);
        st_shared(&st.nB, 0u);
        st_shared(&st.overflow, 0u);
        st_shared(&st.arrive[0], 0u);
        st_shared(&st.arrive[1], 0u);
        st_shared(&st.arrive[2], 0u);
    }
}

// ============================================================== the sampler step
// Slice s of row r.  The slice (CPT 16-byte chunks per thread) is read from HBM
// once into registers; every later phase works on the registers.
template <int DT, int CPT>
FIE_DEV void sample_row(const Params& P, int r, int s, SampleLds& L)
{
    constexpr int EPC = Dt<DT>::EPC;
    constexpr int NE = CPT * EPC;
    const int tid = threadIdx.x;
    RowState& st = P.st[r];
    const bool argmax_only = P.argmax_only != 0;
    const bool greedy = argmax_only || (P.flags[r] & 1);
    const int Lp = argmax_only ? -1 : P.logprobs[r];
    const int k = greedy ? 0 : P.top_k[r];
    const int kind = greedy ? kKindGreedy : (k > 0 ? kKindTopK : kKindWide);
    const int kk = kind == kKindTopK ? (k > Lp ? k : Lp) : Lp;
    const bool need_sel = kk > 0;
    const bool need_mass = kind == kKindWide || Lp >= 0;
    const float sc = argmax_only ? 1.0f : P.scale[r];
    trace_mark(r, s, P.S, 0);

    // ---- the slice, into registers (penalty patches applied on the way)
    PatchView pv{0, true, slice_begin(P, s), nullptr, nullptr};
    if (!argmax_only) pv = stage_patches(P, r, s, L.patch);
    const char* row = row_ptr(P, r);
    const int64_t nch = (P.vocab + EPC - 1) / EPC;
    const int64_t cbase = (int64_t)s * P.cps + tid;
    float v[NE];
    int nv[CPT];                         // valid elements in each chunk
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int64_t c = cbase + (int64_t)j * kThreads;
        const int64_t left = (int64_t)P.vocab - c * EPC;
        nv[j] = left >= EPC ? EPC : (left > 0 ? (int)left : 0);
        if (nv[j] == EPC) {
            load_chunk<DT>(row, c * EPC, P.vec_ok, &v[j * EPC]);
        } else {
#pragma unroll
            for (int q = 0; q < EPC; ++q)
                v[j * EPC + q] = (q < nv[j]) ? load_one<DT>(row, c * EPC + q) : -INFINITY;
        }
    }
    if (pv.n) {
#pragma unroll
        for (int j = 0; j < CPT; ++j)
            if (nv[j] > 0) apply_patches<EPC>(pv, L.patch, (cbase + (int64_t)j * kThreads) * EPC, &v[j * EPC]);
    }
    (void)nch;
    trace_mark(r, s, P.S, 1);

    // ---- phase 1: max (first index on ties), min, per-thread max
    uint64_t best = 0;
    uint32_t minv = 0;
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const uint32_t e0 = (uint32_t)((cbase + (int64_t)j * kThreads) * EPC);
#pragma unroll
        for (int q = 0; q < EPC; ++q) {
            if (q < nv[j]) {
                const uint32_t key = fkey(v[j * EPC + q] + 0.0f);
                const uint64_t pack = ((uint64_t)key << 32) | (0xFFFFFFFFu - (e0 + q));
                best = pack > best ? pack : best;
                minv = (~key) > minv ? ~key : minv;
            }
        }
    }
    const uint32_t tmax = (uint32_t)(best >> 32);
    const uint64_t bbest = block_max_u64<kThreads>(best, L.red);
    const uint64_t bmin = (kind == kKindWide) ? block_max_u64<kThreads>(minv, L.red) : 0;
    if (tid == 0) {
        atomicMax(&st.maxpack, (unsigned long long)bbest);
        if (kind == kKindWide) atomicMax(&st.minkey_inv, (unsigned int)bmin);
    }

    if (kind == kKindGreedy && Lp < 0) {
        // sampler.py:103-106 and :236-238: the argmax is the answer
        if (arrive(&st.arrive[0], P.S, &L.flag) && tid == 0) {
            const unsigned long long mp = ld_shared(&st.maxpack);
            const int argmax = (int)(0xFFFFFFFFu - (uint32_t)(mp & 0xFFFFFFFFu));
            P.tokens[r] = argmax;
            if (!argmax_only) {
                write_row_outputs_default(P, r);
                P.row_max[r] = key_to_float((uint32_t)(mp >> 32));
                P.kept_mass[r] = weight_of(1.0f);
            }
            st_shared(&st.maxpack, 0ull);
            st_shared(&st.arrive[0], 0u);
        }
        return;
    }

    // ---- phase 2 (rank selection): histogram of keys that can be in the top kk.
    // The kk-th largest per-thread maximum bounds the row's kk-th largest value
    // from below, so smaller keys need not be counted.
    if (need_sel) {
        uint32_t theta = 0;
        if (kk <= kThreads) {
            // largest theta with #(thread maxima >= theta) >= kk, built bit by bit
            // from the top (the count is non-increasing in theta): 32 fixed steps
            for (int bit = 31; bit >= 0; --bit) {
                const uint32_t cand = theta | (1u << bit);
                const uint64_t m = __ballot(tmax >= cand);
                if ((tid & 63) == 0) L.ured[tid >> 6] = (uint32_t)__popcll(m);
                __syncthreads();
                uint32_t cnt = 0;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) cnt += L.ured[w];
                __syncthreads();
                if (cnt >= (uint32_t)kk) theta = cand;
            }
        }
        for (int i = tid; i < kCountBins; i += kThreads) L.u.chist[i] = 0;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < CPT; ++j)
#pragma unroll
            for (int q = 0; q < EPC; ++q)
                if (q < nv[j]) {
                    const uint32_t key = fkey(v[j * EPC + q] + 0.0f);
                    if (key >= theta) atomicAdd(&L.u.chist[key >> kCountShift], 1u);
                }
        __syncthreads();
        uint32_t* gh = P.chist + (int64_t)r * kCountBins;
        for (int i = tid; i < kCountBins; i += kThreads)
            if (L.u.chist[i]) atomicAdd(&gh[i], L.u.chist[i]);
    }

    // ---- hand-off 1: row max (and rank bin) for every workgroup of the row
    trace_mark(r, s, P.S, 2);
    if (arrive(&st.arrive[0], P.S, &L.flag)) {
        uint32_t keyA = 0;
        if (need_sel) keyA = plan_rank(P, r, kk, L);
        if (tid == 0) {
            const unsigned long long mp = ld_shared(&st.maxpack);
            const float M = scaled(key_to_float((uint32_t)(mp >> 32)), sc);
            st_shared(&st.M, M);
            st_shared(&st.keyA, keyA);
            if (kind == kKindWide) {
                const float ymin = scaled(key_to_float(~ld_shared(&st.minkey_inv)), sc);
                const float R = fminf(M - ymin, 28.0f);
                st_shared(&st.dscale, (R > 0.0f) ? (float)(kMassBins - 1) / R : 0.0f);
            }
            P.row_max[r] = M;
        }
        publish_plan(&st.arrive[0]);
    } else if (!wait_plan(&st.arrive[0], &L.flag)) {
        if (tid == 0) set_status(P, r, FIE_ROW_TIMEOUT);
        return;
    }
    const float M = ld_shared(&st.M);
    trace_mark(r, s, P.S, 3);

    // ---- phase 3: integer weights (row mass; survivor mass histogram of wide rows)
    if (need_mass) {
        const float ds = ld_shared(&st.dscale);
        const float mp = P.min_p[r];
        const bool hist = kind == kKindWide;
        if (hist) {
            for (int i = tid; i < kMassBins; i += kThreads) { L.u.mh.cnt[i] = 0; L.u.mh.mass[i] = 0; }
            __syncthreads();
        }
        uint64_t sall = 0;
#pragma unroll
        for (int j = 0; j < CPT; ++j)
#pragma unroll
            for (int q = 0; q < EPC; ++q)
                if (q < nv[j]) {
                    const float d = scaled(v[j * EPC + q], sc) - M;
                    const float e = cexp(d);
                    const uint64_t wt = weight_of(e);
                    sall += wt;
                    if (hist && !(mp > 0.0f && e < mp)) {
                        const int b = d_bin(d, ds);
                        atomicAdd(&L.u.mh.cnt[b], 1u);
                        atomicAdd(&L.u.mh.mass[b], (unsigned long long)wt);
                    }
                }
        sall = block_sum_u64<kThreads>(sall, L.red);
        if (tid == 0) atomicAdd(&st.sall, (unsigned long long)sall);
        if (hist) {
            __syncthreads();
            uint32_t* gc = P.mcnt + (int64_t)r * kMassBins;
            unsigned long long* gm = P.mmass + (int64_t)r * kMassBins;
            for (int i = tid; i < kMassBins; i += kThreads)
                if (L.u.mh.cnt[i]) {
                    atomicAdd(&gc[i], L.u.mh.cnt[i]);
                    atomicAdd(&gm[i], L.u.mh.mass[i]);
                }
        }
    }

    // ---- hand-off 2 (wide rows): cut and draw windows
    trace_mark(r, s, P.S, 4);
    if (kind == kKindWide) {
        if (arrive(&st.arrive[1], P.S, &L.flag)) {
            plan_wide(P, r, L);
            publish_plan(&st.arrive[1]);
        } else if (!wait_plan(&st.arrive[1], &L.flag)) {
            if (tid == 0) set_status(P, r, FIE_ROW_TIMEOUT);
            return;
        }
        const uint32_t lo0 = ld_shared(&st.wlo[0]), hi0 = ld_shared(&st.whi[0]);
        const int nw = ld_shared(&st.nwin);
        const uint32_t lo1 = nw > 1 ? ld_shared(&st.wlo[1]) : 1u;
        const uint32_t hi1 = nw > 1 ? ld_shared(&st.whi[1]) : 0u;
        const float mp = P.min_p[r];
        uint64_t* candB = P.candB + (int64_t)r * kCap;
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const uint32_t e0 = (uint32_t)((cbase + (int64_t)j * kThreads) * EPC);
#pragma unroll
            for (int q = 0; q < EPC; ++q) {
                const float w = v[j * EPC + q];
                const uint32_t key = fkey(w + 0.0f);
                bool in = q < nv[j] && ((key >= lo0 && key <= hi0) || (key >= lo1 && key <= hi1));
                if (in && mp > 0.0f) in = !(cexp(scaled(w, sc) - M) < mp);
                append_candidate(in, w, e0 + q, &st.nB, candB);
            }
        }
    }

    // ---- rank candidates (top-k survivors, logprob lists)
    if (need_sel) {
        const uint32_t keyA = ld_shared(&st.keyA);
        uint64_t* candA = P.candA + (int64_t)r * kCap;
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const uint32_t e0 = (uint32_t)((cbase + (int64_t)j * kThreads) * EPC);
#pragma unroll
            for (int q = 0; q < EPC; ++q) {
                const float w = v[j * EPC + q];
                append_candidate(q < nv[j] && fkey(w + 0.0f) >= keyA, w, e0 + q, &st.nA, candA);
            }
        }
    }

    // ---- the last workgroup finishes the row
    trace_mark(r, s, P.S, 5);
    if (!arrive(&st.arrive[2], P.S, &L.flag)) { trace_mark(r, s, P.S, 6); return; }
    trace_mark(r, s, P.S, 6);
    if (kind == kKindWide) finalize_wide(P, r, L);
    else finalize_topk(P, r, kind, L);
    __syncthreads();
    reset_row(P, r, kind == kKindWide);
    trace_mark(r, s, P.S, 7);
}

// Persistent row groups: the grid is as large as the GPU holds at once, in
// groups of S consecutive workgroups; group g handles rows g, g + groups, ...,
// so the S workgroups that cooperate on a row start it together and every wait
// is on a workgroup that is already running.
template <int DT, int CPT>
__global__ __launch_bounds__(kThreads) void k_sample(Params P)
{
    __shared__ SampleLds L;
    const int g = blockIdx.x / P.S, s = blockIdx.x % P.S;
    for (int r = g; r < P.rows; r += P.groups) {
        sample_row<DT, CPT>(P, r, s, L);
        __syncthreads();
    }
}

// ============================================================== kept set / probs
template <int DT>
__global__ __launch_bounds__(kThreads) void k_kept(Params P, uint8_t* kept, float* probs)
{
    __shared__ PatchLds L;
    const int r = blockIdx.x / P.S, s = blockIdx.x % P.S;
    const PatchView pv = stage_patches(P, r, s, L);
    __syncthreads();
    const bool greedy = P.flags[r] & 1;
    const float sc = P.scale[r], M = P.row_max[r], mp = P.min_p[r];
    const uint32_t tk = P.tk_key[r];
    const uint64_t cut = P.cut_comp[r];
    const uint64_t T = P.kept_mass[r];
    const int64_t tok = P.tokens[r];
    const int64_t base = (int64_t)r * P.vocab;
    for_each_element<DT>(P, r, s, pv, L, [&](float w, uint32_t idx) {
        bool k;
        float pr;
        if (greedy) {
            k = true;
            pr = (idx == tok) ? 1.0f : 0.0f;
        } else {
            const float y = scaled(w, sc);
            const uint32_t yk = fkey(y);
            const float e = cexp(y - M);
            k = yk >= tk && !(mp > 0.0f && e < mp) && (cut == 0 || comp_key(yk, idx) >= cut);
            pr = k ? (float)((double)e * 1099511627776.0 / (double)T) : 0.0f;
        }
        if (kept) kept[base + idx] = k ? 1 : 0;
        if (probs) probs[base + idx] = pr;
    });
}

// ============================================================== exact fallback
// Rows whose candidate sets overflowed: sort the whole row by rank key in global
// memory (one workgroup per row) and apply rules R2-R5 over the sorted row.
__global__ __launch_bounds__(1024) void k_fallback_keys(Params P, const int32_t* rows, int count)
{
    const int g = blockIdx.x;
    if (g >= count) return;
    const int r = rows[g];
    uint64_t* key = P.fb_keys + (int64_t)g * P.fb_pow2;
    const char* row = row_ptr(P, r);
    const float s = P.scale[r];
    // penalties: read the slice segments directly (no LDS staging)
    for (int64_t i = threadIdx.x; i < P.fb_pow2; i += 1024) {
        uint64_t c = 0;
        if (i < P.vocab) {
            float w;
            if (P.dtype == FIE_F32) w = load_one<FIE_F32>(row, i);
            else if (P.dtype == FIE_F16) w = load_one<FIE_F16>(row, i);
            else w = load_one<FIE_BF16>(row, i);
            if (P.apply_pen) {
                const int32_t* seg = P.seg + (int64_t)r * (kMaxSlices + 1);
                const int nv = seg[P.S];
                const int32_t* ids = P.pen_ids + P.hist_off[r];
                int lo = 0, hi = nv;
                while (lo < hi) { int mid = (lo + hi) >> 1; if (ids[mid] < i) lo = mid + 1; else hi = mid; }
                if (lo < nv && ids[lo] == i && !(i == 0 && token0_patch_dropped(P, r)))
                    w = P.pen_vals[P.hist_off[r] + lo];
            }
            c = comp_key(fkey(scaled(w, s)), (uint32_t)i);
        }
        key[i] = c;
    }
}

// One bitonic merge stage over every fallback row (launched per stage).
__global__ void k_fallback_stage(Params P, int count, int64_t k, int64_t j)
{
    const int64_t n = P.fb_pow2;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t g = t / (n / 2);
    if (g >= count) return;
    const int64_t q = t % (n / 2);
    const int64_t i = ((q / j) * 2 * j) + (q % j);
    const int64_t ixj = i + j;
    uint64_t* key = P.fb_keys + g * n;
    const uint64_t a = key[i], b = key[ixj];
    const bool up = (i & k) != 0;
    if (up ? (a > b) : (a < b)) { key[i] = b; key[ixj] = a; }
}

__global__ __launch_bounds__(1024) void k_fallback_finish(Params P, const int32_t* rows, int count)
{
    __shared__ uint64_t red[1024 / 64 + 1];
    __shared__ uint64_t scal[2];
    const int g = blockIdx.x;
    if (g >= count) return;
    const int r = rows[g];
    const uint64_t* key = P.fb_keys + (int64_t)g * P.fb_pow2;
    const int V = P.vocab;
    const bool greedy = P.flags[r] & 1;
    const float M = key_to_float((uint32_t)(key[0] >> 32));
    const int k = greedy ? 0 : P.top_k[r];
    const float mp = P.min_p[r], p = P.top_p[r];
    const uint32_t tk = (k > 0) ? (uint32_t)(key[k - 1] >> 32) : 0u;
    const int per = (V + 1023) / 1024;
    const int j0 = threadIdx.x * per;
    // pass A: survivor mass S and whole-row mass
    uint64_t loc = 0, locall = 0;
    for (int j = j0; j < j0 + per && j < V; ++j) {
        const uint32_t yk = (uint32_t)(key[j] >> 32);
        const float e = cexp(key_to_float(yk) - M);
        locall += weight_of(e);
        if (yk >= tk && !(mp > 0.0f && e < mp)) loc += weight_of(e);
    }
    uint64_t S;
    const uint64_t ex0 = block_excl_scan_u64<1024>(loc, red, &S);
    const uint64_t sall = block_sum_u64<1024>(locall, red);
    const uint64_t thr = (!greedy && p < 1.0f) ? ceil_mul_f32(p, S) : ~0ull;
    uint64_t ex = ex0, keptl = 0, cut = ~0ull;
    for (int j = j0; j < j0 + per && j < V; ++j) {
        const uint32_t yk = (uint32_t)(key[j] >> 32);
        const float e = cexp(key_to_float(yk) - M);
        const bool sv = yk >= tk && !(mp > 0.0f && e < mp);
        const uint64_t w = sv ? weight_of(e) : 0;
        if (sv && ex < thr) { keptl += w; cut = key[j] < cut ? key[j] : cut; }
        ex += w;
    }
    const uint64_t T = block_sum_u64<1024>(keptl, red);
    cut = block_min_u64<1024>(cut, red);
    const uint64_t t = floor_mul_f64(P.uniform[r], T);
    if (threadIdx.x == 0) scal[0] = ~0ull;
    __syncthreads();
    ex = ex0;
    for (int j = j0; j < j0 + per && j < V; ++j) {
        const uint32_t yk = (uint32_t)(key[j] >> 32);
        const float e = cexp(key_to_float(yk) - M);
        const bool sv = yk >= tk && !(mp > 0.0f && e < mp);
        const uint64_t w = sv ? weight_of(e) : 0;
        if (sv && ex < thr && ex <= t && t < ex + w) scal[0] = key[j];
        ex += w;
    }
    __syncthreads();
    const uint64_t chosen = scal[0];
    const int Lp = P.logprobs[r];
    const double lse = log((double)sall / 1099511627776.0);
    for (int j = threadIdx.x; j < P.lp_cols && Lp >= 0; j += 1024) {
        const int64_t o = (int64_t)r * P.lp_cols + j;
        if (j < Lp && j < V) {
            P.top_ids[o] = comp_idx(key[j]);
            P.top_lp[o] = (float)(((double)key_to_float((uint32_t)(key[j] >> 32)) - (double)M) - lse);
        } else {
            P.top_ids[o] = -1;
            P.top_lp[o] = 0.0f;
        }
    }
    if (threadIdx.x == 0) {
        // greedy rows: argmax = the first rank (value descending, index ascending)
        const uint64_t pick = greedy ? key[0] : chosen;
        P.tokens[r] = (pick == ~0ull) ? -1 : (int64_t)comp_idx(pick);
        P.status[r] = (pick == ~0ull) ? FIE_ROW_OVERFLOW : 0;
        P.tk_key[r] = greedy ? 0 : tk;
        P.cut_comp[r] = (!greedy && p < 1.0f && cut != ~0ull) ? cut : 0;
        P.row_max[r] = M;
        P.kept_mass[r] = greedy ? weight_of(1.0f) : T;
        P.row_mass[r] = sall;
        if (Lp >= 0) {
            const float yc = key_to_float((uint32_t)(pick >> 32));
            P.chosen_lp[r] = (float)(((double)yc - (double)M) - lse);
        }
    }
}

// ============================================================== utilities
__global__ void k_fill_zero(uint4* p, size_t n16)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16;
         i += (size_t)gridDim.x * blockDim.x)
        p[i] = make_uint4(0, 0, 0, 0);
}

__global__ void k_cexp(const float* in, float* out, int64_t n)
{
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        out[i] = cexp(in[i]);
}

}  // namespace fie

// ================================================================== C ABI
using namespace fie;

static thread_local char g_err[256] = "";

static int fail(int code, const char* msg)
{
    snprintf(g_err, sizeof g_err, "%s", msg);
    return code;
}

static int check_launch(const char* what)
{
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        snprintf(g_err, sizeof g_err, "%s: %s", what, hipGetErrorString(e));
        return FIE_E_LAUNCH;
    }
    return FIE_OK;
}

// Chunks per slice: 256 threads x CPT 16-byte chunks, CPT = 8 unless that leaves
// fewer than 1024 workgroups (small batches), then CPT = 2.
static void choose_slices(Params& P)
{
    const int64_t nch = (P.vocab + P.epc - 1) / P.epc;
    int cpt = 8;
    if ((int64_t)P.rows * ((nch + kThreads * 8 - 1) / (kThreads * 8)) < 1024) cpt = 2;
    P.cps = kThreads * cpt;
    P.S = (int)((nch + P.cps - 1) / P.cps);
}

static int fill_layout(Params& P, const fie_workspace* ws, int rows, int64_t hist)
{
    if (!ws || !ws->ptr) return fail(FIE_E_WORKSPACE, "workspace is NULL");
    if (rows > ws->max_rows) return fail(FIE_E_WORKSPACE, "more rows than the workspace holds");
    if (hist > ws->max_hist) return fail(FIE_E_WORKSPACE, "more history than the workspace holds");
    if (P.vocab > ws->vocab) return fail(FIE_E_WORKSPACE, "vocab larger than the workspace's");
    const Layout Ly = make_layout(ws->max_rows, ws->max_hist, ws->vocab);
    if (ws->bytes < Ly.total) return fail(FIE_E_WORKSPACE, "workspace smaller than its size");
    char* b = (char*)ws->ptr;
    P.st = (RowState*)(b + Ly.rows);
    P.pen = (PenMeta*)(b + Ly.pen);
    P.wbatch = (unsigned long long*)(b + Ly.wbatch);
    P.chist = (uint32_t*)(b + Ly.chist);
    P.mcnt = (uint32_t*)(b + Ly.mcnt);
    P.mmass = (unsigned long long*)(b + Ly.mmass);
    P.candA = (uint64_t*)(b + Ly.candA);
    P.candB = (uint64_t*)(b + Ly.candB);
    P.seg = (int32_t*)(b + Ly.seg);
    P.pen_ids = (int32_t*)(b + Ly.pen_ids);
    P.pen_vals = (float*)(b + Ly.pen_vals);
    P.pen_cnt = (uint32_t*)(b + Ly.pen_cnt);
    P.fb_keys = (uint64_t*)(b + Ly.fb_keys);
    int64_t vp = 64;
    while (vp < ws->vocab) vp <<= 1;
    P.fb_pow2 = vp;
    return FIE_OK;
}

static int fill_params(Params& P, const fie_sampler_args* a, const fie_workspace* ws)
{
    memset(&P, 0, sizeof P);
    if (!a || !a->logits) return fail(FIE_E_ARG, "logits is NULL");
    if (a->dtype < FIE_F32 || a->dtype > FIE_BF16) return fail(FIE_E_ARG, "unknown dtype");
    if (a->rows <= 0 || a->vocab <= 0) return fail(FIE_E_ARG, "rows and vocab must be positive");
    if (a->vocab > kMaxPenWords * 32) return fail(FIE_E_ARG, "vocab above 262144 is not supported");
    if (a->lp_cols < 0 || a->lp_cols > 20) return fail(FIE_E_ARG, "lp_cols must be in [0, 20]");
    if (a->row_stride < a->vocab) return fail(FIE_E_ARG, "row_stride smaller than vocab");
    const int es = a->dtype == FIE_F32 ? 4 : 2;
    P.logits = (const char*)a->logits;
    P.row_stride_bytes = a->row_stride * es;
    P.dtype = a->dtype;
    P.rows = a->rows;
    P.vocab = a->vocab;
    P.lp_cols = a->lp_cols;
    P.epc = 16 / es;
    P.vec_ok = (((uintptr_t)a->logits % 16) == 0 && (P.row_stride_bytes % 16) == 0) ? 1 : 0;
    choose_slices(P);
    if (P.S > kMaxSlices) return fail(FIE_E_ARG, "vocab too large for the slice table");
    P.apply_pen = a->apply_penalties ? 1 : 0;
    P.epoch = a->epoch;
    P.scale = a->scale; P.top_k = a->top_k; P.top_p = a->top_p; P.min_p = a->min_p;
    P.flags = a->flags; P.logprobs = a->logprobs; P.uniform = a->uniform;
    P.rep = a->repetition; P.pres = a->presence; P.freq = a->frequency;
    P.hist_off = a->hist_offsets; P.hist_ids = a->hist_ids;
    P.tokens = a->tokens; P.status = a->status; P.tk_key = a->tk_key; P.cut_comp = a->cut_comp;
    P.row_max = a->row_max; P.kept_mass = a->kept_mass; P.row_mass = a->row_mass;
    P.chosen_lp = a->chosen_logprob; P.top_ids = a->top_ids; P.top_lp = a->top_logprobs;
    if (!P.scale || !P.top_k || !P.top_p || !P.min_p || !P.flags || !P.logprobs || !P.uniform)
        return fail(FIE_E_ARG, "a per-row parameter array is NULL");
    if (!P.tokens || !P.status || !P.tk_key || !P.cut_comp || !P.row_max || !P.kept_mass ||
        !P.row_mass || !P.chosen_lp)
        return fail(FIE_E_ARG, "an output array is NULL");
    if (P.lp_cols > 0 && (!P.top_ids || !P.top_lp)) return fail(FIE_E_ARG, "top_ids/top_logprobs is NULL");
    if (P.apply_pen && (!P.rep || !P.pres || !P.freq || !P.hist_off || (a->hist_total > 0 && !P.hist_ids)))
        return fail(FIE_E_ARG, "penalty arrays are NULL");
    return fill_layout(P, ws, a->rows, P.apply_pen ? a->hist_total : 0);
}

// Workgroups of a kernel that the device holds at once.
static int resident_capacity(const void* kernel)
{
    int dev = 0, cus = 0, per = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, kThreads, 0) != hipSuccess) return 0;
    return cus * per;
}

template <int DT, int CPT>
static void launch_sample_cpt(Params P, hipStream_t st)
{
    const void* fn = (const void*)k_sample<DT, CPT>;
    static thread_local int cap = -1;
    if (cap < 0) cap = resident_capacity(fn);
    int groups = cap / P.S;
    if (groups < 1) groups = 1;
    if (groups > P.rows) groups = P.rows;
    P.groups = groups;
    hipLaunchKernelGGL((k_sample<DT, CPT>), dim3((unsigned)(groups * P.S)), dim3(kThreads), 0,
                       st, P);
}

template <int DT>
static void launch_sample(const Params& P, hipStream_t st)
{
    if (P.cps == kThreads * 8) launch_sample_cpt<DT, 8>(P, st);
    else launch_sample_cpt<DT, 2>(P, st);
}

static int launch_stage(const Params& P, int stage, hipStream_t st)
{
    switch (stage) {
    case FIE_STAGE_PENALTY:
        if (!P.apply_pen) return FIE_OK;
        hipLaunchKernelGGL(k_penalty, dim3(P.rows), dim3(kPenThreads),
                           (size_t)((P.vocab + 31) / 32) * 2 * sizeof(uint32_t), st, P);
        return check_launch("k_penalty");
    case FIE_STAGE_SAMPLE:
        if (P.dtype == FIE_F32) launch_sample<FIE_F32>(P, st);
        else if (P.dtype == FIE_F16) launch_sample<FIE_F16>(P, st);
        else launch_sample<FIE_BF16>(P, st);
        return check_launch("k_sample");
    default:
        return fail(FIE_E_ARG, "unknown stage");
    }
}

extern "C" {

size_t fie_sampler_workspace_size(int32_t max_rows, int32_t vocab, int64_t max_hist)
{
    return make_layout(max_rows, max_hist, vocab).total;
}

int fie_sampler_workspace_init(const fie_workspace* ws, void* stream)
{
    if (!ws || !ws->ptr) return fail(FIE_E_WORKSPACE, "workspace is NULL");
    const Layout Ly = make_layout(ws->max_rows, ws->max_hist, ws->vocab);
    if (ws->bytes < Ly.total) return fail(FIE_E_WORKSPACE, "workspace smaller than its size");
    const size_t n16 = Ly.total / 16;
    hipLaunchKernelGGL(k_fill_zero, dim3(1024), dim3(256), 0, (hipStream_t)stream,
                       (uint4*)ws->ptr, n16);
    return check_launch("workspace_init");
}

int fie_sampler_sample(const fie_sampler_args* a, const fie_workspace* ws, void* stream)
{
    Params P;
    int rc = fill_params(P, a, ws);
    if (rc) return rc;
    for (int stage = FIE_STAGE_PENALTY; stage <= FIE_STAGE_SAMPLE; ++stage)
        if ((rc = launch_stage(P, stage, (hipStream_t)stream))) return rc;
    return FIE_OK;
}

int fie_sampler_stage(const fie_sampler_args* a, const fie_workspace* ws, int32_t stage,
                      void* stream)
{
    Params P;
    int rc = fill_params(P, a, ws);
    if (rc) return rc;
    return launch_stage(P, stage, (hipStream_t)stream);
}

int fie_sampler_resolve_overflow(const fie_sampler_args* a, const int32_t* row_list,
                                 int32_t count, const fie_workspace* ws, void* stream)
{
    Params P;
    int rc = fill_params(P, a, ws);
    if (rc) return rc;
    if (count <= 0) return FIE_OK;
    if (!row_list) return fail(FIE_E_ARG, "row_list is NULL");
    hipStream_t st = (hipStream_t)stream;
    for (int g0 = 0; g0 < count; g0 += kFallbackRows) {
        const int cnt = count - g0 < kFallbackRows ? count - g0 : kFallbackRows;
        hipLaunchKernelGGL(k_fallback_keys, dim3(cnt), dim3(1024), 0, st, P, row_list + g0, cnt);
        if ((rc = check_launch("k_fallback_keys"))) return rc;
        const int64_t n = P.fb_pow2;
        const int64_t threads = (int64_t)cnt * (n / 2);
        const unsigned blocks = (unsigned)((threads + 255) / 256);
        for (int64_t k = 2; k <= n; k <<= 1)
            for (int64_t j = k >> 1; j > 0; j >>= 1) {
                hipLaunchKernelGGL(k_fallback_stage, dim3(blocks), dim3(256), 0, st, P, cnt, k, j);
            }
        if ((rc = check_launch("k_fallback_stage"))) return rc;
        hipLaunchKernelGGL(k_fallback_finish, dim3(cnt), dim3(1024), 0, st, P, row_list + g0, cnt);
        if ((rc = check_launch("k_fallback_finish"))) return rc;
    }
    return FIE_OK;
}

int fie_sampler_argmax(const void* logits, int32_t dtype, int32_t rows, int32_t vocab,
                       int64_t row_stride, int64_t* tokens, const fie_workspace* ws, void* stream)
{
    Params P;
    memset(&P, 0, sizeof P);
    if (!logits || !tokens) return fail(FIE_E_ARG, "logits or tokens is NULL");
    if (dtype < FIE_F32 || dtype > FIE_BF16) return fail(FIE_E_ARG, "unknown dtype");
    if (rows <= 0 || vocab <= 0 || row_stride < vocab) return fail(FIE_E_ARG, "bad shape");
    const int es = dtype == FIE_F32 ? 4 : 2;
    P.logits = (const char*)logits;
    P.row_stride_bytes = row_stride * es;
    P.dtype = dtype;
    P.rows = rows;
    P.vocab = vocab;
    P.epc = 16 / es;
    P.vec_ok = (((uintptr_t)logits % 16) == 0 && (P.row_stride_bytes % 16) == 0) ? 1 : 0;
    choose_slices(P);
    if (P.S > kMaxSlices) return fail(FIE_E_ARG, "vocab too large for the slice table");
    P.argmax_only = 1;
    P.tokens = tokens;
    int rc = fill_layout(P, ws, rows, 0);
    if (rc) return rc;
    return launch_stage(P, FIE_STAGE_SAMPLE, (hipStream_t)stream);
}

int fie_sampler_kept(const fie_sampler_args* a, uint8_t* kept, float* probs,
                     const fie_workspace* ws, void* stream)
{
    Params P;
    int rc = fill_params(P, a, ws);
    if (rc) return rc;
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid((unsigned)(P.rows * P.S)), block(kThreads);
    if (P.dtype == FIE_F32) hipLaunchKernelGGL(k_kept<FIE_F32>, grid, block, 0, st, P, kept, probs);
    else if (P.dtype == FIE_F16) hipLaunchKernelGGL(k_kept<FIE_F16>, grid, block, 0, st, P, kept, probs);
    else hipLaunchKernelGGL(k_kept<FIE_BF16>, grid, block, 0, st, P, kept, probs);
    return check_launch("k_kept");
}

int fie_sampler_cexp(const float* in, float* out, int64_t n, void* stream)
{
    if (!in || !out || n < 0) return fail(FIE_E_ARG, "bad cexp arguments");
    if (n == 0) return FIE_OK;
    hipLaunchKernelGGL(k_cexp, dim3(1024), dim3(256), 0, (hipStream_t)stream, in, out, n);
    return check_launch("k_cexp");
}

const char* fie_sampler_last_error(void) { return g_err; }

int fie_sampler_set_trace(void* buffer)
{
    uint64_t* p = (uint64_t*)buffer;
    if (hipMemcpyToSymbol(HIP_SYMBOL(g_trace), &p, sizeof p) != hipSuccess)
        return fail(FIE_E_LAUNCH, "cannot set the trace buffer");
    return FIE_OK;
}

}  // extern "C"
