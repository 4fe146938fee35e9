// MI355X fused token sampler: kernels behind the C ABI of include/fie_sampler.h.
//
//   k_prep      penalty histories bucketed by span                (here)
//   k_scan      one streaming read of the logits, tile partials   (scan.h)
//   k_finish    one workgroup per row: exact selection and draw   (finish.h)
//   k_argmax_*  the greedy fast path, logits.argmax(-1)           (sampler.py:106)
//   k_kept      kept set / probabilities of the last step (verification aid)
//   k_cexp      the canonical exponential (verification aid)
//   k_uniforms  the on-device counter-based draws (verification aid)
//   k_history_write  appends tokens to a device-resident penalty history
#include <hip/hip_runtime.h>

#include <stdio.h>
#include <string.h>

#include <mutex>

#include "launchers.h"
#include "fie_sampler.h"

namespace fie {

// ---------------------------------------------------------------- k_prep
// Buckets the history of every penalised row by span (sampler.py:134-144 counts
// the same ids): the offsets inside the span of the first kBucketCap ids of each
// span, the number of ids per span, the occurrences of token 0 and of ids >= vocab.
// Each k_scan workgroup then reads its own span's bucket instead of the whole
// history.  The order inside a bucket is free: only counts are taken from it.
__global__ __launch_bounds__(kPrepThreads) void k_prep(const KParams P)
{
    __shared__ uint32_t sc[kMaxSpans];
    __shared__ uint32_t zc, badc;
    const fie_sampler_args& a = P.a;
    const int row = blockIdx.x, tid = threadIdx.x, NS = P.NS;
    const uint32_t V = (uint32_t)a.vocab;
    // the row's flags and history range are loaded together (one round trip)
    const int32_t fl = a.flags[row];
    const int64_t h0 = a.hist_offsets[row], h1 = hist_end(a, row);
    if (!(a.apply_penalties && (fl & FIE_FLAG_PENALTY))) return;
    if (tid < NS) sc[tid] = 0;
    if (tid == 0) { zc = 0; badc = 0; }
    __syncthreads();
    uint16_t* bk = P.w.bk + (size_t)row * NS * kBucketCap;
    constexpr int kPer = 8;   // ids per thread per batch, loaded together
    for (int64_t base = h0; base < h1; base += (int64_t)kPer * kPrepThreads) {
        uint32_t ids[kPer];
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            const int64_t h = base + q * kPrepThreads + tid;
            ids[q] = h < h1 ? (uint32_t)a.hist_ids[h] : 0xFFFFFFFFu;
        }
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            const uint32_t id = ids[q];
            if (id == 0) {
                atomicAdd(&zc, 1u);
            } else if (id < V) {
                const uint32_t sp = id / (uint32_t)kSpan;
                const uint32_t at = atomicAdd(&sc[sp], 1u);
                if (at < (uint32_t)kBucketCap) bk[sp * kBucketCap + at] = (uint16_t)(id % (uint32_t)kSpan);
            } else if (base + q * kPrepThreads + tid < h1) {
                atomicAdd(&badc, 1u);
            }
        }
    }
    __syncthreads();
    if (tid < NS) P.w.nb[(size_t)row * NS + tid] = sc[tid];
    if (tid == 0) {
        P.w.tok0c[row] = zc;
        P.w.bad[row] = badc;
    }
}

// ---------------------------------------------------------------- greedy fast path
constexpr int kArgChunk = 8192;   // tokens per workgroup of the argmax pass

// Chunk maxima of the raw logits (token 0 included, no penalties, no scaling).
template <int DT, bool VEC>
__global__ __launch_bounds__(kScanThreads) void k_argmax_scan(const void* logits, int V,
                                                              int64_t stride, int NT,
                                                              uint64_t* maxc)
{
    constexpr int EPL = DTy<DT>::EPL, SZ = DTy<DT>::SZ, NL = kArgChunk / kScanThreads / EPL;
    __shared__ uint32_t scr[32];
    const int tile = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    const int lo = tile * kArgChunk;
    const char* rowp = (const char*)logits + (size_t)row * (size_t)stride * SZ;
    uint4 raw[NL];
#pragma unroll
    for (int j = 0; j < NL; ++j) raw[j] = load_group<DT, VEC>(rowp, lo + (j * kScanThreads + tid) * EPL, V);
    uint32_t tm = 0, ti = 0xFFFFFFFFu;
#pragma unroll
    for (int j = 0; j < NL; ++j) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const int idx = lo + (j * kScanThreads + tid) * EPL + e;
            const uint32_t k = idx < V ? fkey(lane_get<DT>(raw[j], e) + 0.0f) : 0u;
            if (k > tm) { tm = k; ti = (uint32_t)idx; }
        }
    }
    const uint32_t km = block_max_u32<kScanThreads>(tm, scr);
    const uint32_t fi = block_min_u32<kScanThreads>(tm == km ? ti : 0xFFFFFFFFu, scr);
    if (tid == 0) maxc[(size_t)row * NT + tile] = km ? comp_key(km, fi) : 0ull;
}

__global__ __launch_bounds__(64) void k_argmax_finish(const uint64_t* maxc, int NT, int rows,
                                                      int64_t* tokens)
{
    const int row = blockIdx.x * 64 + threadIdx.x;
    if (row >= rows) return;
    uint64_t best = 0;
    for (int t = 0; t < NT; ++t) {
        const uint64_t c = maxc[(size_t)row * NT + t];
        best = c > best ? c : best;
    }
    tokens[row] = best ? (int64_t)comp_idx(best) : 0;
}

// ---------------------------------------------------------------- kept set
template <int DT, bool VEC>
__global__ __launch_bounds__(kScanThreads) void k_kept(const KParams P, uint8_t* kept, float* probs)
{
    constexpr int EPL = DTy<DT>::EPL, SZ = DTy<DT>::SZ, NL = kArgChunk / kScanThreads / EPL;
    __shared__ uint32_t cnt[kArgChunk];
    const fie_sampler_args& a = P.a;
    const int row = blockIdx.y, tid = threadIdx.x;
    const int NT = P.NT, V = a.vocab;
    const int lo = blockIdx.x * kArgChunk, hi = min(lo + kArgChunk, V);
    const RowRes rr = P.w.res[row];
    const bool pen = a.apply_penalties && (a.flags[row] & FIE_FLAG_PENALTY);
    const float* mt = P.w.mt + (size_t)row * (NT + 1);
    const uint64_t* ct = P.w.ct + (size_t)row * (NT + 1);
    const u128 T = ((u128)rr.khi << 64) | rr.klo;
    const double Td = u128_to_double(T);
    float rep = 1.0f, pres = 0.0f, freq = 0.0f;
    if (pen) {
        rep = a.repetition[row];
        pres = a.presence[row];
        freq = a.frequency[row];
        for (int i = tid; i < kArgChunk; i += kScanThreads) cnt[i] = 0;
        __syncthreads();
        const int64_t h0 = a.hist_offsets[row], h1 = hist_end(a, row);
        for (int64_t h = h0 + tid; h < h1; h += kScanThreads) {
            const uint32_t id = (uint32_t)a.hist_ids[h];
            if (id >= (uint32_t)lo && id < (uint32_t)hi && id != 0) atomicAdd(&cnt[id - lo], 1u);
        }
        __syncthreads();
    }
    const char* rowp = (const char*)a.logits + (size_t)row * (size_t)a.row_stride * SZ;
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        const int e0 = lo + (j * kScanThreads + tid) * EPL;
        const uint4 raw = load_group<DT, VEC>(rowp, e0, V);
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const int idx = e0 + e;
            if (idx >= V) continue;
            float y;
            int slot;
            if (idx == 0) {
                y = mt[0];
                slot = 0;
            } else {
                float x = lane_get<DT>(raw, e);
                if (pen && cnt[idx - lo]) x = penalize(x, rep, pres, freq, cnt[idx - lo]);
                y = rr.s == 1.0f ? x + 0.0f : scaled(x, rr.s);
                slot = 1 + idx / kTile;
            }
            const uint64_t c = comp_key(fkey(y), (uint32_t)idx);
            bool k;
            float p;
            if (rr.greedy) {
                k = true;
                p = idx == rr.token ? 1.0f : 0.0f;
            } else {
                k = comp_k(c) >= rr.tau && c >= rr.cut;
                const u128 w = (u128)tok_weight(y, mt[slot]) * ct[slot];
                p = (k && T > 0) ? (float)(u128_to_double(w) / Td) : 0.0f;
            }
            const size_t o = (size_t)row * V + idx;
            if (kept) kept[o] = k ? 1 : 0;
            if (probs) probs[o] = p;
        }
    }
}

__global__ void k_history_write(int32_t* ids, const int64_t* dst, const int32_t* src, int64_t n)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) ids[dst[i]] = src[i];
}

__global__ void k_uniforms(const uint64_t* rng, double* out, int32_t rows)
{
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r < rows) out[r] = philox_uniform(rng + 3 * (size_t)r);
}

__global__ void k_cexp(const float* in, float* out, int64_t n)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = cexp(in[i]);
}

// ---------------------------------------------------------------- host side
static thread_local char g_err[512];

static int fail(int code, const char* msg)
{
    snprintf(g_err, sizeof g_err, "%s", msg);
    return code;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct Layout {
    size_t maxc, sw, bound, ncand, nu, nb, bk, cand, tok0x, tok0c, bad, res, mt, ct, dq, dqrows, dfr;
    size_t harr, hmk, hpc, hlo, hhi, hoff, hcomp;   // span helpers (0: none)
    size_t total;
};

static bool layout_of(int32_t R, int32_t V, Layout* L)
{
    if (R < 0 || V < 1 || V > kMaxTiles * kTile) return false;
    const size_t NT = (size_t)(V + kTile - 1) / kTile;
    const size_t r = (size_t)(R > 0 ? R : 1);
    size_t o = 0;
    auto take = [&](size_t bytes) { size_t at = o; o = align256(o + bytes); return at; };
    L->maxc = take(r * NT * 8);
    L->sw = take(r * NT * 8);
    L->bound = take(r * NT * 4);
    L->ncand = take(r * NT * 4);
    L->nu = take(r * NT * 4);
    const size_t NS = (NT + kWavesPerWG - 1) / kWavesPerWG;
    L->nb = take(r * NS * 4);
    L->bk = take(r * NS * kBucketCap * 2);
    L->cand = take(r * NT * kCapW * 8);
    L->tok0x = take(r * 4);
    L->tok0c = take(r * 4);
    L->bad = take(r * 4);
    L->res = take(r * sizeof(RowRes));
    L->mt = take(r * (NT + 1) * 4);
    L->ct = take(r * (NT + 1) * 8);
    L->dq = take(2 * 4);
    L->dqrows = take(r * 4);
    L->dfr = take(r * sizeof(DeferRec));
    // span helpers of k_finish: only workspaces for at most kHelpRows rows hold them
    L->harr = L->hmk = L->hpc = L->hlo = L->hhi = L->hoff = L->hcomp = 0;
    if (R <= kHelpRows) {
        L->harr = take(r * 4);
        L->hmk = take(r * NS * 4);
        L->hpc = take(r * NS * kHBins * 4);
        L->hlo = take(r * NS * kHBins * 8);
        L->hhi = take(r * NS * kHBins * 8);
        L->hoff = take(r * NS * kHOffs * 4);
        L->hcomp = take(r * NS * kSpan * 8);
    }
    L->total = o;
    return true;
}

static int ws_of(const fie_workspace* ws, int32_t rows, int32_t V, Ws* w)
{
    if (!ws || !ws->ptr) return fail(FIE_E_WORKSPACE, "workspace missing");
    if (((uintptr_t)ws->ptr & 255u) != 0) return fail(FIE_E_WORKSPACE, "workspace not 256-byte aligned");
    if (rows > ws->max_rows || V > ws->vocab) return fail(FIE_E_WORKSPACE, "workspace sized for fewer rows or a smaller vocabulary");
    Layout L;
    if (!layout_of(ws->max_rows, ws->vocab, &L)) return fail(FIE_E_WORKSPACE, "workspace sizes invalid");
    if (ws->bytes < L.total) return fail(FIE_E_WORKSPACE, "workspace too small");
    // Offsets follow the workspace's own (max_rows, vocab), so one workspace serves
    // every smaller call; rows index the arrays with the call's own NT, which is no
    // larger than the workspace's.
    char* b = (char*)ws->ptr;
    w->maxc = (uint64_t*)(b + L.maxc);
    w->sw = (uint64_t*)(b + L.sw);
    w->bound = (uint32_t*)(b + L.bound);
    w->ncand = (uint32_t*)(b + L.ncand);
    w->nu = (uint32_t*)(b + L.nu);
    w->nb = (uint32_t*)(b + L.nb);
    w->bk = (uint16_t*)(b + L.bk);
    w->cand = (uint64_t*)(b + L.cand);
    w->tok0x = (float*)(b + L.tok0x);
    w->tok0c = (uint32_t*)(b + L.tok0c);
    w->bad = (uint32_t*)(b + L.bad);
    w->res = (RowRes*)(b + L.res);
    w->mt = (float*)(b + L.mt);
    w->ct = (uint64_t*)(b + L.ct);
    w->dq = (uint32_t*)(b + L.dq);
    w->dqrows = (uint32_t*)(b + L.dqrows);
    w->dfr = (DeferRec*)(b + L.dfr);
    const bool h = L.harr != 0;
    w->harr = h ? (uint32_t*)(b + L.harr) : nullptr;
    w->hmk = h ? (uint32_t*)(b + L.hmk) : nullptr;
    w->hpc = h ? (uint32_t*)(b + L.hpc) : nullptr;
    w->hlo = h ? (uint64_t*)(b + L.hlo) : nullptr;
    w->hhi = h ? (uint64_t*)(b + L.hhi) : nullptr;
    w->hoff = h ? (uint32_t*)(b + L.hoff) : nullptr;
    w->hcomp = h ? (uint64_t*)(b + L.hcomp) : nullptr;
    return FIE_OK;
}

static int check_args(const fie_sampler_args* a)
{
    if (!a) return fail(FIE_E_ARG, "args is NULL");
    if (a->dtype < FIE_F32 || a->dtype > FIE_BF16) return fail(FIE_E_ARG, "unknown dtype");
    if (a->rows < 0) return fail(FIE_E_ARG, "rows < 0");
    if (a->vocab < 1 || a->vocab > kMaxTiles * kTile) return fail(FIE_E_ARG, "vocab out of range [1, 524288]");
    if (a->lp_cols < 0 || a->lp_cols > 20) return fail(FIE_E_ARG, "lp_cols out of range [0, 20]");
    if (a->row_stride < a->vocab) return fail(FIE_E_ARG, "row_stride < vocab");
    if (a->rows == 0) return FIE_OK;
    if (!a->logits || !a->tokens || !a->scale || !a->top_k || !a->top_p || !a->min_p || !a->flags ||
        (!a->uniform && !a->rng))
        return fail(FIE_E_ARG, "a required pointer is NULL");
    if (a->apply_penalties && (!a->repetition || !a->presence || !a->frequency || !a->hist_offsets || !a->hist_ids))
        return fail(FIE_E_ARG, "penalties applied but a penalty pointer is NULL");
    if (a->lp_cols > 0 && a->logprobs && (!a->top_ids && !a->top_logprobs))
        return fail(FIE_E_ARG, "lp_cols > 0 but no top-logprob output");
    return FIE_OK;
}

static bool vec_ok(const void* p, int64_t stride, int sz)
{
    return ((uintptr_t)p % 16) == 0 && ((stride * sz) % 16) == 0;
}

#define FIE_LAUNCH_CHECK(what)                                                          \
    do {                                                                                \
        hipError_t e_ = hipGetLastError();                                              \
        if (e_ != hipSuccess) {                                                         \
            snprintf(g_err, sizeof g_err, "%s: %s", what, hipGetErrorString(e_));       \
            return FIE_E_LAUNCH;                                                        \
        }                                                                               \
    } while (0)

static int launch_status(hipError_t e, const char* what)
{
    if (e == hipSuccess) return FIE_OK;
    snprintf(g_err, sizeof g_err, "%s: %s", what, hipGetErrorString(e));
    return FIE_E_LAUNCH;
}

// Compute units of the current device (queried once per device; 0 when unknown,
// which selects the narrow k_finish).
static int cu_count()
{
    static int cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = -1;
        cus[dev] = n;
    }
    return cus[dev] > 0 ? cus[dev] : 0;
}

// With no more rows than CUs, k_finish runs the wide variant, which takes a row its
// candidates cannot settle through the full-row path itself: k_deep has no queue.
static bool finish_in_place(const KParams& P) { return P.a.rows <= cu_count(); }

static int run_stage(const KParams& P, int stage, hipStream_t st)
{
    const int sz = P.a.dtype == FIE_F32 ? 4 : 2;
    const bool vec = vec_ok(P.a.logits, P.a.row_stride, sz);
    const bool longh = P.a.apply_penalties && P.a.max_row_hist > 65535;
    if (stage == FIE_STAGE_PREP) {
        if (P.a.apply_penalties) {
            k_prep<<<P.a.rows, kPrepThreads, 0, st>>>(P);
            FIE_LAUNCH_CHECK("k_prep");
        }
        return FIE_OK;
    }
    hipError_t e;
    const char* what;
    if (stage == FIE_STAGE_SCAN) {
        e = launch_scan(P, vec, longh, st);
        what = "k_scan";
    } else {
        const bool deep = stage == FIE_STAGE_DEEP;
        const bool wide = finish_in_place(P);
        switch (P.a.dtype) {
        case FIE_F32: e = launch_finish_f32(P, vec, deep, wide, st); break;
        case FIE_F16: e = launch_finish_f16(P, vec, deep, wide, st); break;
        default: e = launch_finish_bf16(P, vec, deep, wide, st); break;
        }
        what = deep ? "k_deep" : "k_finish";
    }
    return launch_status(e, what);
}

static int prepare(const fie_sampler_args* args, const fie_workspace* ws, KParams* P)
{
    int rc = check_args(args);
    if (rc != FIE_OK) return rc;
    P->a = *args;
    P->NT = (args->vocab + kTile - 1) / kTile;
    P->NS = (P->NT + kWavesPerWG - 1) / kWavesPerWG;
    P->helpers = 0;
    if (args->rows == 0) return FIE_OK;
    rc = ws_of(ws, args->rows, args->vocab, &P->w);
    if (rc != FIE_OK) return rc;
    // small batches, settled in place by the wide k_finish, in a workspace that
    // holds the helpers' arrays
    P->helpers = (P->w.harr && args->rows <= kHelpRows && finish_in_place(*P)) ? 1 : 0;
    return FIE_OK;
}

// ---------------------------------------------------------------- static scratch
// The workspace of fie_sampler_sample_noalloc: a device array per GPU, reached
// through the address hipGetSymbolAddress returns on that device (the array's
// name is a host-side stand-in, never a device address).
static __device__ __align__(256) unsigned char scratch[FIE_SCRATCH_BYTES];
constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch[kMaxDevices];

static int scratch_of(void** out)
{
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) return fail(FIE_E_LAUNCH, "hipGetDevice failed");
    if (dev < 0 || dev >= kMaxDevices) return fail(FIE_E_ARG, "device ordinal out of range [0, 64)");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            snprintf(g_err, sizeof g_err, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
            return FIE_E_LAUNCH;
        }
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return FIE_OK;
}

}  // namespace fie

using namespace fie;

extern "C" {

size_t fie_sampler_workspace_size(int32_t max_rows, int32_t vocab)
{
    Layout L;
    return layout_of(max_rows, vocab, &L) ? L.total : 0;
}

int fie_sampler_sample(const fie_sampler_args* args, const fie_workspace* ws, void* stream)
{
    KParams P;
    int rc = prepare(args, ws, &P);
    if (rc != FIE_OK || args->rows == 0) return rc;
    hipStream_t st = (hipStream_t)stream;
    rc = run_stage(P, FIE_STAGE_PREP, st);
    if (rc != FIE_OK) return rc;
    rc = run_stage(P, FIE_STAGE_SCAN, st);
    if (rc != FIE_OK) return rc;
    rc = run_stage(P, FIE_STAGE_FINISH, st);
    if (rc != FIE_OK || finish_in_place(P)) return rc;
    return run_stage(P, FIE_STAGE_DEEP, st);
}

static int lmhead_run(const fie_sampler_args* args, const void* hidden, const void* weight, int32_t hidden_dim,
                      const fie_workspace* ws, void* stream, bool whole)
{
    if (!args) return fail(FIE_E_ARG, "args is NULL");
    if (args->dtype != FIE_F16 && args->dtype != FIE_BF16)
        return fail(FIE_E_ARG, "the fused lm_head takes fp16 or bf16 (the logits dtype is the model's)");
    if (hidden_dim < kLhKAlign || hidden_dim % kLhKAlign != 0)
        return fail(FIE_E_ARG, "hidden_dim must be a positive multiple of 128");
    KParams P;
    int rc = prepare(args, ws, &P);
    if (rc != FIE_OK || args->rows == 0) return rc;
    if (!hidden || !weight) return fail(FIE_E_ARG, "hidden or weight is NULL");
    if (((uintptr_t)hidden % 16) != 0 || ((uintptr_t)weight % 16) != 0)
        return fail(FIE_E_ARG, "hidden and weight must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    if (whole) {
        rc = run_stage(P, FIE_STAGE_PREP, st);
        if (rc != FIE_OK) return rc;
    }
    const bool vec = vec_ok(args->logits, args->row_stride, 2);
    const bool longh = args->apply_penalties && args->max_row_hist > 65535;
    rc = launch_status(launch_lmhead(P, hidden, weight, hidden_dim, vec, longh, st), "k_lmhead");
    if (rc != FIE_OK || !whole) return rc;
    rc = run_stage(P, FIE_STAGE_FINISH, st);
    if (rc != FIE_OK || finish_in_place(P)) return rc;
    return run_stage(P, FIE_STAGE_DEEP, st);
}

int fie_sampler_lmhead_sample(const fie_sampler_args* args, const void* hidden, const void* weight,
                              int32_t hidden_dim, const fie_workspace* ws, void* stream)
{
    return lmhead_run(args, hidden, weight, hidden_dim, ws, stream, true);
}

int fie_sampler_lmhead_stage(const fie_sampler_args* args, const void* hidden, const void* weight,
                             int32_t hidden_dim, const fie_workspace* ws, void* stream)
{
    return lmhead_run(args, hidden, weight, hidden_dim, ws, stream, false);
}

int fie_sampler_stage(const fie_sampler_args* args, const fie_workspace* ws, int32_t stage, void* stream)
{
    if (stage != FIE_STAGE_PREP && stage != FIE_STAGE_SCAN && stage != FIE_STAGE_FINISH &&
        stage != FIE_STAGE_DEEP)
        return fail(FIE_E_ARG, "unknown stage");
    KParams P;
    int rc = prepare(args, ws, &P);
    if (rc != FIE_OK || args->rows == 0) return rc;
    return run_stage(P, stage, (hipStream_t)stream);
}

int fie_sampler_argmax(const void* logits, int32_t dtype, int32_t rows, int32_t vocab,
                       int64_t row_stride, int64_t* tokens, const fie_workspace* ws, void* stream)
{
    if (dtype < FIE_F32 || dtype > FIE_BF16) return fail(FIE_E_ARG, "unknown dtype");
    if (rows < 0 || vocab < 1 || vocab > kMaxTiles * kTile || row_stride < vocab)
        return fail(FIE_E_ARG, "sizes out of range");
    if (rows == 0) return FIE_OK;
    if (!logits || !tokens) return fail(FIE_E_ARG, "a required pointer is NULL");
    Ws w;
    int rc = ws_of(ws, rows, vocab, &w);
    if (rc != FIE_OK) return rc;
    const int NT = (vocab + kArgChunk - 1) / kArgChunk;
    const int sz = dtype == FIE_F32 ? 4 : 2;
    const bool vec = vec_ok(logits, row_stride, sz);
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid(NT, rows);
#define FIE_ARGMAX(DT)                                                                                   \
    if (vec) k_argmax_scan<DT, true><<<grid, kScanThreads, 0, st>>>(logits, vocab, row_stride, NT, w.maxc); \
    else k_argmax_scan<DT, false><<<grid, kScanThreads, 0, st>>>(logits, vocab, row_stride, NT, w.maxc);
    switch (dtype) {
    case FIE_F32: FIE_ARGMAX(FIE_F32) break;
    case FIE_F16: FIE_ARGMAX(FIE_F16) break;
    default: FIE_ARGMAX(FIE_BF16) break;
    }
#undef FIE_ARGMAX
    FIE_LAUNCH_CHECK("k_argmax_scan");
    k_argmax_finish<<<(rows + 63) / 64, 64, 0, st>>>(w.maxc, NT, rows, tokens);
    FIE_LAUNCH_CHECK("k_argmax_finish");
    return FIE_OK;
}

int fie_sampler_kept(const fie_sampler_args* args, uint8_t* kept, float* probs,
                     const fie_workspace* ws, void* stream)
{
    KParams P;
    int rc = prepare(args, ws, &P);
    if (rc != FIE_OK || args->rows == 0) return rc;
    const int sz = args->dtype == FIE_F32 ? 4 : 2;
    const bool vec = vec_ok(args->logits, args->row_stride, sz);
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid((args->vocab + kArgChunk - 1) / kArgChunk, args->rows);
#define FIE_KEPT(DT)                                                                  \
    if (vec) k_kept<DT, true><<<grid, kScanThreads, 0, st>>>(P, kept, probs);        \
    else k_kept<DT, false><<<grid, kScanThreads, 0, st>>>(P, kept, probs);
    switch (args->dtype) {
    case FIE_F32: FIE_KEPT(FIE_F32) break;
    case FIE_F16: FIE_KEPT(FIE_F16) break;
    default: FIE_KEPT(FIE_BF16) break;
    }
#undef FIE_KEPT
    FIE_LAUNCH_CHECK("k_kept");
    return FIE_OK;
}

int fie_sampler_cexp(const float* in, float* out, int64_t n, void* stream)
{
    if (n < 0 || (n > 0 && (!in || !out))) return fail(FIE_E_ARG, "bad cexp arguments");
    if (n == 0) return FIE_OK;
    k_cexp<<<(unsigned)((n + 255) / 256), 256, 0, (hipStream_t)stream>>>(in, out, n);
    FIE_LAUNCH_CHECK("k_cexp");
    return FIE_OK;
}

int fie_sampler_history_write(int32_t* ids, const int64_t* dst, const int32_t* src, int64_t n,
                              void* stream)
{
    if (n < 0 || (n > 0 && (!ids || !dst || !src))) return fail(FIE_E_ARG, "bad history_write arguments");
    if (n == 0) return FIE_OK;
    k_history_write<<<(unsigned)((n + 255) / 256), 256, 0, (hipStream_t)stream>>>(ids, dst, src, n);
    FIE_LAUNCH_CHECK("k_history_write");
    return FIE_OK;
}

int fie_sampler_uniforms(const uint64_t* rng, double* out, int32_t rows, void* stream)
{
    if (rows < 0 || (rows > 0 && (!rng || !out))) return fail(FIE_E_ARG, "bad uniforms arguments");
    if (rows == 0) return FIE_OK;
    k_uniforms<<<(rows + 255) / 256, 256, 0, (hipStream_t)stream>>>(rng, out, rows);
    FIE_LAUNCH_CHECK("k_uniforms");
    return FIE_OK;
}

const char* fie_sampler_last_error(void) { return g_err; }

int fie_sampler_sample_noalloc(const fie_sampler_args* args, void* stream)
{
    int rc = check_args(args);
    if (rc != FIE_OK || args->rows == 0) return rc;
    Layout L;
    if (!layout_of(args->rows, args->vocab, &L)) return fail(FIE_E_ARG, "sizes out of range");
    int32_t ws_rows = args->rows;
    if (L.total > FIE_SCRATCH_BYTES && ws_rows <= kHelpRows) {
        // the span helpers' arrays do not fit: lay the array out without them
        ws_rows = kHelpRows + 1;
        if (!layout_of(ws_rows, args->vocab, &L)) return fail(FIE_E_ARG, "sizes out of range");
    }
    if (L.total > FIE_SCRATCH_BYTES)
        return fail(FIE_E_WORKSPACE, "rows x vocab need more than the 64 MiB static scratch");
    void* p = nullptr;
    rc = scratch_of(&p);
    if (rc != FIE_OK) return rc;
    const fie_workspace ws{p, FIE_SCRATCH_BYTES, ws_rows, args->vocab};
    return fie_sampler_sample(args, &ws, stream);
}

}  // extern "C"
