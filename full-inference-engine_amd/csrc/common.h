// Shared device helpers of the MI355X sampler: order keys, the canonical
// exponential, fixed-point weights, exact integer scaling, block scans.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define FIE_DEV __device__ __forceinline__

namespace fie {

constexpr int kThreads = 256;                 // pass kernels: 4 wave64 per workgroup
constexpr int kWaves = kThreads / 64;

// ---------------------------------------------------------------- order keys
// Order-preserving key of an fp32 value (larger value -> larger key).  Callers
// fold -0 into +0 first so equal values have equal keys.
FIE_DEV uint32_t fkey(float v)
{
    uint32_t b = __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

FIE_DEV float key_to_float(uint32_t k)
{
    uint32_t b = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
    return __uint_as_float(b);
}

constexpr uint32_t kKeyNegInf = 0x007FFFFFu;  // fkey(-inf)
constexpr uint32_t kKeyPosInf = 0xFF800000u;  // fkey(+inf)

// Rank order of the sampler: value descending, then token index ascending.
FIE_DEV uint64_t comp_key(uint32_t ykey, uint32_t idx)
{
    return ((uint64_t)ykey << 32) | (uint64_t)(0xFFFFFFFFu - idx);
}

FIE_DEV uint32_t comp_idx(uint64_t c) { return 0xFFFFFFFFu - (uint32_t)(c & 0xFFFFFFFFu); }

// The scaled logit y = w / s exactly as sampler.py:185 computes it (IEEE divide),
// with -0 folded into +0.
FIE_DEV float scaled(float w, float s) { return w / s + 0.0f; }

// ---------------------------------------------------------------- exponential
// Canonical fp32 exponential of d <= 0: Cody-Waite reduction by a two-part ln 2,
// degree-7 Taylor polynomial on |r| <= ln2/2 by Horner with fused multiply-adds,
// exact scaling by 2^n.  Every step is one IEEE binary32 operation, so any
// implementation performing the same steps returns the same bits.
FIE_DEV float cexp(float d)
{
    if (!(d > -80.0f)) return 0.0f;
    if (d >= 0.0f) return 1.0f;
    float n = __builtin_rintf(d * 1.44269502f);
    float r = __builtin_fmaf(n, -0.693145752f, d);
    r = __builtin_fmaf(n, -1.42860677e-06f, r);
    float p = 1.98412701e-04f;
    p = __builtin_fmaf(p, r, 1.38888892e-03f);
    p = __builtin_fmaf(p, r, 8.33333377e-03f);
    p = __builtin_fmaf(p, r, 4.16666679e-02f);
    p = __builtin_fmaf(p, r, 1.66666672e-01f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return __builtin_ldexpf(p, (int)n);
}

// floor(e * 2^40) of e in [0, 1]: the integer weight of a token.  e * 2^40 is an
// exact product, so the conversion only truncates.
FIE_DEV uint64_t weight_of(float e)
{
    return (uint64_t)((double)e * 1099511627776.0);
}

// ceil(p * S) for an fp32 p in (0, 1) and S < 2^63, exactly.
FIE_DEV uint64_t ceil_mul_f32(float p, uint64_t S)
{
    uint32_t b = __float_as_uint(p);
    uint32_t eb = (b >> 23) & 0xFFu;
    uint64_t mant = (b & 0x7FFFFFu) | (eb ? 0x800000u : 0u);
    int q = eb ? 150 - (int)eb : 149;
    unsigned __int128 prod = (unsigned __int128)mant * S;
    if (q >= 127) return prod ? 1 : 0;
    unsigned __int128 fl = prod >> q;
    return (uint64_t)(fl + (((fl << q) != prod) ? 1 : 0));
}

// floor(u * T) for a double u in [0, 1) and T < 2^63, exactly.
FIE_DEV uint64_t floor_mul_f64(double u, uint64_t T)
{
    if (!(u > 0.0)) return 0;
    uint64_t b = (uint64_t)__double_as_longlong(u);
    uint32_t eb = (uint32_t)((b >> 52) & 0x7FFu);
    uint64_t mant = (b & 0xFFFFFFFFFFFFFull) | (eb ? (1ull << 52) : 0ull);
    int q = eb ? 1075 - (int)eb : 1074;
    if (q >= 127) return 0;
    unsigned __int128 prod = (unsigned __int128)mant * T;
    return (uint64_t)(prod >> q);
}

// ---------------------------------------------------------------- coherence
// Workgroups of one pass hand results to the row's last workgroup without an
// agent-scope fence (which writes back and invalidates the whole L2 of an XCD):
// every value crossing workgroups is an agent-scope atomic (RMW, or a load/store
// with the sc1 coherence bit), and a writer drains its memory counters before it
// signals arrival, which orders those accesses the way the release fence would.
template <typename T>
FIE_DEV T ld_shared(const T* p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T>
FIE_DEV void st_shared(T* p, T v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

FIE_DEV void drain_memory()
{
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// ---------------------------------------------------------------- reductions
FIE_DEV uint64_t shfl_u64(uint64_t v, int src)
{
    uint32_t lo = __shfl((uint32_t)v, src, 64);
    uint32_t hi = __shfl((uint32_t)(v >> 32), src, 64);
    return ((uint64_t)hi << 32) | lo;
}

FIE_DEV uint64_t shfl_up_u64(uint64_t v, int d)
{
    uint32_t lo = __shfl_up((uint32_t)v, d, 64);
    uint32_t hi = __shfl_up((uint32_t)(v >> 32), d, 64);
    return ((uint64_t)hi << 32) | lo;
}

FIE_DEV uint64_t shfl_xor_u64(uint64_t v, int m)
{
    uint32_t lo = __shfl_xor((uint32_t)v, m, 64);
    uint32_t hi = __shfl_xor((uint32_t)(v >> 32), m, 64);
    return ((uint64_t)hi << 32) | lo;
}

FIE_DEV uint64_t wave_max_u64(uint64_t v)
{
    for (int m = 32; m > 0; m >>= 1) {
        uint64_t o = shfl_xor_u64(v, m);
        v = o > v ? o : v;
    }
    return v;
}

FIE_DEV uint64_t wave_min_u64(uint64_t v)
{
    for (int m = 32; m > 0; m >>= 1) {
        uint64_t o = shfl_xor_u64(v, m);
        v = o < v ? o : v;
    }
    return v;
}

FIE_DEV uint64_t wave_sum_u64(uint64_t v)
{
    for (int m = 32; m > 0; m >>= 1) v += shfl_xor_u64(v, m);
    return v;
}

FIE_DEV uint32_t wave_max_u32(uint32_t v)
{
    for (int m = 32; m > 0; m >>= 1) {
        uint32_t o = __shfl_xor(v, m, 64);
        v = o > v ? o : v;
    }
    return v;
}

// Inclusive scan over the 64 lanes of a wave.
FIE_DEV uint64_t wave_incl_scan_u64(uint64_t v)
{
    const int lane = threadIdx.x & 63;
    for (int d = 1; d < 64; d <<= 1) {
        uint64_t o = shfl_up_u64(v, d);
        if (lane >= d) v += o;
    }
    return v;
}

// Block-wide exclusive scan of one u64 per thread (blockDim.x == nthreads, a
// multiple of 64, at most 1024).  `scratch` holds nthreads/64 + 1 values.
template <int NT>
FIE_DEV uint64_t block_excl_scan_u64(uint64_t v, uint64_t* scratch, uint64_t* total)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint64_t incl = wave_incl_scan_u64(v);
    if (lane == 63) scratch[wave] = incl;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t run = 0;
        for (int w = 0; w < NT / 64; ++w) {
            uint64_t t = scratch[w];
            scratch[w] = run;
            run += t;
        }
        scratch[NT / 64] = run;
    }
    __syncthreads();
    uint64_t res = scratch[wave] + incl - v;
    *total = scratch[NT / 64];
    __syncthreads();
    return res;
}

template <int NT>
FIE_DEV uint64_t block_sum_u64(uint64_t v, uint64_t* scratch)
{
    v = wave_sum_u64(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    uint64_t t = 0;
    for (int w = 0; w < NT / 64; ++w) t += scratch[w];
    __syncthreads();
    return t;
}

template <int NT>
FIE_DEV uint64_t block_max_u64(uint64_t v, uint64_t* scratch)
{
    v = wave_max_u64(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    uint64_t t = 0;
    for (int w = 0; w < NT / 64; ++w) t = scratch[w] > t ? scratch[w] : t;
    __syncthreads();
    return t;
}

template <int NT>
FIE_DEV uint64_t block_min_u64(uint64_t v, uint64_t* scratch)
{
    v = wave_min_u64(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    uint64_t t = ~0ull;
    for (int w = 0; w < NT / 64; ++w) t = scratch[w] < t ? scratch[w] : t;
    __syncthreads();
    return t;
}

// In-LDS bitonic sort of n (a power of two) u64 keys into descending order.
template <int NT>
FIE_DEV void bitonic_sort_desc(uint64_t* key, int n)
{
    for (int k = 2; k <= n; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < n; i += NT) {
                int ixj = i ^ j;
                if (ixj > i) {
                    uint64_t a = key[i], b = key[ixj];
                    bool up = (i & k) != 0;            // this pair ends ascending
                    if (up ? (a > b) : (a < b)) {
                        key[i] = b;
                        key[ixj] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
}

FIE_DEV int pow2_at_least(int n)
{
    int p = 64;
    while (p < n) p <<= 1;
    return p;
}

}  // namespace fie
