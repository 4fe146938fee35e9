// Device helpers of the MI355X sampler: order keys, the canonical exponential,
// fixed-point weights, exact 128/192-bit integer scaling, wave64 and block
// reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define FIE_DEV __device__ __forceinline__

namespace fie {

typedef unsigned __int128 u128;

// Tokens per tile.  Part of the canonical weight rule: a token's weight is taken
// relative to the largest scaled logit of its tile (token 0 is a tile of its own,
// then [1, kTile), [kTile, 2 kTile), ...).
constexpr int kTile = 2048;

// ---------------------------------------------------------------- order keys
// Order-preserving key of an fp32 value: larger value -> larger key.  Callers fold
// -0 into +0 first (v + 0.0f) so equal values have equal keys.  Keys of non-NaN
// values are never 0, which the kernels use as "no element".
FIE_DEV uint32_t fkey(float v)
{
    uint32_t b = __float_as_uint(v);
    return b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
}

FIE_DEV float key_to_float(uint32_t k)
{
    uint32_t b = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
    return __uint_as_float(b);
}

constexpr uint32_t kKeyNegInf = 0x007FFFFFu;  // fkey(-inf)
constexpr uint32_t kKeyPosInf = 0xFF800000u;  // fkey(+inf)

// Rank order of the sampler: value descending, then token index ascending, as one
// u64 compared descending.
FIE_DEV uint64_t comp_key(uint32_t key, uint32_t idx)
{
    return ((uint64_t)key << 32) | (uint64_t)(0xFFFFFFFFu - idx);
}
FIE_DEV uint32_t comp_idx(uint64_t c) { return 0xFFFFFFFFu - (uint32_t)c; }
FIE_DEV uint32_t comp_k(uint64_t c) { return (uint32_t)(c >> 32); }

// The scaled logit exactly as sampler.py:185 computes it (IEEE fp32 divide), with
// -0 folded into +0.
FIE_DEV float scaled(float w, float s) { return w / s + 0.0f; }

// ---------------------------------------------------------------- exponential
// Canonical fp32 exponential of d <= 0: 0 for d <= -80 (and -inf, NaN), 1 for
// d >= 0, otherwise Cody-Waite reduction by a two-part ln 2, a degree-7 Taylor
// polynomial on |r| <= ln2/2 by Horner with fused multiply-adds, and an exact
// scaling by 2^n.  Each step is one IEEE binary32 operation, so any
// implementation performing the same steps returns the same bits.
//
// cexp_scaled(d, extra) is cexp(d) * 2^extra, computed without branches: the
// polynomial runs on max(d, -80) and the two special cases are selected after.
// The final ldexp is exact for the small `extra` used here because cexp(d) >=
// 2^-116 stays normal on (-80, 0).
FIE_DEV float cexp_scaled(float d, int extra)
{
    const float dc = __builtin_fmaxf(d, -80.0f);
    const float n = __builtin_rintf(dc * 1.44269502f);
    float r = __builtin_fmaf(n, -0.693145752f, dc);
    r = __builtin_fmaf(n, -1.42860677e-06f, r);
    float p = 1.98412701e-04f;
    p = __builtin_fmaf(p, r, 1.38888892e-03f);
    p = __builtin_fmaf(p, r, 8.33333377e-03f);
    p = __builtin_fmaf(p, r, 4.16666679e-02f);
    p = __builtin_fmaf(p, r, 1.66666672e-01f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const float v = __builtin_ldexpf(p, (int)n + extra);
    const float one = __builtin_ldexpf(1.0f, extra);
    return (d > -80.0f) ? ((d >= 0.0f) ? one : v) : 0.0f;
}

FIE_DEV float cexp(float d) { return cexp_scaled(d, 0); }

// floor(cexp(d) * 2^40) for d <= 0 or NaN, the token weight, as an integer-valued
// float (< 2^41).  Without the special cases of cexp: on d <= -80 (and NaN, via the
// clamp) the polynomial at -80 is below 2^-40 and floors to 0 exactly as cexp's 0
// does, and at d = 0 the polynomial is exactly 1.  p * 2^(n + 40) is exact since
// n >= -115 keeps it normal.
FIE_DEV float weight40(float d)
{
    const float dc = d > -80.0f ? d : -80.0f;
    const float n = __builtin_rintf(dc * 1.44269502f);
    float r = __builtin_fmaf(n, -0.693145752f, dc);
    r = __builtin_fmaf(n, -1.42860677e-06f, r);
    float p = 1.98412701e-04f;
    p = __builtin_fmaf(p, r, 1.38888892e-03f);
    p = __builtin_fmaf(p, r, 8.33333377e-03f);
    p = __builtin_fmaf(p, r, 4.16666679e-02f);
    p = __builtin_fmaf(p, r, 1.66666672e-01f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return __builtin_floorf(__builtin_ldexpf(p, (int)n + 40));
}

// x / s correctly rounded by Markstein's correction from r = RN(1/s):
// q = RN(x r), e = x - q s (exact by FMA), RN(q + e r).  Exact (equal to the IEEE
// quotient) when the quotient and the intermediates stay normal; callers keep
// 2^-96 <= |x| <= 2^96 and 2^-30 <= s <= 2^30 and divide directly otherwise.  Checked
// against the IEEE divide on every fp16 and bf16 input and on random fp32 inputs
// (the oracle's markstein check).
FIE_DEV float div_markstein(float x, float s, float r)
{
    const float q = x * r;
    const float e = __builtin_fmaf(-q, s, x);
    return __builtin_fmaf(e, r, q);
}

FIE_DEV bool markstein_ok(float x)
{
    const float a = __builtin_fabsf(x);
    return a >= 0x1p-96f && a <= 0x1p96f;
}

// ---------------------------------------------------------------- counter-based draws
// Philox4x64-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as
// 1, 2, 3", SC 2011): ten rounds of two 64x64->128 multiplies by the published
// multipliers, the key bumped by the published Weyl constants between rounds.
FIE_DEV void philox4x64_10(uint64_t (&x)[4], uint64_t k0, uint64_t k1)
{
    constexpr uint64_t kM0 = 0xD2E7470EE14C6C93ull, kM1 = 0xCA5A826395121157ull;
    constexpr uint64_t kW0 = 0x9E3779B97F4A7C15ull, kW1 = 0xBB67AE8584CAA73Bull;
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        if (r) { k0 += kW0; k1 += kW1; }
        const uint64_t lo0 = kM0 * x[0], hi0 = __umul64hi(kM0, x[0]);
        const uint64_t lo1 = kM1 * x[2], hi1 = __umul64hi(kM1, x[2]);
        const uint64_t y0 = hi1 ^ x[1] ^ k0, y2 = hi0 ^ x[3] ^ k1;
        x[0] = y0; x[1] = lo1; x[2] = y2; x[3] = lo0;
    }
}

// The draw of one (key0, key1, counter) triple: the block's first word as a double
// in [0, 1) with 53 random bits.
FIE_DEV double philox_uniform(const uint64_t* t)
{
    uint64_t x[4] = {t[2], 0, 0, 0};
    philox4x64_10(x, t[0], t[1]);
    return (double)(x[0] >> 11) * 0x1p-53;
}

// floor(e * 2^40) of e in [0, 1].  e * 2^40 is exact in double, so the conversion
// only truncates.
FIE_DEV uint64_t fixed40(float e)
{
    return (uint64_t)((double)e * 1099511627776.0);
}

// Token weight relative to its tile maximum m: floor(cexp(y - m) * 2^40).
FIE_DEV uint64_t tok_weight(float y, float m) { return fixed40(cexp(y - m)); }

// ---------------------------------------------------------------- wide integers
FIE_DEV u128 mul64(uint64_t a, uint64_t b) { return (u128)a * b; }

// floor(m * X / 2^q) for m < 2^53, X < 2^128, exactly (a 192-bit product).
FIE_DEV u128 mul_shift(uint64_t m, u128 X, int q)
{
    u128 lo = (u128)m * (uint64_t)X;
    u128 hi = (u128)m * (uint64_t)(X >> 64);
    uint64_t p0 = (uint64_t)lo;
    u128 mid = (lo >> 64) + hi;
    uint64_t p1 = (uint64_t)mid;
    uint64_t p2 = (uint64_t)(mid >> 64);
    if (q >= 192) return 0;
    if (q >= 128) return (u128)(p2 >> (q - 128));
    if (q >= 64) {
        int s = q - 64;
        u128 v = ((u128)p2 << 64) | p1;
        return s ? (v >> s) : v;
    }
    u128 v = ((u128)p1 << 64) | p0;
    return q ? ((v >> q) | ((u128)p2 << (128 - q))) : v;
}

// Exact ceil(p * S) for an fp32 p in (0, 1) and S < 2^104.
FIE_DEV u128 ceil_mul_f32(float p, u128 S)
{
    uint32_t b = __float_as_uint(p);
    uint32_t eb = (b >> 23) & 0xFFu;
    uint64_t mant = (b & 0x7FFFFFu) | (eb ? 0x800000u : 0u);
    int q = eb ? 150 - (int)eb : 149;
    u128 P = (u128)mant * S;
    if (q >= 128) return P ? 1 : 0;
    return (P >> q) + (((P & ((((u128)1) << q) - 1)) != 0) ? 1 : 0);
}

// Exact floor(u * K) for a double u in [0, 1) and K < 2^104.
FIE_DEV u128 floor_mul_f64(double u, u128 K)
{
    if (!(u > 0.0)) return 0;
    uint64_t b = (uint64_t)__double_as_longlong(u);
    uint32_t eb = (uint32_t)((b >> 52) & 0x7FFu);
    uint64_t mant = (b & 0xFFFFFFFFFFFFFull) | (eb ? (1ull << 52) : 0ull);
    int q = eb ? 1075 - (int)eb : 1074;
    return mul_shift(mant, K, q);
}

FIE_DEV double u128_to_double(u128 x)
{
    return (double)(uint64_t)(x >> 64) * 18446744073709551616.0 + (double)(uint64_t)x;
}

// ---------------------------------------------------------------- wave64 helpers
FIE_DEV uint64_t shfl_xor_u64(uint64_t v, int m)
{
    uint32_t lo = __shfl_xor((uint32_t)v, m, 64);
    uint32_t hi = __shfl_xor((uint32_t)(v >> 32), m, 64);
    return ((uint64_t)hi << 32) | lo;
}

FIE_DEV uint64_t shfl_up_u64(uint64_t v, int d)
{
    uint32_t lo = __shfl_up((uint32_t)v, d, 64);
    uint32_t hi = __shfl_up((uint32_t)(v >> 32), d, 64);
    return ((uint64_t)hi << 32) | lo;
}

FIE_DEV uint64_t shfl_u64(uint64_t v, int src)
{
    uint32_t lo = __shfl((uint32_t)v, src, 64);
    uint32_t hi = __shfl((uint32_t)(v >> 32), src, 64);
    return ((uint64_t)hi << 32) | lo;
}

FIE_DEV u128 shfl_up_u128(u128 v, int d)
{
    uint64_t lo = shfl_up_u64((uint64_t)v, d), hi = shfl_up_u64((uint64_t)(v >> 64), d);
    return ((u128)hi << 64) | lo;
}

FIE_DEV u128 shfl_xor_u128(u128 v, int m)
{
    uint64_t lo = shfl_xor_u64((uint64_t)v, m), hi = shfl_xor_u64((uint64_t)(v >> 64), m);
    return ((u128)hi << 64) | lo;
}

FIE_DEV uint32_t wave_max_u32(uint32_t v)
{
    for (int m = 32; m > 0; m >>= 1) {
        uint32_t o = __shfl_xor(v, m, 64);
        v = o > v ? o : v;
    }
    return v;
}

FIE_DEV uint32_t wave_min_u32(uint32_t v)
{
    for (int m = 32; m > 0; m >>= 1) {
        uint32_t o = __shfl_xor(v, m, 64);
        v = o < v ? o : v;
    }
    return v;
}

FIE_DEV uint32_t wave_sum_u32(uint32_t v)
{
    for (int m = 32; m > 0; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

FIE_DEV uint64_t wave_max_u64(uint64_t v)
{
    for (int m = 32; m > 0; m >>= 1) {
        uint64_t o = shfl_xor_u64(v, m);
        v = o > v ? o : v;
    }
    return v;
}

FIE_DEV uint64_t wave_sum_u64(uint64_t v)
{
    for (int m = 32; m > 0; m >>= 1) v += shfl_xor_u64(v, m);
    return v;
}

FIE_DEV u128 wave_sum_u128(u128 v)
{
    for (int m = 32; m > 0; m >>= 1) v += shfl_xor_u128(v, m);
    return v;
}

// Inclusive prefix sum over the lanes of a wave (lane 0 first).
FIE_DEV uint32_t wave_incl_scan_u32(uint32_t v)
{
    const int lane = threadIdx.x & 63;
    for (int d = 1; d < 64; d <<= 1) {
        uint32_t o = __shfl_up(v, d, 64);
        if (lane >= d) v += o;
    }
    return v;
}

FIE_DEV u128 wave_incl_scan_u128(u128 v)
{
    const int lane = threadIdx.x & 63;
    for (int d = 1; d < 64; d <<= 1) {
        u128 o = shfl_up_u128(v, d);
        if (lane >= d) v += o;
    }
    return v;
}

// ---------------------------------------------------------------- DPP wave helpers
// Cross-lane steps by data-parallel primitives (no LDS round trip).  After the four
// steps inside a row of 16 lanes every lane of the row holds the row's result; the
// four row results are then combined from lanes 0, 16, 32, 48 in scalar registers.
template <int CTRL>
FIE_DEV uint32_t dpp_mov(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

FIE_DEV uint32_t rl(uint32_t v, int lane) { return (uint32_t)__builtin_amdgcn_readlane((int)v, lane); }

FIE_DEV uint32_t dwave_max_u32(uint32_t v)
{
    v = max(v, dpp_mov<kDppXor1>(v));
    v = max(v, dpp_mov<kDppXor2>(v));
    v = max(v, dpp_mov<kDppHalfMirror>(v));
    v = max(v, dpp_mov<kDppMirror>(v));
    return max(max(rl(v, 0), rl(v, 16)), max(rl(v, 32), rl(v, 48)));
}

FIE_DEV uint32_t dwave_min_u32(uint32_t v)
{
    v = min(v, dpp_mov<kDppXor1>(v));
    v = min(v, dpp_mov<kDppXor2>(v));
    v = min(v, dpp_mov<kDppHalfMirror>(v));
    v = min(v, dpp_mov<kDppMirror>(v));
    return min(min(rl(v, 0), rl(v, 16)), min(rl(v, 32), rl(v, 48)));
}

FIE_DEV uint64_t dwave_sum_u64(uint64_t v)
{
    auto step = [](uint64_t x, auto mv) {
        const uint32_t lo = mv((uint32_t)x), hi = mv((uint32_t)(x >> 32));
        return x + (((uint64_t)hi << 32) | lo);
    };
    v = step(v, [](uint32_t a) { return dpp_mov<kDppXor1>(a); });
    v = step(v, [](uint32_t a) { return dpp_mov<kDppXor2>(a); });
    v = step(v, [](uint32_t a) { return dpp_mov<kDppHalfMirror>(a); });
    v = step(v, [](uint32_t a) { return dpp_mov<kDppMirror>(a); });
    uint64_t t = 0;
#pragma unroll
    for (int r = 0; r < 4; ++r)
        t += ((uint64_t)rl((uint32_t)(v >> 32), 16 * r) << 32) | rl((uint32_t)v, 16 * r);
    return t;
}

// Exclusive prefix sum over the lanes of a wave (lane 0 first), and the total.
FIE_DEV uint32_t dwave_excl_scan_u32(uint32_t v, uint32_t* total)
{
    const int lane = threadIdx.x & 63;
    uint32_t x = v;
    // inclusive scan inside each row of 16: shifts by 1, 2, 4, 8 (0 shifted in)
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xF, 0xF, true);
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xF, 0xF, true);
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xF, 0xF, true);
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xF, 0xF, true);
    const uint32_t r0 = rl(x, 15), r1 = rl(x, 31), r2 = rl(x, 47), r3 = rl(x, 63);
    const int row = lane >> 4;
    const uint32_t before = (row > 0 ? r0 : 0u) + (row > 1 ? r1 : 0u) + (row > 2 ? r2 : 0u);
    *total = r0 + r1 + r2 + r3;
    return before + x - v;
}

FIE_DEV uint32_t popc64(uint64_t m) { return (uint32_t)__builtin_popcountll(m); }

// Orders this wave's earlier LDS writes before its later LDS reads (other lanes'
// writes included) without a workgroup barrier.
FIE_DEV void wave_lds_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// ---------------------------------------------------------------- block helpers
// All take a __shared__ scratch area of at least NT/64 entries of the value type
// and end with a barrier, so the scratch can be reused at once.
template <int NT>
FIE_DEV uint32_t block_max_u32(uint32_t v, uint32_t* scratch)
{
    v = wave_max_u32(v);
    if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
    __syncthreads();
    uint32_t t = 0;
    for (int w = 0; w < NT / 64; ++w) t = scratch[w] > t ? scratch[w] : t;
    __syncthreads();
    return t;
}

template <int NT>
FIE_DEV uint32_t block_min_u32(uint32_t v, uint32_t* scratch)
{
    v = wave_min_u32(v);
    if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
    __syncthreads();
    uint32_t t = 0xFFFFFFFFu;
    for (int w = 0; w < NT / 64; ++w) t = scratch[w] < t ? scratch[w] : t;
    __syncthreads();
    return t;
}

template <int NT>
FIE_DEV uint32_t block_sum_u32(uint32_t v, uint32_t* scratch)
{
    v = wave_sum_u32(v);
    if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
    __syncthreads();
    uint32_t t = 0;
    for (int w = 0; w < NT / 64; ++w) t += scratch[w];
    __syncthreads();
    return t;
}

template <int NT>
FIE_DEV uint64_t block_max_u64(uint64_t v, uint64_t* scratch)
{
    v = wave_max_u64(v);
    if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
    __syncthreads();
    uint64_t t = 0;
    for (int w = 0; w < NT / 64; ++w) t = scratch[w] > t ? scratch[w] : t;
    __syncthreads();
    return t;
}

template <int NT>
FIE_DEV uint64_t block_sum_u64(uint64_t v, uint64_t* scratch)
{
    v = wave_sum_u64(v);
    if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
    __syncthreads();
    uint64_t t = 0;
    for (int w = 0; w < NT / 64; ++w) t += scratch[w];
    __syncthreads();
    return t;
}

template <int NT>
FIE_DEV u128 block_sum_u128(u128 v, u128* scratch)
{
    v = wave_sum_u128(v);
    if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
    __syncthreads();
    u128 t = 0;
    for (int w = 0; w < NT / 64; ++w) t += scratch[w];
    __syncthreads();
    return t;
}

// Exclusive prefix sum in thread order; *total receives the block sum.
template <int NT>
FIE_DEV uint32_t block_excl_scan_u32(uint32_t v, uint32_t* scratch, uint32_t* total)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t incl = wave_incl_scan_u32(v);
    if (lane == 63) scratch[wave] = incl;
    __syncthreads();
    uint32_t before = 0, all = 0;
    for (int w = 0; w < NT / 64; ++w) {
        if (w < wave) before += scratch[w];
        all += scratch[w];
    }
    __syncthreads();
    *total = all;
    return before + incl - v;
}

}  // namespace fie
