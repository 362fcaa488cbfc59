// mm_common.h -- device helpers shared by the gfx950 selective-scan kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace mm {

// ---- element types -------------------------------------------------------------------------
struct bf16_t { uint16_t bits; };
struct f16_t { _Float16 v; };

template <typename T> struct ElemSize { static constexpr int value = sizeof(T); };

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16_t x) { return __uint_as_float(uint32_t(x.bits) << 16); }
__device__ __forceinline__ float to_f32(f16_t x) { return float(x.v); }

// float -> bf16 with round-to-nearest-even (NaN kept quiet), matching torch's .to(bfloat16).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return uint16_t(u >> 16);
}

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) { return bf16_t{f32_to_bf16_bits(x)}; }
template <> __device__ __forceinline__ f16_t from_f32<f16_t>(float x) { return f16_t{(_Float16)x}; }

// ---- math ------------------------------------------------------------------------------------
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// exp2(dt * A2 + kExpBiasOffset) for a decay argument dt * (A log2 e) <= 0, as one FMA and one
// v_exp_f32. Measured on gfx950 over 2^24 arguments, v_exp_f32 returns the correctly rounded 2^x
// for ~95 % of them and is 1 ulp low for most of the rest: for |x| < 1e-3 (decays just below 1,
// the states with the longest memory) its mean relative error is -7e-9 per call, -3.4e-9 for
// |x| > 0.2. A recurrence multiplies that bias over its memory: in the coupled P/Q scan, 8,192
// float32 steps drift 3.1e-4 from float64 where a correctly rounded exp2 drifts 2.4e-5 (a float32
// emulation of the kernel's operation order). The offset 1e-8 (2^1e-8 = 1 + 6.9e-9) removes the
// mean bias of the long-memory decays (the same emulation: 2.0e-5); for |x| >= 0.25 it is below
// half an ulp of x and vanishes, and exp2(1e-8) is 1 (a zero step stays the identity).
constexpr float kExpBiasOffset = 1.0e-8f;
__device__ __forceinline__ float decay_exp2(float dt, float A2) {
    return __builtin_amdgcn_exp2f(__builtin_fmaf(dt, A2, kExpBiasOffset));
}

// softplus with torch's threshold: x > 20 ? x : log1p(exp(x)).
__device__ __forceinline__ float softplus_f32(float x) {
    return x > 20.f ? x : log1pf(expf(x));
}

// silu(z) = z / (1 + exp(-z)), in float32.
__device__ __forceinline__ float silu_f32(float z) { return z / (1.f + expf(-z)); }

// softplus with torch's threshold semantics (x > 20 ? x : log1p(exp(x))) built on v_exp_f32 /
// v_log_f32, evaluated as max(x, 0) + log1p(e) with e = exp(-|x|): the same function, no overflow,
// and equal to x in float32 for x > 20 (there e < 2.1e-9 is below half an ulp of x). With e <= 1,
// u = fl(1 + e) lies in [1, 2] and log1p(e) = log(u) + lost / u + O(lost^2), where lost = e - (u - 1)
// is exact (Fast2Sum). lost is added without the 1/u: |lost| <= 2^-24 and lost (1 - 1/u) stays
// below 2^-24 e, so the relative error is a few ulp for every x, including x << 0 where
// softplus(x) ~ e.
__device__ __forceinline__ float softplus_fast(float x) {
    const float e = __builtin_amdgcn_exp2f(-__builtin_fabsf(x) * kLog2e);
    const float u = 1.f + e;
    const float lost = e - (u - 1.f);
    return __builtin_fmaxf(x, 0.f) + __builtin_fmaf(__builtin_amdgcn_logf(u), kLn2, lost);
}

// silu(z) = z * 1 / (1 + 2^(-z log2 e)) with v_exp_f32 and v_rcp_f32 (both ~1 ulp).
__device__ __forceinline__ float silu_fast(float z) {
    return z * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-z * kLog2e));
}

// ---- vector I/O of 8 consecutive elements (16 B for 16-bit types, 32 B for float) -----------
template <typename T> struct Vec8;
template <> struct Vec8<float> { uint4 lo, hi; };
template <> struct Vec8<bf16_t> { uint4 v; };
template <> struct Vec8<f16_t> { uint4 v; };

__device__ __forceinline__ void unpack8(const Vec8<float> &v, float *o) {
    o[0] = __uint_as_float(v.lo.x); o[1] = __uint_as_float(v.lo.y);
    o[2] = __uint_as_float(v.lo.z); o[3] = __uint_as_float(v.lo.w);
    o[4] = __uint_as_float(v.hi.x); o[5] = __uint_as_float(v.hi.y);
    o[6] = __uint_as_float(v.hi.z); o[7] = __uint_as_float(v.hi.w);
}
__device__ __forceinline__ void unpack_bf16x2(uint32_t w, float &a, float &b) {
    a = __uint_as_float(w << 16);
    b = __uint_as_float(w & 0xffff0000u);
}
__device__ __forceinline__ void unpack8(const Vec8<bf16_t> &v, float *o) {
    unpack_bf16x2(v.v.x, o[0], o[1]); unpack_bf16x2(v.v.y, o[2], o[3]);
    unpack_bf16x2(v.v.z, o[4], o[5]); unpack_bf16x2(v.v.w, o[6], o[7]);
}
__device__ __forceinline__ void unpack_f16x2(uint32_t w, float &a, float &b) {
    union { uint32_t u; _Float16 h[2]; } c; c.u = w;
    a = float(c.h[0]); b = float(c.h[1]);
}
__device__ __forceinline__ void unpack8(const Vec8<f16_t> &v, float *o) {
    unpack_f16x2(v.v.x, o[0], o[1]); unpack_f16x2(v.v.y, o[2], o[3]);
    unpack_f16x2(v.v.z, o[4], o[5]); unpack_f16x2(v.v.w, o[6], o[7]);
}

__device__ __forceinline__ Vec8<float> pack8_f32(const float *x) {
    Vec8<float> v;
    v.lo = make_uint4(__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]), __float_as_uint(x[3]));
    v.hi = make_uint4(__float_as_uint(x[4]), __float_as_uint(x[5]), __float_as_uint(x[6]), __float_as_uint(x[7]));
    return v;
}
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
// Two floats -> packed bf16 pair, round-to-nearest-even (one v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    const f32x2_t v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
    union { uint32_t u; _Float16 h[2]; } c; c.h[0] = (_Float16)a; c.h[1] = (_Float16)b;
    return c.u;
}

template <typename T> __device__ __forceinline__ Vec8<T> pack8(const float *x);
template <> __device__ __forceinline__ Vec8<float> pack8<float>(const float *x) { return pack8_f32(x); }
template <> __device__ __forceinline__ Vec8<bf16_t> pack8<bf16_t>(const float *x) {
    Vec8<bf16_t> v;
    v.v = make_uint4(pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3]), pack_bf16x2(x[4], x[5]), pack_bf16x2(x[6], x[7]));
    return v;
}
template <> __device__ __forceinline__ Vec8<f16_t> pack8<f16_t>(const float *x) {
    Vec8<f16_t> v;
    v.v = make_uint4(pack_f16x2(x[0], x[1]), pack_f16x2(x[2], x[3]), pack_f16x2(x[4], x[5]), pack_f16x2(x[6], x[7]));
    return v;
}

template <typename T> __device__ __forceinline__ void load8(const T *p, float *o) {
    unpack8(*reinterpret_cast<const Vec8<T> *>(p), o);
}
template <typename T> __device__ __forceinline__ void store8(T *p, const float *x) {
    *reinterpret_cast<Vec8<T> *>(p) = pack8<T>(x);
}

// ---- vectors of N consecutive elements of T, as raw words --------------------------------
// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E).
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// N consecutive elements moved as one vector (N * sizeof(T) bytes: 4, 8, 16 or 32).
template <typename T, int N> struct RawVec { uint32_t w[(N * sizeof(T) + 3) / 4]; };

template <typename T, int N>
__device__ __forceinline__ RawVec<T, N> load_raw(const T *p) {
    RawVec<T, N> r;
    constexpr int W = sizeof(r.w) / 4;
    if constexpr (W == 8) {
        const uint4 *q = reinterpret_cast<const uint4 *>(p);
        const uint4 a = q[0], b = q[1];
        r.w[0] = a.x; r.w[1] = a.y; r.w[2] = a.z; r.w[3] = a.w; r.w[4] = b.x; r.w[5] = b.y; r.w[6] = b.z; r.w[7] = b.w;
    } else if constexpr (W == 4) {
        const uint4 a = *reinterpret_cast<const uint4 *>(p);
        r.w[0] = a.x; r.w[1] = a.y; r.w[2] = a.z; r.w[3] = a.w;
    } else if constexpr (W == 2) {
        const uint2 a = *reinterpret_cast<const uint2 *>(p);
        r.w[0] = a.x; r.w[1] = a.y;
    } else {
        r.w[0] = *reinterpret_cast<const uint32_t *>(p);
    }
    return r;
}

template <typename T, int N>
__device__ __forceinline__ void unpack_raw(const RawVec<T, N> &r, float *o) {
    if constexpr (std::is_same_v<T, float>) {
#pragma unroll
        for (int i = 0; i < N; ++i) o[i] = __uint_as_float(r.w[i]);
    } else if constexpr (std::is_same_v<T, bf16_t>) {
#pragma unroll
        for (int i = 0; i < N / 2; ++i) unpack_bf16x2(r.w[i], o[2 * i], o[2 * i + 1]);
    } else {
#pragma unroll
        for (int i = 0; i < N / 2; ++i) unpack_f16x2(r.w[i], o[2 * i], o[2 * i + 1]);
    }
}

template <typename T, int N>
__device__ __forceinline__ void store_vec(T *p, const float *x) {
    if constexpr (std::is_same_v<T, float>) {
        if constexpr (N == 8) {
            uint4 *q = reinterpret_cast<uint4 *>(p);
            q[0] = make_uint4(__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]), __float_as_uint(x[3]));
            q[1] = make_uint4(__float_as_uint(x[4]), __float_as_uint(x[5]), __float_as_uint(x[6]), __float_as_uint(x[7]));
        } else if constexpr (N == 4) {
            *reinterpret_cast<uint4 *>(p) = make_uint4(__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]), __float_as_uint(x[3]));
        } else {
            *reinterpret_cast<uint2 *>(p) = make_uint2(__float_as_uint(x[0]), __float_as_uint(x[1]));
        }
    } else {
        uint32_t w[N / 2];
#pragma unroll
        for (int i = 0; i < N / 2; ++i)
            w[i] = std::is_same_v<T, bf16_t> ? pack_bf16x2(x[2 * i], x[2 * i + 1]) : pack_f16x2(x[2 * i], x[2 * i + 1]);
        if constexpr (N == 8) *reinterpret_cast<uint4 *>(p) = make_uint4(w[0], w[1], w[2], w[3]);
        else if constexpr (N == 4) *reinterpret_cast<uint2 *>(p) = make_uint2(w[0], w[1]);
        else *reinterpret_cast<uint32_t *>(p) = w[0];
    }
}

// ---- buffer instructions -----------------------------------------------------------------------
// Raw buffer resource over [base, base + 4 GiB): the address of an access is base + the lane's
// VGPR byte offset + a scalar byte offset, range-checked against 2^32 - 1 bytes (gfx9 resource
// word 3). A kernel that addresses a row group this way keeps one scalar base per tensor and a
// 32-bit offset per lane instead of a 64-bit pointer per lane and tensor.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, -1, 0x00020000);
}

// N consecutive elements of T (4, 8 or 16 bytes) through a buffer resource.
template <typename T, int N>
__device__ __forceinline__ RawVec<T, N> buffer_load_raw(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    RawVec<T, N> x;
    constexpr int W = sizeof(x.w) / 4;
    if constexpr (W == 1) {
        x.w[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
    } else if constexpr (W == 2) {
        typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
        x.w[0] = v.x;
        x.w[1] = v.y;
    } else {
        static_assert(W == 4, "buffer_load_raw moves 4, 8 or 16 bytes");
        typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
        const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
        x.w[0] = v.x;
        x.w[1] = v.y;
        x.w[2] = v.z;
        x.w[3] = v.w;
    }
    return x;
}

// N consecutive elements of T of any 4-byte-multiple size, as 16-byte buffer loads and a last,
// shorter one.
template <typename T, int N>
__device__ __forceinline__ RawVec<T, N> buffer_load_rawn(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    constexpr int W = sizeof(RawVec<T, N>) / 4;
    if constexpr (W <= 4) {
        return buffer_load_raw<T, N>(r, voff, soff);
    } else {
        static_assert(W % 4 == 0, "buffer_load_rawn splits into 16-byte pieces");
        constexpr int NP = 16 / int(sizeof(T));   // elements per piece
        RawVec<T, N> x;
#pragma unroll
        for (int i = 0; i < W / 4; ++i) {
            const RawVec<T, NP> v = buffer_load_raw<T, NP>(r, voff + 16 * i, soff);
#pragma unroll
            for (int k = 0; k < 4; ++k) x.w[4 * i + k] = v.w[k];
        }
        return x;
    }
}

// N floats converted to T (bf16 round-to-nearest-even) and stored as one 4-, 8- or 16-byte access.
template <typename T, int N>
__device__ __forceinline__ void buffer_store_vec(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, const float *x) {
    constexpr int W = (N * int(sizeof(T)) + 3) / 4;
    uint32_t w[W];
    if constexpr (std::is_same_v<T, float>) {
#pragma unroll
        for (int i = 0; i < N; ++i) w[i] = __float_as_uint(x[i]);
    } else {
#pragma unroll
        for (int i = 0; i < N / 2; ++i)
            w[i] = std::is_same_v<T, bf16_t> ? pack_bf16x2(x[2 * i], x[2 * i + 1]) : pack_f16x2(x[2 * i], x[2 * i + 1]);
    }
    if constexpr (W == 1) {
        __builtin_amdgcn_raw_buffer_store_b32(w[0], r, voff, soff, 0);
    } else if constexpr (W == 2) {
        typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{w[0], w[1]}, r, voff, soff, 0);
    } else {
        static_assert(W == 4, "buffer_store_vec moves 4, 8 or 16 bytes");
        typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{w[0], w[1], w[2], w[3]}, r, voff, soff, 0);
    }
}

// N floats stored as T through a buffer resource, in 16-byte pieces when they take more than 16.
template <typename T, int N>
__device__ __forceinline__ void buffer_store_vecn(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, const float *x) {
    if constexpr (N * int(sizeof(T)) <= 16) {
        buffer_store_vec<T, N>(r, voff, soff, x);
    } else {
        constexpr int H = 16 / int(sizeof(T));
        static_assert(N % H == 0, "buffer_store_vecn splits into 16-byte pieces");
#pragma unroll
        for (int i = 0; i < N / H; ++i) buffer_store_vec<T, H>(r, voff + 16 * i, soff, x + H * i);
    }
}

// ---- Sums over the LPR consecutive lanes of a group (a channel's lanes) with DPP ----

// x + x[lane permuted by CTRL] as one v_add_f32 with a DPP operand (the compiler inserts the DPP
// read hazard wait states itself for the builtin).
template <int CTRL>
__device__ __forceinline__ float dpp_add(float x) {
    const int o = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false);
    return x + __builtin_bit_cast(float, o);
}

// x of the lane CTRL pairs this lane with.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}

// Sum over the LPR consecutive lanes of a group. Every step pairs two partial sums and adds them
// in both lanes (a + b == b + a exactly), so all LPR lanes hold bit-identical totals.
template <int LPR>
__device__ __forceinline__ float group_sum(float x) {
    static_assert(LPR == 4 || LPR == 8 || LPR == 16, "LPR");
    x = dpp_add<0xB1>(x);                           // quad_perm [1,0,3,2]
    x = dpp_add<0x4E>(x);                           // quad_perm [2,3,0,1]
    if constexpr (LPR >= 8) x = dpp_add<0x141>(x);  // row_half_mirror: the other quad of 8 lanes
    if constexpr (LPR >= 16) x = dpp_add<0x140>(x); // row_mirror: the other half of the 16-lane row
    return x;
}

// R sums over the LPR lanes of a group at once (R a power of 2, 2 <= R <= LPR), the DPP stages of
// group_sum run as a transposed reduction. The stages pair lanes by kLaneStage<LPR, 0>, <1>, ...
// (row_mirror, row_half_mirror, quad_perm [2,3,0,1], [1,0,3,2] at 16 lanes; the last three at 8;
// quad_perm [3,2,1,0], [1,0,3,2] at 4), outermost first. Lane k of the group holds its partials in
// the order x[t] = partial of sum t ^ c_k, c_k = lane_rank_offset<LPR, R>(k): then at stage j < log2 R
// each lane adds the upper half of its partner's live values to the lower half of its own (the
// partner's upper half holds the sums this lane keeps), halving the live values with one DPP add
// each; the remaining stages add the single live value symmetrically; and the other totals come back
// by the transposed stages' patterns in reverse (x[t + 2^i] = x[t] of the stage-(log2 R - 1 - i)
// partner). On return x[t] is the total of sum t ^ c_k, the same bits in every lane that holds that
// sum. R - 1 + log2(LPR / R) DPP adds and R - 1 DPP moves (which the compiler folds into a
// consuming multiply where it can), against R log2(LPR) adds for R separate butterflies. The lane
// orders were derived and checked by simulating the stages on symbolic partials.
template <int LPR, int J>
constexpr int kLaneStage = LPR == 16 ? (J == 0 ? 0x140 : J == 1 ? 0x141 : J == 2 ? 0x4E : 0xB1)
                         : LPR == 8  ? (J == 0 ? 0x141 : J == 1 ? 0x4E : 0xB1)
                                     : (J == 0 ? 0x1B : 0xB1);

template <int LPR, int R>
__device__ __forceinline__ int lane_rank_offset(int k) {
    static_assert((LPR == 4 || LPR == 8 || LPR == 16) && (R == 2 || R == 4 || R == 8) && R <= LPR, "shape");
    // c_k of lane k in bits 4k .. 4k + 3.
    constexpr uint64_t tab = LPR == 4  ? (R == 2 ? 0x1100ull : 0x2310ull)
                           : LPR == 8  ? (R == 2 ? 0x11110000ull : R == 4 ? 0x22331100ull : 0x45673210ull)
                                       : (R == 2 ? 0x1111111100000000ull : R == 4 ? 0x2222333311110000ull
                                                                                  : 0x4455776622331100ull);
    return int((tab >> (4 * k)) & 15u);
}

template <int LPR, int R>
__device__ __forceinline__ void lane_sums(float (&x)[R]) {
    constexpr int M = R == 2 ? 1 : R == 4 ? 2 : 3;               // transposed stages
    constexpr int NS = LPR == 4 ? 2 : LPR == 8 ? 3 : 4;          // all stages
    static_for<0, M>([&](auto Jc) {
        constexpr int j = decltype(Jc)::value, n = R >> j;
#pragma unroll
        for (int t = 0; t < n / 2; ++t) x[t] = x[t] + dpp_mov<kLaneStage<LPR, j>>(x[n / 2 + t]);
    });
    static_for<M, NS>([&](auto Jc) { x[0] = dpp_add<kLaneStage<LPR, decltype(Jc)::value>>(x[0]); });
    static_for<0, M>([&](auto Ic) {
        constexpr int i = decltype(Ic)::value, j = M - 1 - i, h = 1 << i;
#pragma unroll
        for (int t = 0; t < h; ++t) x[t + h] = dpp_mov<kLaneStage<LPR, j>>(x[t]);
    });
}

}  // namespace mm
