// Shared device/host helpers of the CRESSO5 gfx950 library.
//
// Conventions used by every kernel in this library:
//  * wave64 (gfx950); block sizes are multiples of 64;
//  * reductions are deterministic: per-thread fp32 partials, wave butterflies
//    in a fixed lane order, then a fixed-order merge over waves/blocks in fp64;
//    histogram-style scatter uses 64-bit fixed-point integer atomics (integer
//    addition is associative, so the result does not depend on arrival order);
//  * per-element transcendental math uses the hardware approximations
//    (v_exp_f32 / v_log_f32 / v_rcp_f32 / v_sqrt_f32); per-tensor scalars use
//    the accurate libm versions in the state dtype.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/cresso_hip.h"

namespace cresso {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// dtype traits
// ---------------------------------------------------------------------------
template <typename T> struct dt;
template <> struct dt<float> { static constexpr int code = CRESSO_F32; };
template <> struct dt<double> { static constexpr int code = CRESSO_F64; };
template <> struct dt<__half> { static constexpr int code = CRESSO_F16; };
template <> struct dt<__hip_bfloat16> { static constexpr int code = CRESSO_BF16; };

__device__ __forceinline__ float to_f(float v) { return v; }
__device__ __forceinline__ float to_f(double v) { return (float)v; }
__device__ __forceinline__ float to_f(__half v) { return __half2float(v); }
__device__ __forceinline__ float to_f(__hip_bfloat16 v) { return __bfloat162float(v); }

template <typename W, typename T> __device__ __forceinline__ W to_w(T v) { return (W)to_f(v); }
template <> __device__ __forceinline__ double to_w<double, double>(double v) { return v; }

// Round a work-dtype value to the storage dtype (round to nearest even).
template <typename T> __device__ __forceinline__ T from_w(float v);
template <> __device__ __forceinline__ float from_w<float>(float v) { return v; }
template <> __device__ __forceinline__ double from_w<double>(float v) { return (double)v; }
template <> __device__ __forceinline__ __half from_w<__half>(float v) { return __float2half_rn(v); }
template <> __device__ __forceinline__ __hip_bfloat16 from_w<__hip_bfloat16>(float v) { return __float2bfloat16(v); }
template <typename T> __device__ __forceinline__ T from_wd(double v) { return from_w<T>((float)v); }
template <> __device__ __forceinline__ double from_wd<double>(double v) { return v; }

// The step of the parameter update p.add_(u, alpha=-lr) (cresso_v5.py:1353,
// 1582, 1432) for a param of storage dtype T: torch's CPU add kernel rounds
// alpha to the tensor's dtype for fp16/bf16 tensors (then computes in fp32),
// so the reference's update uses -lr rounded to the param dtype there; fp32
// and fp64 params keep it.
template <typename T> __device__ __forceinline__ double update_alpha(double a) { return a; }
template <> __device__ __forceinline__ double update_alpha<__half>(double a) {
    return (double)__half2float(__float2half_rn((float)a));
}
template <> __device__ __forceinline__ double update_alpha<__hip_bfloat16>(double a) {
    return (double)__bfloat162float(__float2bfloat16((float)a));
}

// ---------------------------------------------------------------------------
// global-memory views of caller pointers: the address-space cast lets the
// compiler emit global_load / global_store (no flat aperture handling, no LDS
// counter waits) for pointers that arrive through generic pointer tables
// ---------------------------------------------------------------------------
#define CRESSO_GLOBAL __attribute__((address_space(1)))
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ f32x4 gload4(const float* p) { return *(const CRESSO_GLOBAL f32x4*)p; }
__device__ __forceinline__ void gstore4(float* p, f32x4 v) { *(CRESSO_GLOBAL f32x4*)p = v; }
__device__ __forceinline__ u32x2 gload2u(const void* p) { return *(const CRESSO_GLOBAL u32x2*)p; }
__device__ __forceinline__ void gstore2u(void* p, u32x2 v) { *(CRESSO_GLOBAL u32x2*)p = v; }

// Buffer view of one array: a resource descriptor (base, size in bytes) in
// SGPRs, addressed by a per-lane byte offset (one VGPR shared by every access
// of a pass) plus a uniform byte offset in an SGPR, so a thread's strided
// accesses need no address registers of their own.  Accesses at or beyond
// `bytes` read 0 and store nothing.  Word 3 is the gfx9-family raw-buffer
// format (32-bit data).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ f32x4 bload4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
// Stores take the whole offset in the VGPR and a literal 0 soffset: after a
// store of more than 8 bytes whose soffset is an SGPR, the compiler does not
// wait before the next VALU overwrites the store's data registers, and on
// gfx950 the last lanes of each 16-lane pass then store the new values.
__device__ __forceinline__ void bstore4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, f32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, voff + soff, 0, 0);
}
__device__ __forceinline__ float bload1(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
__device__ __forceinline__ uint32_t bload1u16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
}
__device__ __forceinline__ void bstore1(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, voff + soff, 0, 0);
}
__device__ __forceinline__ u32x2 bload2u(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
}
__device__ __forceinline__ void bstore2u(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, u32x2 v) {
    __builtin_amdgcn_raw_buffer_store_b64(v, r, voff + soff, 0, 0);
}

// ---------------------------------------------------------------------------
// Program-order pins.  sched_barrier only orders the machine scheduler; IR
// passes still hoist cheap per-element math of many elements ahead of the
// transcendental chains, or sink accumulations to the end of a loop with
// every element's inputs kept alive, and the kernel spills.  An empty asm that
// reads and writes a value fixes the point where it is materialized:
//  * pin4 on a slot's inputs: nothing that depends on them moves above it;
//  * pin1 on an accumulator at the end of a slot or row: its contributions
//    are complete there.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void pin4(float* v) {
    asm volatile("" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]));
}
__device__ __forceinline__ void pin1(float& v) { asm volatile("" : "+v"(v)); }

// ---------------------------------------------------------------------------
// fast per-element math (hardware approximations, ~1 ulp on their domain)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float flog2(float x) { return __builtin_amdgcn_logf(x); }
__device__ __forceinline__ float frcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float fsqrt(float x) { return __builtin_amdgcn_sqrtf(x); }
__device__ __forceinline__ float fexp(float x) { return fexp2(x * 1.4426950408889634f); }
__device__ __forceinline__ float flog(float x) { return flog2(x) * 0.6931471805599453f; }
// x^y for x > 0
__device__ __forceinline__ float fpow(float x, float y) { return fexp2(y * flog2(x)); }
// log(1 + x) for x >= 0 (absolute error ~1e-7; only ever averaged)
__device__ __forceinline__ float flog1p(float x) { return flog2(1.0f + x) * 0.6931471805599453f; }
// tanh with absolute error ~1e-7
__device__ __forceinline__ float ftanh(float x) {
    float e = fexp2(-2.8853900817779268f * fabsf(x));   // exp(-2|x|)
    float r = (1.0f - e) * frcp(1.0f + e);
    return copysignf(r, x);
}
__device__ __forceinline__ float fsign(float x) { return x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : 0.0f); }
__device__ __forceinline__ float clampf(float x, float lo, float hi) { return fminf(fmaxf(x, lo), hi); }
// clamp to [lo, hi] (lo <= hi) in one instruction: the median of three
__device__ __forceinline__ float med3f(float x, float lo, float hi) { return __builtin_amdgcn_fmed3f(x, lo, hi); }
// |m| with the sign of s (one bitfield insert)
__device__ __forceinline__ float with_sign(float m, float s) { return copysignf(m, s); }
// m times the sign of s (+-1; m unchanged for s = +0): flips the sign bit
__device__ __forceinline__ float xorsign(float m, float s) {
    return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, m) ^ (__builtin_bit_cast(uint32_t, s) & 0x80000000u));
}
// tanh(c x) given k2 = -2 log2(e) c (c > 0): exp(-2c|x|) by one exp2
__device__ __forceinline__ float ftanh_k(float x, float k2) {
    const float ex = fexp2(k2 * fabsf(x));
    const float r = frcp(1.0f + ex);
    return copysignf(fmaf(-ex, r, r), x);
}

// Unsigned parts of the drive shaping of t (cresso_v5.py:1321-1324, scalar
// route 1563-1566) from at = |t|:
//   rat  = t/(1+|t|/clip)           -> |rat|  = at/(1+at/clip)
//   tanh(t/clip)                    -> |tanh| = (1-e)/(1+e), e = exp(-2 at/clip)
//   root = sign(t) sqrt(min(|t|,clip^2)+eps) -> |root| (0 when t == 0)
// All three carry the sign of t, so every product of two of them, or of one
// with t, equals the product of their magnitudes.  k2 = -2 log2(e) / clip.
struct Shape3A {
    float rat, th, root;
};
__device__ __forceinline__ Shape3A shape3a(float at, float k2, float iclip, float clip2, float eps) {
    Shape3A s;
    const float ex = fexp2(k2 * at);
    const float d1 = 1.0f + ex;
    const float d2 = fmaf(at, iclip, 1.0f);
    const float inv = frcp(d1 * d2);
    const float u = d2 * inv;   // 1/d1
    s.th = fmaf(-ex, u, u);     // (1-e)/(1+e)
    s.rat = at * (d1 * inv);    // at/d2
    const float r = fsqrt(fminf(at, clip2) + eps);
    s.root = at > 0.0f ? r : 0.0f;
    return s;
}

// shape3a of at together with the unsigned novelty tanh(|e| k) (k2n = -2 k
// log2 e), the two quotients from one reciprocal:
// 1/(d1 d2) = dn rr, 1/dn = d1 d2 rr with rr = 1/(d1 d2 dn).  Returns tanh(e k).
__device__ __forceinline__ float shape3a_nov(float at, float e, float k2, float k2n, float iclip, float clip2,
                                             float eps, Shape3A& s) {
    const float es = fexp2(k2 * at);
    const float d1 = 1.0f + es;
    const float d2 = fmaf(at, iclip, 1.0f);
    const float ex = fexp2(k2n * fabsf(e));
    const float dn = 1.0f + ex;
    const float d12 = d1 * d2;
    const float rr = frcp(d12 * dn);
    const float inv = dn * rr;   // 1/(d1 d2)
    const float ri = d12 * rr;   // 1/dn
    const float u = d2 * inv;    // 1/d1
    s.th = fmaf(-es, u, u);
    s.rat = at * (d1 * inv);
    const float r = fsqrt(fminf(at, clip2) + eps);
    s.root = at > 0.0f ? r : 0.0f;
    return copysignf(fmaf(-ex, ri, ri), e);
}

// double versions for the f64 work dtype (accurate libm)
__device__ __forceinline__ double fexp(double x) { return exp(x); }
__device__ __forceinline__ double flog(double x) { return log(x); }
__device__ __forceinline__ double fpow(double x, double y) { return pow(x, y); }
__device__ __forceinline__ double flog1p(double x) { return log1p(x); }
__device__ __forceinline__ double ftanh(double x) { return tanh(x); }
__device__ __forceinline__ double frcp(double x) { return 1.0 / x; }
__device__ __forceinline__ double fsqrt(double x) { return sqrt(x); }
__device__ __forceinline__ double fsign(double x) { return x > 0.0 ? 1.0 : (x < 0.0 ? -1.0 : 0.0); }
__device__ __forceinline__ double clampf(double x, double lo, double hi) { return fmin(fmax(x, lo), hi); }

// ---------------------------------------------------------------------------
// wave / block reductions (deterministic)
// ---------------------------------------------------------------------------
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
    return v;
}

// Wave total of a double by DPP row operations (VALU only, no LDS round
// trips); the total lands in lane 63, other lanes hold partial sums.  Each
// step moves both 32-bit halves with the same DPP control; lanes without a
// source receive +0.0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ double dpp_add_d(double v) {
    const int lo = __builtin_amdgcn_update_dpp(0, __double2loint(v), CTRL, ROW_MASK, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, __double2hiint(v), CTRL, ROW_MASK, 0xF, false);
    return v + __hiloint2double(hi, lo);
}
__device__ __forceinline__ double wave_total_d(double v) {
    v = dpp_add_d<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
    v = dpp_add_d<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
    v = dpp_add_d<0x124, 0xF>(v);  // row_ror:4
    v = dpp_add_d<0x128, 0xF>(v);  // row_ror:8
    v = dpp_add_d<0x142, 0xA>(v);  // row_bcast:15 -> rows 1, 3
    v = dpp_add_d<0x143, 0xC>(v);  // row_bcast:31 -> rows 2, 3
    return v;
}

// Issue priority that falls as a wave works through its share: q = the
// quarter of the work reached (0..3).  Several blocks share each CU's SIMDs
// and the arbiter favours the oldest wave, so in a launch of one round the
// blocks of a CU otherwise finish one after another, and the last ones run
// alone at a fraction of the occupancy; with the priority, waves that are
// behind win the arbitration and the blocks finish together.
__device__ __forceinline__ void progress_prio(int q) {
    if (q <= 0)
        __builtin_amdgcn_s_setprio(3);
    else if (q == 1)
        __builtin_amdgcn_s_setprio(2);
    else if (q == 2)
        __builtin_amdgcn_s_setprio(1);
    else
        __builtin_amdgcn_s_setprio(0);
}

// Wave sum of a float in a fixed lane order with DPP (quad xor 1, 2; row
// rotate 4, 8; row broadcasts 15, 31): the total lands in lane 63.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK,
                                                                        0xF, false));
}
__device__ __forceinline__ float wave_total(float v) {
    v = dpp_add<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
    v = dpp_add<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
    v = dpp_add<0x124, 0xF>(v);  // row_ror:4
    v = dpp_add<0x128, 0xF>(v);  // row_ror:8
    v = dpp_add<0x142, 0xA>(v);  // row_bcast:15 -> rows 1, 3
    v = dpp_add<0x143, 0xC>(v);  // row_bcast:31 -> rows 2, 3
    return v;                    // lane 63 holds the sum
}

// Sum V floats over the block; every thread receives the totals (fp64).  Each
// wave sums a value in fp32 with DPP (full-rate adds; a wave holds 64 lanes'
// partials, so fp32 loses nothing the lanes' own fp32 sums kept), threads
// v < V add the wave totals in wave order in fp64 and publish the block total
// once, and every thread reads the V published totals.
//   lds: (blockDim.x / 64) * V doubles;  pub: V doubles, not inside lds.
// Two barriers; the next call may reuse both areas at once.
template <int V>
__device__ __forceinline__ void block_sum_f(const float (&x)[V], double (&out)[V], double* lds, double* pub) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int nw = blockDim.x / kWave;
    float w[V];
#pragma unroll
    for (int i = 0; i < V; ++i) w[i] = wave_total(x[i]);
    if (lane == kWave - 1) {
#pragma unroll
        for (int i = 0; i < V; ++i) lds[wave * V + i] = (double)w[i];
    }
    __syncthreads();
    if (threadIdx.x < V) {
        double s = 0.0;
        for (int k = 0; k < nw; ++k) s += lds[k * V + threadIdx.x];
        pub[threadIdx.x] = s;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < V; ++i) out[i] = pub[i];
}

// Sum V values over the block; every thread receives the totals.
// lds must hold (blockDim.x/64) * V doubles.  Two barriers.
template <int V>
__device__ __forceinline__ void block_sum(double (&v)[V], double* lds) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int nw = blockDim.x / kWave;
#pragma unroll
    for (int i = 0; i < V; ++i) v[i] = wave_total_d(v[i]);
    if (lane == kWave - 1) {
#pragma unroll
        for (int i = 0; i < V; ++i) lds[wave * V + i] = v[i];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < V; ++i) {
        double s = 0.0;
        for (int w = 0; w < nw; ++w) s += lds[w * V + i];
        v[i] = s;
    }
    __syncthreads();
}

// Float (already scaled by a power of two, |x| < 2^62) to a 64-bit fixed-point
// integer, rounded to nearest even (unbiased: a bin collects up to ~10^6
// elements, so a one-sided rounding such as truncation would add a coherent
// half quantum per element): rint, then two exact 32-bit conversions.
__device__ __forceinline__ unsigned long long to_fixed_u(float x) {
    x = rintf(x);
    const float hf = floorf(x * 2.3283064365386963e-10f);  // x / 2^32 (exact scaling)
    const float lf = fmaf(-hf, 4294967296.0f, x);           // x - hi*2^32: exact, in [0, 2^32)
    return ((unsigned long long)(unsigned)hf << 32) | (unsigned long long)(unsigned)lf;
}
// two's complement of the magnitude's conversion (rounding is symmetric)
__device__ __forceinline__ unsigned long long to_fixed_s(float x) {
    const unsigned long long u = to_fixed_u(fabsf(x));
    return x < 0.f ? (0ull - u) : u;
}

// ---------------------------------------------------------------------------
// Coordinate hash (cresso_v5.py:495-516): int64 wrap, arithmetic shifts,
// floor-mod.  `i` is the row-major linear index.
// ---------------------------------------------------------------------------
struct HashSalt {
    uint64_t a, b, c, d;   // multiplier, offset, 2nd and 3rd multipliers
};

__host__ __device__ inline HashSalt hash_salt(int64_t salt) {
    uint64_t s = (uint64_t)(salt + 1);
    HashSalt h;
    h.a = 1103515245ULL + 97ULL * s;
    h.b = 12345ULL + 0x9E3779B1ULL * s;
    h.c = 2246822519ULL + 1315423911ULL * s;
    h.d = 3266489917ULL + 374761393ULL * s;
    return h;
}

__device__ __forceinline__ uint64_t ashr64(uint64_t x, int k) { return (uint64_t)((int64_t)x >> k); }

__device__ __forceinline__ int64_t hash_raw(uint64_t i, const HashSalt& s) {
    uint64_t h = i * s.a + s.b;
    h ^= ashr64(h, 16);
    h *= s.c;
    h ^= ashr64(h, 13);
    h *= s.d;
    h ^= ashr64(h, 16);
    return (int64_t)h;
}

// bins > 0; mask = bins-1 when bins is a power of two (floor-mod == low bits
// in two's complement), else -1 and a signed floor-mod is used.
__device__ __forceinline__ int hash_bin(uint64_t i, const HashSalt& s, int64_t bins, int64_t mask) {
    int64_t h = hash_raw(i, s);
    if (mask >= 0) return (int)(h & mask);
    int64_t r = h % bins;
    if (r < 0) r += bins;
    return (int)r;
}

}  // namespace cresso

// error reporting shared by all host entry points (abi.cpp)
namespace cresso {
int32_t fail(int32_t code, const char* fmt, ...);
int32_t hip_fail(hipError_t e, const char* what);
}  // namespace cresso
