// Scalar (LoRA-thin / small tensor) route of CRESSO5 on gfx950.
//
// Math: the reference's PyTorch scalar step, cresso_v5.py:1505-1582 (its
// fused scalar_update_2d_cuda, cresso_cuda_kernel.cu:3225-3605, mirrors it for
// 2D tensors in 8 dense passes and 17 launches per tensor).
//
// ONE call updates every scalar-route tensor; one 1024-thread workgroup owns
// one tensor.  The step's dependent global reductions become block
// reductions:
//   A: sum f^2                                -> force-RMS reservoir, scale s
//   B: sum log1p((|f|/s+eps)^p), axis sums of the density
//                                             -> metric oscillator, instant metric
//   C: t = f / (s M I + eps); 13 moments of t  -> surprise, contact oscillator and,
//                                                in closed form, every RMS of the
//                                                drive shaping (root, shaped, core,
//                                                residual)
//   D: drive; sum drive^2                     -> drive-energy reservoir, gain
//   E: param -= lr * cast(drive * gain)
//
// Three kernels:
//  * scalar_resident_kernel: 2D tensors of <= 64 Ki elements whose rows map to
//    lane groups (LoRA-thin (L,16)) or whose rows are exactly one block wide
//    ((16,4096)); f, then t, then drive stay on chip (half of each thread's
//    64 elements in VGPRs, half in a 128 KiB LDS slot array), so HBM traffic is
//    the compulsory grad read + param read/write.  Axis sums use register
//    partials, fixed-order wave butterflies (DPP) and LDS, never float atomics.
//  * scalar_stream_kernel: every other shape/size/dtype; re-reads the grad in
//    each pass and keeps general-ndim axis sums as 64-bit fixed-point integers
//    in a global scratch area (integer atomics: order-independent results).
//  * micro_kernel: the dense micro-field route (descriptor route 1) of
//    cresso_v5.py:1355-1432, same plan, table and launch grouping.
#include "common.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

namespace cresso {
namespace {

constexpr int SR_NT = 1024;                                  // threads per tensor
constexpr int SR_SLOTS = 16;                                 // float4 slots per thread
constexpr int SR_VSLOTS = 8;                                 // slots held in VGPRs; the rest live in LDS
constexpr size_t SR_XLDS = (size_t)(SR_SLOTS - SR_VSLOTS) * SR_NT * 16;  // LDS bytes of the LDS slots (128 KiB)
constexpr size_t SR_LDS_MAX = 160 * 1024 - 4096;             // dynamic LDS budget of one workgroup (static LDS aside)
constexpr int64_t SR_RESIDENT_MAX = (int64_t)SR_NT * SR_SLOTS * 4;

enum Layout : int32_t { L_NONE = 0, L_1D = 1, L_ROWGROUP = 2, L_COLBLOCK = 3, L_GENERIC = 4, L_2D = 5 };

struct ScalarRec {
    cresso_scalar_desc d;
    int32_t layout;
    int32_t group;          // ROWGROUP: lanes per row (power of two <= 64)
    int64_t rows, cols;     // 2D geometry
    int64_t stride[8];      // row-major strides (GENERIC)
    int64_t axis_off[8];    // offset of each axis in the axis-sum array (GENERIC)
    int64_t sum_dims;       // GENERIC: sum of dims
    int64_t scratch_off;    // GENERIC: byte offset of the axis-sum scratch in the table
    int32_t frac_bits;      // GENERIC: fixed-point fraction bits of the axis sums
    int32_t resident;       // 1: scalar_resident_kernel
    int64_t ctl_off;        // wide form: byte offset of the tensor's StreamCtl in the table
    int32_t blk0, nblk;     // wide form: first block (within its group's launches) and block count
};

__device__ __forceinline__ float uni(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
}
__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }
// Read of a value that every thread of the block reads at the same address
// (a 0-dim state tensor): a scalar load through the constant address space.
// Each value is read once, before this kernel writes it back at its end.
__device__ __forceinline__ float ld_uniform(const float* p) {
    return *(const __attribute__((address_space(4))) float*)p;
}


// ---- vector access -------------------------------------------------------
template <typename T> struct V4;
template <> struct V4<float> {
    // buffer forms: 4 consecutive elements at byte offset voff + soff
    __device__ static void bld(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, float* o) {
        const f32x4 v = bload4(r, voff, soff);
        o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
    }
    __device__ static void bst(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, const float* v) {
        f32x4 w;
        w.x = v[0]; w.y = v[1]; w.z = v[2]; w.w = v[3];
        bstore4(r, voff, soff, w);
    }
    __device__ static void ld(const float* p, int64_t e, float* o) {
        const f32x4 v = gload4(p + e);
        o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
    }
    __device__ static void st(float* p, int64_t e, const float* v) {
        f32x4 w;
        w.x = v[0]; w.y = v[1]; w.z = v[2]; w.w = v[3];
        gstore4(p + e, w);
    }
};
template <typename T> struct V4h {
    __device__ static void bld(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, float* o) {
        const u32x2 q = bload2u(r, voff, soff);
        uint2 raw;
        raw.x = q.x; raw.y = q.y;
        const T* h = reinterpret_cast<const T*>(&raw);
        o[0] = to_f(h[0]); o[1] = to_f(h[1]); o[2] = to_f(h[2]); o[3] = to_f(h[3]);
    }
    __device__ static void bst(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, const float* v) {
        uint2 raw;
        T* h = reinterpret_cast<T*>(&raw);
        h[0] = from_w<T>(v[0]); h[1] = from_w<T>(v[1]); h[2] = from_w<T>(v[2]); h[3] = from_w<T>(v[3]);
        u32x2 q;
        q.x = raw.x; q.y = raw.y;
        bstore2u(r, voff, soff, q);
    }
    __device__ static void ld(const T* p, int64_t e, float* o) {
        const u32x2 r = gload2u(p + e);
        uint2 raw;
        raw.x = r.x; raw.y = r.y;
        const T* h = reinterpret_cast<const T*>(&raw);
        o[0] = to_f(h[0]); o[1] = to_f(h[1]); o[2] = to_f(h[2]); o[3] = to_f(h[3]);
    }
    __device__ static void st(T* p, int64_t e, const float* v) {
        uint2 raw;
        T* h = reinterpret_cast<T*>(&raw);
        h[0] = from_w<T>(v[0]); h[1] = from_w<T>(v[1]); h[2] = from_w<T>(v[2]); h[3] = from_w<T>(v[3]);
        u32x2 r;
        r.x = raw.x; r.y = raw.y;
        gstore2u(p + e, r);
    }
};
template <> struct V4<__half> : V4h<__half> {};
template <> struct V4<__hip_bfloat16> : V4h<__hip_bfloat16> {};

// Sum over aligned groups of G lanes (G a power of two <= 64), pairing lanes
// xor 1, 2, 4, ... in that order: xor 1 and 2 by DPP quad permutes, wider by
// shuffles (only when a group spans more than 4 lanes).
__device__ __forceinline__ float lanes_group_sum(float v, int G) {
    float o = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    v += G > 1 ? o : 0.0f;
    o = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    v += G > 2 ? o : 0.0f;
    if (G > 4)
        for (int m = 4; m < G; m <<= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// The same group sum in the work dtype (fp64 work pairs lanes by shuffles).
template <typename W> __device__ __forceinline__ W lanes_group_sum_w(W v, int G);
template <> __device__ __forceinline__ float lanes_group_sum_w<float>(float v, int G) { return lanes_group_sum(v, G); }
template <> __device__ __forceinline__ double lanes_group_sum_w<double>(double v, int G) {
    for (int m = 1; m < G; m <<= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// ---- shared scalar math (work dtype W) ------------------------------------
template <typename W> __device__ __forceinline__ W reservoir(W old, W cur, double decay, int step) {
    // cresso_v5.py:900-905: copy on the first step, else in-place EMA
    if (step <= 1) return cur;
    return old * (W)decay + (W)(1.0 - decay) * cur;
}

// rat = t/(1+|t|/clip), bnd = clip*tanh(t/clip), root = sign(t)*sqrt(min(|t|,clip^2)+eps)
// (cresso_v5.py:1563-1566); rat and bnd share one reciprocal.
template <typename W>
__device__ __forceinline__ void shape3(W t, W iclip, W clip, W clip2, W eps, W& rat, W& bnd, W& root) {
    const W at = t < 0 ? -t : t;
    const W ex = fexp((W)-2 * at * iclip);
    const W d1 = (W)1 + ex;
    const W d2 = (W)1 + at * iclip;
    const W inv = frcp(d1 * d2);
    const W th = ((W)1 - ex) * d2 * inv;
    bnd = (t < 0 ? -th : th) * clip;
    rat = t * d1 * inv;
    root = fsign(t) * fsqrt((at < clip2 ? at : clip2) + eps);
}

// Everything a drive evaluation needs after the pass-C reduction.
template <typename W> struct DriveCoef {
    W q1, cA, cB, cN, cD, cr, cb, co, ct, nscale;
};

// Scalar-state update between passes C and D: surprise, contact oscillator
// (cresso_v5.py:1525-1547) and the drive-shaping coefficients in closed form
// from the moments M (cresso_v5.py:1549-1576).
template <typename W>
__device__ DriveCoef<W> contact_and_coefs(const double* M, double dn, const cresso_hyper& h, int step, W q0, W& imp,
                                          W& act, W& sur) {
    const W eps = (W)h.eps;
    sur = reservoir(sur, (W)sqrt((double)(W)(M[1] / dn) + (double)eps), h.surprise_decay, step);
    const W port = (W)(M[0] / dn);
    const W S = sur;
    const W dt = (W)h.dt;
    const W plast = (W)1 + (W)h.surprise_gain * S / ((W)1 + S);
    const W brake = (W)1 / ((W)1 + (W)h.surprise_brake * S);
    const W energy = (W)0.5 * (imp * imp + q0 * q0);
    act = act * (W)0.985 + dt * (port * imp - energy);
    const W fric = (W)h.impulse_friction + (W)h.contact_gain * (W)tanh((double)(act < 0 ? -act : act));
    const W damp = (W)1 - dt * fric;
    imp = imp * (damp > 0 ? damp : (W)0);
    imp = imp + dt * (plast * brake * port - (W)h.restoring * q0 - (W)h.cubic * (q0 * q0 * q0));
    W q1 = q0 + dt * imp;
    q1 = q1 < (W)-8 ? (W)-8 : (q1 > (W)8 ? (W)8 : q1);

    const W frms = (W)sqrt((double)((W)(M[3] / dn) + eps));
    const W prms = (W)sqrt((double)(q1 * q1 + eps));
    W align = (W)((double)q1 * M[2] / dn) / (frms * prms + eps);
    align = align < (W)-1 ? (W)-1 : (align > (W)1 ? (W)1 : align);
    W agate = (align + (W)1) * (W)0.5;
    agate = agate < 0 ? (W)0 : (agate > 1 ? (W)1 : agate);
    // the predicate prms > sqrt(eps) in fp64 (in fp32 it is a rounding tie
    // when q1^2 is below half an ulp of eps)
    if (!(sqrt((double)q1 * (double)q1 + h.eps) > sqrt(h.eps))) agate = 0;
    const double warm = h.warmup_steps == 0 ? 1.0 : 1.0 - exp(-(double)step / (double)(h.warmup_steps > 1 ? h.warmup_steps : 1));
    const W mix = (W)(h.prediction_mix * warm) * agate / ((W)1 + S);
    const W rms_rat = (W)sqrt((double)((W)(M[4] / dn) + eps));
    const W rms_root = (W)sqrt((double)((W)(M[6] / dn) + eps));
    const W kroot = rms_rat / (rms_root > eps ? rms_root : eps);
    const W spike = (W)h.spike_mix / ((W)1 + S);
    const W rmix = (W)h.root_channel_mix / ((W)1 + (W)0.5 * S);
    const double ar = (double)(((W)1 - rmix) * ((W)1 - spike));
    const double ab = (double)(((W)1 - rmix) * spike);
    const double ao = (double)(rmix * kroot);
    const double Srr = M[4], Sbb = M[5], Soo = M[6], Srb = M[7], Sro = M[8], Sbo = M[9];
    const double Stt = M[3], Str = M[10], Stb = M[11], Sto = M[12];
    const double sh2 = ar * ar * Srr + ab * ab * Sbb + ao * ao * Soo + 2.0 * (ar * ab * Srb + ar * ao * Sro + ab * ao * Sbo);
    const W srms = (W)sqrt((double)((W)(sh2 / dn) + eps));
    const W dmix = (W)h.direct_force_mix / ((W)1 + (W)0.35 * S);
    const W kdir = srms / (frms > eps ? frms : eps);
    const double cr = (1.0 - (double)dmix) * ar, cb = (1.0 - (double)dmix) * ab, co = (1.0 - (double)dmix) * ao;
    const double ct = (double)(dmix * kdir);
    const double core2 = cr * cr * Srr + cb * cb * Sbb + co * co * Soo + ct * ct * Stt +
                         2.0 * (cr * cb * Srb + cr * co * Sro + cb * co * Sbo + ct * cr * Str + ct * cb * Stb + ct * co * Sto);
    const W crms = (W)sqrt((double)((W)(core2 / dn) + eps));
    const double delta = (double)q1 - (double)q0;
    const double ee1 = fmax(M[1] - 2.0 * delta * M[0] + dn * delta * delta, 0.0);
    const W erms = (W)sqrt((double)((W)(ee1 / dn) + eps));
    const W resmix = (W)h.residual_feedback_mix / ((W)1 + S);
    const W kres = crms / (erms > eps ? erms : eps);
    DriveCoef<W> c;
    c.q1 = q1;
    c.cA = (W)1 - mix;
    c.cB = mix * q1;
    c.cN = (W)h.novelty_mix;
    c.cD = resmix * kres;
    c.cr = (W)cr; c.cb = (W)cb; c.co = (W)co; c.ct = (W)ct;
    c.nscale = (W)1 / ((W)h.drive_clip * ((W)1 + S));
    return c;
}

// ---------------------------------------------------------------------------
// register-resident kernel (2D, <= 64 Ki elements, float4-aligned)
// ---------------------------------------------------------------------------
// FAST: numel is exactly SR_NT*SR_SLOTS*4 (65536, e.g. (4096,16) and
// (16,4096)), so every slot of every thread is valid with no guard at all and
// the loads of a pass are all in flight together, and the options that add
// per-element work are off (weight decay, local sharpness, an instant-metric
// power other than 1).  The drive shaping then
// runs on |t| (shape3a): the moments need no signs, and the drive takes the
// sign of t once.
template <typename PT, typename GT, int LAYOUT, bool FAST>
__device__ __forceinline__ void resident_body(const ScalarRec* __restrict__ recs, int32_t* __restrict__ steps,
                                              const void* const* __restrict__ grads, int32_t first,
                                              const cresso_hyper& h, double* __restrict__ red, int& s_step) {
    extern __shared__ __align__(16) unsigned char dyn[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int ri = first + blockIdx.x;
    const ScalarRec& R = recs[ri];
    const int64_t n = R.d.numel;
    const int64_t rows = R.rows;
    const int C0 = (int)R.cols;
    const int G = R.group;                        // ROWGROUP: a power of two <= 64
    const int lgG = G > 0 ? __builtin_ctz(G) : 0;
    const float eps = (float)h.eps;
    double* const pub = red + 16 * SR_SLOTS;                          // block totals (block_sum_f)
    float* const s_dc = reinterpret_cast<float*>(pub + SR_SLOTS);     // drive coefficients, wave 0 -> all
    float* sp[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) sp[i] = reinterpret_cast<float*>(R.d.state[i]);
    // uniform state: scalar loads into SGPRs (issued together, no VGPRs held)
    float q0 = ld_uniform(sp[0]), imp = ld_uniform(sp[1]), mq = ld_uniform(sp[2]), mp = ld_uniform(sp[3]);
    float fr = ld_uniform(sp[4]), de = ld_uniform(sp[5]), sur = ld_uniform(sp[6]), act = ld_uniform(sp[7]);
    if (tid == 0) {
        const int s = steps[ri] + 1;
        steps[ri] = s;
        s_step = s;
    }
    const GT* __restrict__ g = reinterpret_cast<const GT*>(grads[ri]);
    PT* __restrict__ p = reinterpret_cast<PT*>(R.d.param);
    const bool wd_on = h.weight_decay != 0.0;
    const float wd = (float)h.weight_decay;

    // per-thread element slots: the first SR_VSLOTS in VGPRs, the rest in LDS
    // ([slot][thread] float4, conflict-free); k is a compile-time constant at
    // every use, so the choice folds away
    float xv[SR_VSLOTS * 4];
    float4* __restrict__ xl = reinterpret_cast<float4*>(dyn);
    unsigned char* const dyn2 = dyn + SR_XLDS;
    auto ldx = [&](int k, float* v) {
        if (k < SR_VSLOTS) {
#pragma unroll
            for (int c = 0; c < 4; ++c) v[c] = xv[4 * k + c];
        } else {
            const float4 q = xl[(k - SR_VSLOTS) * SR_NT + tid];
            v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
        }
    };
    auto stx = [&](int k, const float* v) {
        if (k < SR_VSLOTS) {
#pragma unroll
            for (int c = 0; c < 4; ++c) xv[4 * k + c] = v[c];
        } else {
            xl[(k - SR_VSLOTS) * SR_NT + tid] = make_float4(v[0], v[1], v[2], v[3]);
        }
    };
    auto e0_of = [&](int k) -> int64_t { return ((int64_t)k * SR_NT + tid) * 4; };

    // FAST: buffer views of grad and param (byte offsets fit in 32 bits)
    const __amdgpu_buffer_rsrc_t rg = make_rsrc(g, FAST ? (uint32_t)(n * (int64_t)sizeof(GT)) : 0u);
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(p, FAST ? (uint32_t)(n * (int64_t)sizeof(PT)) : 0u);
    const uint32_t vog = (uint32_t)(tid * 4 * sizeof(GT)), vop = (uint32_t)(tid * 4 * sizeof(PT));

    // ---- pass A ----
    float a_ff = 0.f;
#pragma unroll
    for (int k = 0; k < SR_SLOTS; ++k) {
        const int64_t e0 = e0_of(k);
        float v[4];
        if constexpr (FAST) {
            // the raw grad is kept: maximize (force = -grad) enters pass C as
            // the sign of the denominator, the only place the force's sign is used
            V4<GT>::bld(rg, vog, (uint32_t)(k * SR_NT * 4 * sizeof(GT)), v);
#pragma unroll
            for (int c = 0; c < 4; ++c) a_ff = fmaf(v[c], v[c], a_ff);
            stx(k, v);
            continue;
        }
        if (e0 < n) {
            V4<GT>::ld(g, e0, v);
            if (h.maximize) {
#pragma unroll
                for (int c = 0; c < 4; ++c) v[c] = -v[c];
            }
            if (wd_on) {
                float pv[4];
                V4<PT>::ld(p, e0, pv);
#pragma unroll
                for (int c = 0; c < 4; ++c) v[c] = v[c] + wd * pv[c];
            }
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c) v[c] = 0.f;
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) a_ff += v[c] * v[c];
        stx(k, v);
    }
    __syncthreads();
    const int step = s_step;
    const double dn = (double)n;
    {
        const float x[1] = {a_ff};
        double v[1];
        block_sum_f<1>(x, v, red, pub);
        fr = reservoir(fr, sqrtf((float)(v[0] / dn) + eps), h.reservoir_decay, step);
    }
    const float scale = fmaxf(fr, eps);
    const float inv_s = uni(1.0f / scale);

    // ---- pass B ----
    const float pw = uni((float)h.energy_power);
    const float ipw = (float)fmax(h.instant_metric_power, 0.25);
    const bool ip_one = ipw == 1.0f;
    const float kappa = (float)(h.instant_metric_coupling / (2.0 * fmax(h.instant_metric_power, 0.25)));
    float* rowfac = reinterpret_cast<float*>(dyn2);                      // [rows]
    double* colred = reinterpret_cast<double*>(dyn2 + ((sizeof(float) * rows + 15) & ~(size_t)15));  // [16][C0]
    float colacc[4] = {0.f, 0.f, 0.f, 0.f};
    float slotrow[SR_SLOTS];  // COLBLOCK: per-slot row partials
    float a_L = 0.f, a_dens = 0.f;
#pragma unroll
    for (int k = 0; k < SR_SLOTS; ++k) {
        const bool ok = FAST || e0_of(k) < n;
        float rs = 0.f;
        if constexpr (FAST) {
            // a_L sums log2(1 + r^p) (scaled by ln 2 after the block sum);
            // r >= eps, so the instant density is min(r, 1e4)
            if (ok) {
                float xk[4];
                ldx(k, xk);
                pin4(xk);
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const float r = fmaf(fabsf(xk[c]), inv_s, eps);
                    a_L += flog2(1.0f + fexp2(pw * flog2(r)));
                    const float dens = fminf(r, 1.0e4f);
                    rs += dens;
                    colacc[c] += dens;
                    sched_fence();
                }
                pin1(a_L);
                a_dens += rs;
            }
        } else {
            float xk[4];
            ldx(k, xk);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const float r = fabsf(xk[c]) * inv_s + eps;
                const float L = flog1p(fpow(r, pw));
                const float rl = fmaxf(fminf(r, 1.0e4f), eps);
                const float dens = fminf(ip_one ? rl : fpow(rl, ipw), 1.0e6f);
                if (ok) {
                    a_L += L;
                    a_dens += dens;
                    rs += dens;
                    colacc[c] += dens;
                }
                sched_fence();
            }
        }
        if (LAYOUT == L_ROWGROUP) {
            rs = lanes_group_sum(rs, G);
            const int row = (k * SR_NT + tid) >> lgG;
            if (ok && (tid & (G - 1)) == 0) rowfac[row] = rs;
        } else if (FAST) {
            // the row of slot k is the whole block: its wave totals now (DPP),
            // summed over the waves in fp64 after the pass
            const float w = wave_total(rs);
            if (lane == 63) red[(tid >> 6) * SR_SLOTS + k] = (double)w;
        } else {
            slotrow[k] = rs;
        }
    }
    double rowsum = 0.0;   // FAST COLBLOCK: density sum of row tid (threads < SR_SLOTS)
    if (FAST && LAYOUT == L_COLBLOCK) {
        __syncthreads();
        if (tid < SR_SLOTS)
            for (int w = 0; w < SR_NT / 64; ++w) rowsum += red[w * SR_SLOTS + tid];
        __syncthreads();   // red is reused by the next block sum
    }
    double gmean;
    {
        const float x[2] = {a_L, a_dens};
        double v[2];
        block_sum_f<2>(x, v, red, pub);
        const float dens_mean = (float)((FAST ? v[0] * 0.6931471805599453 : v[0]) / dn);
        gmean = v[1] / dn;
        // scalar metric oscillator (cresso_v5.py:1510-1518)
        const float mport = dens_mean - tanhf(mq);
        mp = mp * (float)fmax(0.0, 1.0 - h.metric_dt * h.metric_friction);
        mp = mp + (float)h.metric_dt * (mport - mq);
        mq = mq + (float)h.metric_dt * mp;
        mq = clampf(mq, -3.0f, 3.0f);
    }
    const float metric = clampf(expf((float)h.metric_coupling * mq), 0.06f, 16.0f);
    const float gden = (float)fmax(gmean, (double)eps);
    float Ec[4];
    if (LAYOUT == L_ROWGROUP) {
        // column sums: butterfly over lanes sharing tid % G, then waves in order
        float cs[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            cs[c] = colacc[c];
            for (int m = G; m < 64; m <<= 1) cs[c] += __shfl_xor(cs[c], m, 64);
        }
        const int wave = tid >> 6;
        if (lane < G) {
#pragma unroll
            for (int c = 0; c < 4; ++c) colred[wave * C0 + lane * 4 + c] = (double)cs[c];
        }
        __syncthreads();   // rowfac and colred complete
        float* colfac = reinterpret_cast<float*>(colred + 16 * C0);
        if (tid < C0) {
            double s = 0.0;
            for (int w = 0; w < SR_NT / 64; ++w) s += colred[w * C0 + tid];
            const float cm = (float)(s / (double)rows);
            colfac[tid] = fexp2(kappa * flog2(fmaxf(cm / gden, eps)));
        }
        for (int64_t i = tid; i < rows; i += SR_NT) {
            const float rm = rowfac[i] / (float)C0;
            rowfac[i] = fexp2(kappa * flog2(fmaxf(rm / gden, eps)));
        }
        __syncthreads();
        const int cg = tid & (G - 1);
#pragma unroll
        for (int c = 0; c < 4; ++c) Ec[c] = colfac[cg * 4 + c];
    } else {
        if (!FAST) {
            double v[SR_SLOTS];
            block_sum_f<SR_SLOTS>(slotrow, v, red, pub);
            if (tid < SR_SLOTS) rowsum = v[tid];
        }
        if (tid < SR_SLOTS && tid < rows) {
            const float rm = (float)(rowsum / (double)C0);
            rowfac[tid] = fexp2(kappa * flog2(fmaxf(rm / gden, eps)));
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float cm = colacc[c] / (float)rows;
            Ec[c] = fexp2(kappa * flog2(fmaxf(cm / gden, eps)));
        }
        __syncthreads();
    }

    // ---- pass C ----
    const float sM = uni(scale * metric);
    const bool ls_on = h.local_sharpness != 0.0;
    const float ls = (float)h.local_sharpness;
    const float clip = uni((float)h.drive_clip);
    const float iclip = uni(1.0f / clip);
    const float clip2 = uni(clip * clip);
    const float k2 = uni(-2.8853900817779268f * iclip);   // -2 log2(e) / clip
    // FAST keeps the raw grad: f / den = grad / (sign * den) with sign = -1 under maximize
    const float sMs = uni(h.maximize ? -sM : sM), epss = uni(h.maximize ? -eps : eps);
    float m[13];
#pragma unroll
    for (int i = 0; i < 13; ++i) m[i] = 0.f;
#pragma unroll
    for (int k = 0; k < SR_SLOTS; ++k) {
        const bool ok = FAST || e0_of(k) < n;
        const int row = LAYOUT == L_ROWGROUP ? (k * SR_NT + tid) >> lgG : k;
        if constexpr (FAST) {
            if (ok) {
                const float Er = rowfac[row];
                float xk[4];
                ldx(k, xk);
                pin4(xk);
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const float inst = med3f(Er * Ec[c], 0.08f, 12.0f);
                    const float t = med3f(xk[c] * frcp(fmaf(sMs, inst, epss)), -1.0e4f, 1.0e4f);
                    xk[c] = t;
                    const float at = fabsf(t);
                    const Shape3A z = shape3a(at, k2, iclip, clip2, eps);
                    const float e = t - q0;
                    m[0] += e; m[1] = fmaf(e, e, m[1]); m[2] += t; m[3] = fmaf(t, t, m[3]);
                    m[4] = fmaf(z.rat, z.rat, m[4]); m[5] = fmaf(z.th, z.th, m[5]); m[6] = fmaf(z.root, z.root, m[6]);
                    m[7] = fmaf(z.rat, z.th, m[7]); m[8] = fmaf(z.rat, z.root, m[8]); m[9] = fmaf(z.th, z.root, m[9]);
                    m[10] = fmaf(at, z.rat, m[10]); m[11] = fmaf(at, z.th, m[11]); m[12] = fmaf(at, z.root, m[12]);
                    sched_fence();
                }
#pragma unroll
                for (int i = 0; i < 13; ++i) pin1(m[i]);
                stx(k, xk);
            }
            continue;
        }
        const float Er = ok ? rowfac[row] : 1.0f;
        float xk[4];
        ldx(k, xk);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float f = xk[c];
            float den = sM;
            if (ls_on) {
                const float rel = fminf(fabsf(f) * inv_s + eps, 1.0e4f);
                den = den * clampf(1.0f + ls * fsqrt(fminf(rel, 100.0f)), 1.0f, 8.0f);
            }
            const float inst = clampf(Er * Ec[c], 0.08f, 12.0f);
            const float t = clampf(f * frcp(den * inst + eps), -1.0e4f, 1.0e4f);
            xk[c] = t;
            if (ok) {
                float rat, bnd, root;
                shape3(t, iclip, clip, clip2, eps, rat, bnd, root);
                const float e = t - q0;
                m[0] += e; m[1] += e * e; m[2] += t; m[3] += t * t;
                m[4] += rat * rat; m[5] += bnd * bnd; m[6] += root * root;
                m[7] += rat * bnd; m[8] += rat * root; m[9] += bnd * root;
                m[10] += t * rat; m[11] += t * bnd; m[12] += t * root;
            }
            sched_fence();
        }
        stx(k, xk);
    }
    double M[13];
    block_sum_f<13>(m, M, red, pub);
    if (FAST) {
        // the FAST sums hold |tanh| where the moments need bnd = clip tanh
        const double dc_ = (double)clip;
        M[5] *= dc_ * dc_;
        M[7] *= dc_;
        M[9] *= dc_;
        M[11] *= dc_;
    }
    // the scalar-state update and the coefficients: wave 0 computes them (the
    // other waves would repeat the same uniform fp64 work), LDS hands them out
    if (tid < kWave) {
        const DriveCoef<float> c = contact_and_coefs<float>(M, dn, h, step, q0, imp, act, sur);
        if (tid == 0) {
            s_dc[0] = c.q1; s_dc[1] = c.cA; s_dc[2] = c.cB; s_dc[3] = c.cN; s_dc[4] = c.cD;
            s_dc[5] = c.cr; s_dc[6] = c.cb; s_dc[7] = c.co; s_dc[8] = c.ct; s_dc[9] = c.nscale;
        }
    }
    __syncthreads();
    DriveCoef<float> dc;
    dc.q1 = uni(s_dc[0]); dc.cA = uni(s_dc[1]); dc.cB = uni(s_dc[2]); dc.cN = uni(s_dc[3]); dc.cD = uni(s_dc[4]);
    dc.cr = uni(s_dc[5]); dc.cb = uni(s_dc[6]); dc.co = uni(s_dc[7]); dc.ct = uni(s_dc[8]); dc.nscale = uni(s_dc[9]);

    // ---- pass D ----
    const float q1 = uni(dc.q1), cA = uni(dc.cA), cB = uni(dc.cB), cN = uni(dc.cN), cD = uni(dc.cD);
    const float cr = uni(dc.cr), cb = uni(dc.cb), co = uni(dc.co), ct = uni(dc.ct), ns = uni(dc.nscale);
    // FAST coefficients: cA folded into the core weights, clip into the tanh weights
    const float kr = uni(cA * cr), kb = uni(cA * (cb * clip)), ko = uni(cA * co), kt = uni(cA * ct);
    const float kN = uni(cN * clip), k2n = uni(-2.8853900817779268f * ns);
    float a_dd = 0.f;
#pragma unroll
    for (int k = 0; k < SR_SLOTS; ++k) {
        const bool ok = FAST || e0_of(k) < n;
        if constexpr (FAST) {
            // drive = sign(t) (kr|rat| + kb|tanh| + ko|root| + kt|t|) + kB + kN tanh(e ns) + kD e
            if (ok) {
                float xk[4];
                ldx(k, xk);
                pin4(xk);
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const float t = xk[c];
                    const float at = fabsf(t);
                    const float e = t - q1;
                    // shape3a's 1/(d1 d2) and the novelty's 1/(1 + ex) from one reciprocal
                    const float es = fexp2(k2 * at);
                    const float d1 = 1.0f + es;
                    const float d2 = fmaf(at, iclip, 1.0f);
                    const float ex = fexp2(k2n * fabsf(e));
                    const float dn1 = 1.0f + ex;
                    const float d12 = d1 * d2;
                    const float rr = frcp(d12 * dn1);
                    const float inv = dn1 * rr;    // 1/(d1 d2)
                    const float ri = d12 * rr;     // 1/(1 + ex)
                    const float u = d2 * inv;      // 1/d1
                    Shape3A z;
                    z.th = fmaf(-es, u, u);
                    z.rat = at * (d1 * inv);
                    const float rt = fsqrt(fminf(at, clip2) + eps);
                    z.root = at > 0.0f ? rt : 0.0f;
                    const float cm = fmaf(kt, at, fmaf(ko, z.root, fmaf(kb, z.th, kr * z.rat)));
                    const float core = xorsign(cm, t);
                    const float nov = with_sign(fmaf(-ex, ri, ri), e);
                    const float drv = fmaf(kN, nov, fmaf(cD, e, core + cB));
                    xk[c] = drv;
                    a_dd = fmaf(drv, drv, a_dd);
                    sched_fence();
                }
                pin1(a_dd);
                stx(k, xk);
            }
            continue;
        }
        float xk[4];
        ldx(k, xk);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float t = xk[c];
            float rat, bnd, root;
            shape3(t, iclip, clip, clip2, eps, rat, bnd, root);
            const float e = t - q1;
            const float nov = ftanh(e * ns) * clip;
            const float core = cr * rat + cb * bnd + co * root + ct * t;
            const float drv = cA * core + cB + cN * nov + cD * e;
            xk[c] = drv;
            if (ok) a_dd += drv * drv;
            sched_fence();
        }
        stx(k, xk);
    }
    {
        const float x[1] = {a_dd};
        double v[1];
        block_sum_f<1>(x, v, red, pub);
        de = reservoir(de, (float)(v[0] / dn), h.reservoir_decay, step);
    }
    const float gain = uni(clampf((float)h.target_update_rms / sqrtf(de + eps), (float)h.min_gain, (float)h.max_gain));

    // ---- pass E ----
    const float nlr = uni((float)update_alpha<PT>(-h.lr));
    if constexpr (FAST) {
        // groups of 4 slots; the param loads of group j+1 are issued before
        // group j is updated (two groups of loads in flight, bounded registers)
        constexpr int GS = 4, NG = SR_SLOTS / GS;
        float pv[2][GS][4];
        auto issue = [&](int j) {
#pragma unroll
            for (int i = 0; i < GS; ++i)
                V4<PT>::bld(rp, vop, (uint32_t)((j * GS + i) * SR_NT * 4 * sizeof(PT)), pv[j & 1][i]);
        };
        issue(0);
#pragma unroll
        for (int j = 0; j < NG; ++j) {
            if (j + 1 < NG) issue(j + 1);
            sched_fence();
#pragma unroll
            for (int i = 0; i < GS; ++i) {
                const int k = j * GS + i;
                float xk[4];
                ldx(k, xk);
                float* pp = pv[j & 1][i];
#pragma unroll
                for (int c = 0; c < 4; ++c) pp[c] = pp[c] + nlr * to_f(from_w<PT>(xk[c] * gain));
                V4<PT>::bst(rp, vop, (uint32_t)(k * SR_NT * 4 * sizeof(PT)), pp);
            }
            sched_fence();
        }
    }
#pragma unroll
    for (int k = 0; k < SR_SLOTS; ++k) {
        if (FAST) break;
        const int64_t e0 = e0_of(k);
        if (e0 < n) {
            float pv[4], xk[4];
            ldx(k, xk);
            V4<PT>::ld(p, e0, pv);
#pragma unroll
            for (int c = 0; c < 4; ++c) pv[c] = pv[c] + nlr * to_f(from_w<PT>(xk[c] * gain));
            V4<PT>::st(p, e0, pv);
        }
    }
    if (tid == 0) {
        *sp[0] = dc.q1; *sp[1] = imp; *sp[2] = mq; *sp[3] = mp; *sp[4] = fr; *sp[5] = de; *sp[6] = sur; *sp[7] = act;
    }
}

// Both resident layouts in one launch (the layout is uniform per workgroup),
// so the plan's resident tensors fill the CUs in one sequence of rounds.
// Staggered start of a multi-round launch.  A resident workgroup streams its
// tensor from HBM (pass A), computes on chip (passes B-D, no HBM traffic), then
// streams the update (pass E).  With identical tensors on every CU all CUs are
// in the same phase, so the HBM phases of the whole chip do not overlap any
// compute phase.  Workgroups [lo, hi) of the first round (the second half of
// the CUs) wait `ticks` of the constant 100 MHz clock before starting, which
// keeps the two halves of the CUs in different phases for the whole launch.
// The wait is bounded; results do not depend on it.
struct Stagger {
    int32_t lo, hi;
    uint32_t ticks;
};

template <typename PT, typename GT, bool FAST>
__global__ __launch_bounds__(SR_NT) void scalar_resident_kernel(const ScalarRec* __restrict__ recs,
                                                                 int32_t* __restrict__ steps,
                                                                 const void* const* __restrict__ grads, int32_t first,
                                                                 cresso_hyper h, Stagger sg) {
    // wave totals [16][<= SR_SLOTS] | published block totals [SR_SLOTS] | drive coefficients
    __shared__ double red[16 * SR_SLOTS + SR_SLOTS + 8];
    __shared__ int s_step;
    if ((int32_t)blockIdx.x >= sg.lo && (int32_t)blockIdx.x < sg.hi) {
        const uint64_t t0 = wall_clock64();
        while (wall_clock64() - t0 < (uint64_t)sg.ticks) __builtin_amdgcn_s_sleep(32);
    }
    if (recs[first + blockIdx.x].layout == L_ROWGROUP)
        resident_body<PT, GT, L_ROWGROUP, FAST>(recs, steps, grads, first, h, red, s_step);
    else
        resident_body<PT, GT, L_COLBLOCK, FAST>(recs, steps, grads, first, h, red, s_step);
}

// ---------------------------------------------------------------------------
// streaming passes (any shape, any size; work dtype W)
// ---------------------------------------------------------------------------
// The five passes of the scalar step over a range of elements, and the
// per-tensor finishes between them, in two launch forms:
//   - scalar_stream_kernel: one workgroup per tensor runs every pass over the
//     whole tensor, with block reductions between the passes;
//   - the wide form (tensors of more than 64 Ki elements, or of 16 Ki and
//     more when the plan holds fewer than 256 of those): each pass is
//     one launch over chunks of SR_WIDE_CH elements of every tensor of the
//     group, writing block partials; a finish kernel (one workgroup per
//     tensor) reduces them in block order and carries the tensor's values
//     (StreamCtl, in the plan table) to the next pass.  Ten launches per
//     step, but a large tensor uses the whole GPU instead of one CU.
// Axis sums of the instant metric are 64-bit fixed-point integer atomics, so
// both forms get the same sums whatever the arrival order.
template <typename W> struct StreamCtl {
    W q0, imp, mq, mp, fr, de, sur, act;   // state scalars, advanced by the finishes
    W scale, inv_s, sM, gden, gain;
    DriveCoef<W> dc;
    int32_t step;
};
constexpr int SR_WIDE_NT = 256;              // threads per block of the wide form
constexpr int64_t SR_WIDE_CH = 8192;         // elements per block of the wide form
constexpr int64_t SR_WIDE_MIN = SR_RESIDENT_MAX + 1;   // non-resident tensors this large use the wide form
constexpr int64_t SR_WIDE_MID = 16384;       // ... and from this size when fewer than SR_WIDE_FILL of them
constexpr int32_t SR_WIDE_FILL = 256;        //     (one workgroup per tensor would leave CUs idle)
constexpr size_t SR_CTL_BYTES = 256;         // table bytes of one StreamCtl
static_assert(sizeof(StreamCtl<double>) <= SR_CTL_BYTES, "StreamCtl slot");

template <typename W, typename T> __device__ __forceinline__ W ldw(const T* p, int64_t i) { return to_w<W>(p[i]); }

// Row and column of a linear index in an L_2D tensor, advanced by a fixed
// stride without divisions.
struct Walk2D {
    uint32_t row, col, dR, dC, C;
    __device__ __forceinline__ void next() {
        col += dC;
        row += dR;
        if (col >= C) {
            col -= C;
            ++row;
        }
    }
};

template <typename W, typename PT, typename GT> struct Stream {
    const ScalarRec& R;
    const cresso_hyper& h;
    const GT* __restrict__ g;
    PT* __restrict__ p;
    int64_t n;
    double dn;
    int nd, layout;
    bool wd_on, neg, ls_on, axes;
    W eps, wd, pw, ipw, kappa, ls, clip, iclip, clip2;
    uint32_t C2, R2;   // L_2D cols and rows (1 otherwise)
    bool mulfac;       // axis factors stored as exp(kappa log r) and multiplied
    double fx_scale;
    unsigned long long* axis_fx;
    W* axis_fac;

    __device__ Stream(const ScalarRec& r, const cresso_hyper& hy, const void* grad, unsigned char* table) : R(r), h(hy) {
        g = reinterpret_cast<const GT*>(grad);
        p = reinterpret_cast<PT*>(R.d.param);
        n = R.d.numel;
        dn = (double)n;
        nd = R.d.ndim;
        layout = R.layout;
        wd_on = h.weight_decay != 0.0;
        neg = h.maximize != 0;
        ls_on = h.local_sharpness != 0.0;
        axes = layout == L_GENERIC || layout == L_2D;
        eps = (W)h.eps;
        wd = (W)h.weight_decay;
        pw = (W)h.energy_power;
        ipw = (W)fmax(h.instant_metric_power, 0.25);
        kappa = nd > 0 ? (W)(h.instant_metric_coupling / ((double)nd * fmax(h.instant_metric_power, 0.25))) : (W)0;
        ls = (W)h.local_sharpness;
        clip = (W)h.drive_clip;
        iclip = (W)1 / clip;
        clip2 = clip * clip;
        C2 = layout == L_2D ? (uint32_t)R.cols : 1u;
        R2 = layout == L_2D ? (uint32_t)R.rows : 1u;
        // r = axis mean / global mean lies in [eps, 1e6 / eps], so the product of
        // the nd factors r^kappa stays within exp(+-kappa nd log(1e6 / eps)): when
        // that is inside the work dtype's range, the factors are stored as powers
        // and multiplied (no exp per element); otherwise as logs, summed, exp'd
        mulfac = (double)kappa * (double)nd * log(1.0e6 / fmin(h.eps, 0.5)) < (sizeof(W) == 8 ? 600.0 : 80.0);
        fx_scale = ldexp(1.0, R.frac_bits);
        axis_fx = reinterpret_cast<unsigned long long*>(table + R.scratch_off);
        axis_fac = reinterpret_cast<W*>(table + R.scratch_off + sizeof(unsigned long long) * R.sum_dims);
    }

    __device__ W* st(int k) const { return reinterpret_cast<W*>(R.d.state[k]); }
    __device__ void load_state(StreamCtl<W>& c) const {
        c.q0 = *st(0); c.imp = *st(1); c.mq = *st(2); c.mp = *st(3);
        c.fr = *st(4); c.de = *st(5); c.sur = *st(6); c.act = *st(7);
    }
    __device__ void store_state(const StreamCtl<W>& c) const {
        *st(0) = c.dc.q1; *st(1) = c.imp; *st(2) = c.mq; *st(3) = c.mp;
        *st(4) = c.fr; *st(5) = c.de; *st(6) = c.sur; *st(7) = c.act;
    }

    // force from the grad and the element's param value pv (read only under weight decay)
    __device__ unsigned long long fx(W v) const { return (unsigned long long)llrint((double)v * fx_scale); }
    __device__ W force(int64_t i, W pv) const {
        W f = ldw<W>(g, i);
        if (neg) f = -f;
        if (wd_on) f = f + wd * pv;
        return f;
    }
    static constexpr int U = sizeof(W) == 8 ? 2 : 8;   // elements per thread whose loads are in flight together

    // The element's axis factors: L_2D the row's and the column's; GENERIC
    // their product (mulfac) or sum in fa, the identity in fb.
    __device__ void axis_load(int64_t i, const Walk2D& w, W& fa, W& fb) const {
        if (layout == L_2D) {
            fa = axis_fac[w.row];
            fb = axis_fac[R2 + w.col];
        } else if (layout == L_GENERIC) {
            W acc = mulfac ? (W)1 : (W)0;
            for (int ax = 0; ax < nd; ++ax) {
                const W v = axis_fac[R.axis_off[ax] + (i / R.stride[ax]) % R.d.shape[ax]];
                acc = mulfac ? acc * v : acc + v;
            }
            fa = acc;
            fb = mulfac ? (W)1 : (W)0;
        }
    }

    // fn(f, pv, fa, fb) for elements i = i0 + tid + k S < i1 in order; the
    // loads of U elements (grad; param when PV or under weight decay; axis
    // factors when AX) are issued before any of them is used.
    template <bool PV, bool AX, typename F>
    __device__ void each(int64_t i0, int64_t i1, int tid, int S, F&& fn) const {
        Walk2D w = walk(i0 + tid, S);
        for (int64_t ib = i0 + tid; ib < i1; ib += (int64_t)U * S) {
            W f[U], pv[U], fa[U], fb[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int64_t i = ib + (int64_t)u * S;
                pv[u] = 0;
                f[u] = 0;
                fa[u] = 0;
                fb[u] = 0;
                if (i < i1) {
                    if (PV || wd_on) pv[u] = ldw<W>(p, i);
                    f[u] = force(i, pv[u]);
                    if (AX) axis_load(i, w, fa[u], fb[u]);
                }
                w.next();
            }
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (ib + (int64_t)u * S < i1) fn(f[u], pv[u], fa[u], fb[u]);
        }
    }
    // Same over whole waves: every lane of a wave makes the same calls
    // fn(i, ok, f, w), with ok false (and f = 0) past i1.
    template <typename F>
    __device__ void each_wave(int64_t i0, int64_t i1, int tid, int S, F&& fn) const {
        const int lane = tid & 63;
        Walk2D w = walk(i0 + tid, S);
        for (int64_t wb = i0 + (tid - lane); wb < i1; wb += (int64_t)U * S) {
            W f[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int64_t i = wb + (int64_t)u * S + lane;
                f[u] = 0;
                if (i < i1) f[u] = force(i, wd_on ? ldw<W>(p, i) : (W)0);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int64_t iw = wb + (int64_t)u * S;
                if (iw < i1) fn(iw + lane, iw + lane < i1, f[u], w);
                w.next();
            }
        }
    }
    __device__ W density(W f, W inv_s) const {
        W rel = (f < 0 ? -f : f) * inv_s + eps;
        rel = rel < (W)1e4 ? rel : (W)1e4;
        rel = rel > eps ? rel : eps;
        const W d = ipw == (W)1 ? rel : fpow(rel, ipw);
        return d < (W)1e6 ? d : (W)1e6;
    }
    // the walk of elements i, i + S, ... (L_2D only; n < 2^31 there)
    __device__ Walk2D walk(int64_t i, int S) const {
        Walk2D w{0u, 0u, 0u, 0u, C2};
        if (layout == L_2D) {
            w.row = (uint32_t)i / C2;
            w.col = (uint32_t)i % C2;
            w.dR = (uint32_t)S / C2;
            w.dC = (uint32_t)S % C2;
        }
        return w;
    }
    // fa, fb: the element's axis factors from axis_load
    __device__ W tangent(const StreamCtl<W>& c, W f, W fa, W fb) const {
        W den = c.sM;
        if (ls_on) {
            W rel = (f < 0 ? -f : f) * c.inv_s + eps;
            rel = rel < (W)100 ? rel : (W)100;
            W lm = (W)1 + ls * fsqrt(rel);
            den = den * (lm < (W)1 ? (W)1 : (lm > (W)8 ? (W)8 : lm));
        }
        W inst = 1;
        if (layout == L_1D) {
            const W r = density(f, c.inv_s) / c.gden;
            inst = fexp(kappa * flog(r > eps ? r : eps));
        } else if (layout == L_GENERIC || layout == L_2D) {
            inst = mulfac ? fa * fb : fexp(fa + fb);
        }
        if (layout != L_NONE) inst = inst < (W)0.08 ? (W)0.08 : (inst > (W)12 ? (W)12 : inst);
        W t = f * frcp(den * inst + eps);
        return t < (W)-1e4 ? (W)-1e4 : (t > (W)1e4 ? (W)1e4 : t);
    }
    __device__ W drive(const StreamCtl<W>& c, W t) const {
        W rat, bnd, root;
        shape3(t, iclip, clip, clip2, eps, rat, bnd, root);
        const W e = t - c.dc.q1;
        const W nov = ftanh(e * c.dc.nscale) * clip;
        const W core = c.dc.cr * rat + c.dc.cb * bnd + c.dc.co * root + c.dc.ct * t;
        return c.dc.cA * core + c.dc.cB + c.dc.cN * nov + c.dc.cD * e;
    }

    // ---- passes over elements i0 + tid + k S < i1 (the whole block calls them) ----
    __device__ W passA(int64_t i0, int64_t i1, int tid, int S) const {
        W a = 0;
        each<false, false>(i0, i1, tid, S, [&](W f, W, W, W) { a += f * f; });
        return a;
    }
    // Energy and instant density sums, and the axis sums (64-bit fixed-point
    // atomics).  L_2D sums are first reduced across the lanes that share a row
    // or a column, so each partial meets the atomics once:
    //   rows: cols % 64 == 0: a wave lies in one row (wave total); cols divides
    //     64: aligned groups of cols lanes (group total); otherwise a segmented
    //     sum over the wave's runs of equal rows (rows grow with the lane);
    //   cols: cols divides S: a thread's column is fixed (one register, reduced
    //     over the lanes l, l + cols, ... at the end); cols < 64: lanes l,
    //     l + cols, ... of each wave; otherwise one atomic per element.
    // Callers keep i0 and S multiples of 64 (S also of cols when cols divides
    // 64), and every lane of a wave runs the same iterations (lanes past i1 add
    // nothing), so the wave-wide reductions always see whole waves.
    // lds: S doubles (column partials of colmode 1).
    __device__ void passB(const StreamCtl<W>& c, int64_t i0, int64_t i1, int tid, int S, W& aL, W& aD,
                          double* lds) const {
        const int lane = tid & 63;
        const bool l2d = layout == L_2D;
        const int rowmode = !l2d ? 0 : (C2 % 64u == 0 ? 1 : (64u % C2 == 0 ? 2 : 3));
        const int colmode = !l2d ? 0 : ((uint32_t)S % C2 == 0 ? 1 : (C2 < 64u ? 2 : 3));
        W colacc = 0;
        const uint32_t col0 = walk(i0 + tid, S).col;
        each_wave(i0, i1, tid, S, [&](int64_t i, bool ok, W f, const Walk2D& w) {
            W d = 0;
            if (ok) {
                const W r = (f < 0 ? -f : f) * c.inv_s + eps;
                aL += flog1p(fpow(r, pw));
                d = density(f, c.inv_s);
                aD += d;
                if (layout == L_GENERIC)
                    for (int ax = 0; ax < nd; ++ax) atomicAdd(&axis_fx[R.axis_off[ax] + (i / R.stride[ax]) % R.d.shape[ax]], fx(d));
            }
            if (!l2d) return;
            if (rowmode == 1) {
                const W s = lanes_group_sum_w<W>(d, 64);   // the wave's (one row's) sum, in every lane
                if (lane == 0) atomicAdd(&axis_fx[w.row], fx(s));
            } else if (rowmode == 2) {
                const W s = lanes_group_sum_w<W>(d, (int)C2);
                if (ok && (uint32_t)lane % C2 == 0) atomicAdd(&axis_fx[w.row], fx(s));
            } else {
                // suffix sums within runs of equal keys; a run's first lane holds its total
                const uint32_t key = ok ? w.row : 0xFFFFFFFFu;
                W s = d;
                for (int off = 1; off < 64; off <<= 1) {
                    const W o = __shfl_down(s, off, 64);
                    const uint32_t ko = __shfl_down(key, off, 64);
                    if (lane + off < 64 && ko == key) s += o;
                }
                const uint32_t kp = __shfl_up(key, 1, 64);
                if (ok && (lane == 0 || kp != key)) atomicAdd(&axis_fx[w.row], fx(s));
            }
            if (colmode == 1) {
                colacc += d;
            } else if (colmode == 2) {
                W s = d;
                for (uint32_t off = C2; off < 64u; off += C2) {
                    const W o = __shfl(d, lane + (int)off, 64);
                    if ((uint32_t)lane + off < 64u) s += o;
                }
                if (ok && (uint32_t)lane < C2) atomicAdd(&axis_fx[R2 + w.col], fx(s));
            } else if (ok) {
                atomicAdd(&axis_fx[R2 + w.col], fx(d));
            }
        });
        if (colmode == 1) {
            // threads of one column: tid = col, col + cols, ... (col0 = tid % cols);
            // summed in thread order through LDS, one atomic per column
            lds[tid] = (double)colacc;   // zero for threads without elements
            __syncthreads();
            if ((uint32_t)tid < C2) {
                double s = 0.0;
                for (int k = tid; k < S; k += (int)C2) s += lds[k];
                atomicAdd(&axis_fx[R2 + col0], (unsigned long long)llrint(s * fx_scale));
            }
            __syncthreads();
        }
    }
    // Wide form, L_2D with more than 256 columns: block k of nblk takes tiles
    // k, k + nblk, ... of 32 rows x 256 columns.  Thread t owns column c0 + t
    // of a tile, so its column sum is one register and each row's sum is a
    // block reduction: one atomic per tile column and per tile row.
    // lds: 128 doubles.
    __device__ void passB_tiles(const StreamCtl<W>& c, int64_t k, int64_t nblk, int tid, W& aL, W& aD, double* lds) const {
        const int lane = tid & 63, wave = tid >> 6;
        const uint32_t ncs = (C2 + 255u) / 256u, nrs = (R2 + 31u) / 32u;
        const int64_t ntiles = (int64_t)ncs * nrs;
        for (int64_t t = k; t < ntiles; t += nblk) {
            const uint32_t r0 = (uint32_t)(t / ncs) * 32u, col = (uint32_t)(t % ncs) * 256u + (uint32_t)tid;
            const bool cok = col < C2;
            const uint32_t nr = R2 - r0 < 32u ? R2 - r0 : 32u;
            W colsum = 0;
            for (uint32_t rb = 0; rb < nr; rb += U) {
                W f[U];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const uint32_t r = rb + (uint32_t)u;
                    f[u] = 0;
                    if (cok && r < nr) {
                        const int64_t i = (int64_t)(r0 + r) * C2 + col;
                        f[u] = force(i, wd_on ? ldw<W>(p, i) : (W)0);
                    }
                }
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const uint32_t r = rb + (uint32_t)u;
                    if (r < nr) {   // uniform over the block
                        W d = 0;
                        if (cok) {
                            const W fv = f[u];
                            const W rr = (fv < 0 ? -fv : fv) * c.inv_s + eps;
                            aL += flog1p(fpow(rr, pw));
                            d = density(fv, c.inv_s);
                            aD += d;
                        }
                        colsum += d;
                        const W ws = lanes_group_sum_w<W>(d, 64);   // this wave's part of row r0 + r
                        if (lane == 0) lds[wave * 32 + (int)r] = (double)ws;
                    }
                }
            }
            if (cok) atomicAdd(&axis_fx[R2 + col], fx(colsum));
            __syncthreads();
            if ((uint32_t)tid < nr) {
                const double s = lds[tid] + lds[32 + tid] + lds[64 + tid] + lds[96 + tid];
                atomicAdd(&axis_fx[r0 + (uint32_t)tid], (unsigned long long)llrint(s * fx_scale));
            }
            __syncthreads();
        }
    }
    __device__ void passC(const StreamCtl<W>& c, int64_t i0, int64_t i1, int tid, int S, W (&m)[13]) const {
        for (int j = 0; j < 13; ++j) m[j] = 0;
        each<false, true>(i0, i1, tid, S, [&](W f, W, W fa, W fb) {
            const W t = tangent(c, f, fa, fb);
            W rat, bnd, root;
            shape3(t, iclip, clip, clip2, eps, rat, bnd, root);
            const W e = t - c.q0;
            m[0] += e; m[1] += e * e; m[2] += t; m[3] += t * t;
            m[4] += rat * rat; m[5] += bnd * bnd; m[6] += root * root;
            m[7] += rat * bnd; m[8] += rat * root; m[9] += bnd * root;
            m[10] += t * rat; m[11] += t * bnd; m[12] += t * root;
        });
    }
    __device__ W passD(const StreamCtl<W>& c, int64_t i0, int64_t i1, int tid, int S) const {
        W add = 0;
        each<false, true>(i0, i1, tid, S, [&](W f, W, W fa, W fb) {
            const W d = drive(c, tangent(c, f, fa, fb));
            add += d * d;
        });
        return add;
    }
    // param -= lr * cast(drive * gain); each element's grad and param are read
    // before this thread stores that element
    __device__ void passE(const StreamCtl<W>& c, int64_t i0, int64_t i1, int tid, int S) const {
        const W nlr = (W)update_alpha<PT>(-h.lr);
        int64_t i = i0 + tid;
        each<true, true>(i0, i1, tid, S, [&](W f, W pv, W fa, W fb) {
            const W d = drive(c, tangent(c, f, fa, fb));
            const W u = to_w<W>(from_wd<PT>((double)(d * c.gain)));
            p[i] = from_wd<PT>((double)(pv + nlr * u));
            i += S;
        });
    }

    // ---- finishes on the tensor's totals (every thread, identical results) ----
    __device__ void finA(StreamCtl<W>& c, double sff) const {
        c.fr = reservoir(c.fr, (W)sqrt((double)((W)(sff / dn) + eps)), h.reservoir_decay, c.step);
        c.scale = c.fr > eps ? c.fr : eps;
        c.inv_s = (W)1 / c.scale;
    }
    // scalar metric oscillator (cresso_v5.py:1510-1518) and the density normaliser
    __device__ void finB(StreamCtl<W>& c, double sL, double sD) const {
        const W dens_mean = (W)(sL / dn);
        const W mport = dens_mean - (W)tanh((double)c.mq);
        c.mp = c.mp * (W)fmax(0.0, 1.0 - h.metric_dt * h.metric_friction);
        c.mp = c.mp + (W)h.metric_dt * (mport - c.mq);
        c.mq = c.mq + (W)h.metric_dt * c.mp;
        c.mq = c.mq < (W)-3 ? (W)-3 : (c.mq > (W)3 ? (W)3 : c.mq);
        W metric = (W)exp((double)((W)h.metric_coupling * c.mq));
        metric = metric < (W)0.06 ? (W)0.06 : (metric > (W)16 ? (W)16 : metric);
        c.sM = c.scale * metric;
        c.gden = (W)fmax(sD / dn, (double)eps);
    }
    // kappa log(max(axis mean / gden, eps)) of axis entries a0 + tid + k S < a1
    __device__ void axis_factors(const StreamCtl<W>& c, int64_t a0, int64_t a1, int tid, int S) const {
        for (int64_t i = a0 + tid; i < a1; i += S) {
            int ax = 0;
            while (ax + 1 < nd && i >= R.axis_off[ax + 1]) ++ax;
            const unsigned long long raw = __hip_atomic_load(&axis_fx[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const W mean = (W)((double)(long long)raw / fx_scale / (dn / (double)R.d.shape[ax]));
            const W r = mean / c.gden;
            const W lf = kappa * flog(r > eps ? r : eps);
            axis_fac[i] = mulfac ? fexp(lf) : lf;
        }
    }
    __device__ void finC(StreamCtl<W>& c, const double* M) const {
        c.dc = contact_and_coefs<W>(M, dn, h, c.step, c.q0, c.imp, c.act, c.sur);
    }
    __device__ void finD(StreamCtl<W>& c, double sdd) const {
        c.de = reservoir(c.de, (W)(sdd / dn), h.reservoir_decay, c.step);
        W gain = (W)h.target_update_rms / (W)sqrt((double)(c.de + eps));
        c.gain = gain < (W)h.min_gain ? (W)h.min_gain : (gain > (W)h.max_gain ? (W)h.max_gain : gain);
    }
};

template <typename W, typename PT, typename GT>
__global__ __launch_bounds__(SR_NT) void scalar_stream_kernel(const ScalarRec* __restrict__ recs, int32_t* __restrict__ steps,
                                                              const void* const* __restrict__ grads, int32_t first,
                                                              unsigned char* table, cresso_hyper h) {
    __shared__ double red[SR_NT];   // block sums (16 x 13) and pass B's column partials
    __shared__ int s_step;
    const int tid = threadIdx.x;
    const int ri = first + blockIdx.x;
    const Stream<W, PT, GT> S(recs[ri], h, grads[ri], table);
    const int64_t n = S.n;
    StreamCtl<W> c;
    S.load_state(c);
    if (tid == 0) {
        const int s = steps[ri] + 1;
        steps[ri] = s;
        s_step = s;
    }
    // ---- pass A ----
    const W a = S.passA(0, n, tid, SR_NT);
    if (S.axes)
        for (int64_t i = tid; i < S.R.sum_dims; i += SR_NT) S.axis_fx[i] = 0ull;
    __syncthreads();
    c.step = s_step;
    {
        double v[1] = {(double)a};
        block_sum<1>(v, red);
        S.finA(c, v[0]);
    }
    // ---- pass B ----
    {
        W aL = 0, aD = 0;
        S.passB(c, 0, n, tid, SR_NT, aL, aD, red);
        double v[2] = {(double)aL, (double)aD};
        block_sum<2>(v, red);
        S.finB(c, v[0], v[1]);
    }
    if (S.axes) {
        S.axis_factors(c, 0, S.R.sum_dims, tid, SR_NT);
        __syncthreads();
    }
    // ---- pass C ----
    {
        W m[13];
        S.passC(c, 0, n, tid, SR_NT, m);
        double M[13];
        for (int j = 0; j < 13; ++j) M[j] = (double)m[j];
        block_sum<13>(M, red);
        S.finC(c, M);
    }
    // ---- pass D ----
    {
        double v[1] = {(double)S.passD(c, 0, n, tid, SR_NT)};
        block_sum<1>(v, red);
        S.finD(c, v[0]);
    }
    // ---- pass E ----
    S.passE(c, 0, n, tid, SR_NT);
    if (tid == 0) S.store_state(c);
}

// Wide form: block k of a tensor's nblk blocks owns axis entries
// [axis_slice(k), axis_slice(k + 1)) (zeroed in pass A, turned into factors by
// scalar_wide_axes).
__device__ __forceinline__ int64_t axis_slice(const ScalarRec& R, int64_t k) {
    const int64_t per = (R.sum_dims + R.nblk - 1) / R.nblk;
    const int64_t a = k * per;
    return a < R.sum_dims ? a : R.sum_dims;
}

// Wide form, pass PH (0..4 = A..E) over one chunk per block.  bmap[b] is the
// tensor of block b; the tensor's chunks are its blocks blk0 .. blk0+nblk-1.
// Block partials: part[b * 16 + v].
template <typename W, typename PT, typename GT, int PH>
__global__ __launch_bounds__(SR_WIDE_NT) void scalar_wide_pass(const ScalarRec* __restrict__ recs,
                                                               const int32_t* __restrict__ bmap,
                                                               const void* const* __restrict__ grads, unsigned char* table,
                                                               double* __restrict__ part, cresso_hyper h) {
    __shared__ double red[SR_WIDE_NT];   // block sums (4 x 13) and pass B's column or row partials
    const int tid = threadIdx.x;
    const int b = blockIdx.x;
    const int ri = bmap[b];
    const ScalarRec& R = recs[ri];
    const Stream<W, PT, GT> S(R, h, grads[ri], table);
    const int64_t i0 = (int64_t)(b - R.blk0) * SR_WIDE_CH;
    const int64_t i1 = S.n < i0 + SR_WIDE_CH ? S.n : i0 + SR_WIDE_CH;
    double* out = part + (size_t)b * 16;
    if constexpr (PH == 0) {
        if (S.axes) {
            // this block's slice of the axis sums starts at zero (pass B adds to them)
            const int64_t a0 = axis_slice(R, b - R.blk0), a1 = axis_slice(R, b - R.blk0 + 1);
            for (int64_t a = a0 + tid; a < a1; a += SR_WIDE_NT) S.axis_fx[a] = 0ull;
        }
        double v[1] = {(double)S.passA(i0, i1, tid, SR_WIDE_NT)};
        block_sum<1>(v, red);
        if (tid == 0) out[0] = v[0];
        return;
    } else {
        const StreamCtl<W> c = *reinterpret_cast<const StreamCtl<W>*>(table + R.ctl_off);
        if constexpr (PH == 1) {
            W aL = 0, aD = 0;
            if (S.layout == L_2D && S.C2 > 256u)
                S.passB_tiles(c, b - R.blk0, R.nblk, tid, aL, aD, red);
            else
                S.passB(c, i0, i1, tid, SR_WIDE_NT, aL, aD, red);
            __syncthreads();   // red is reused by the block sum
            double v[2] = {(double)aL, (double)aD};
            block_sum<2>(v, red);
            if (tid == 0) {
                out[0] = v[0];
                out[1] = v[1];
            }
        } else if constexpr (PH == 2) {
            W m[13];
            S.passC(c, i0, i1, tid, SR_WIDE_NT, m);
            double M[13];
            for (int j = 0; j < 13; ++j) M[j] = (double)m[j];
            block_sum<13>(M, red);
            if (tid == 0)
                for (int j = 0; j < 13; ++j) out[j] = M[j];
        } else if constexpr (PH == 3) {
            double v[1] = {(double)S.passD(c, i0, i1, tid, SR_WIDE_NT)};
            block_sum<1>(v, red);
            if (tid == 0) out[0] = v[0];
        } else {
            S.passE(c, i0, i1, tid, SR_WIDE_NT);
        }
    }
}

// Wide form, finish after pass PH (0..3): one workgroup per tensor sums the
// tensor's block partials in block order and advances its StreamCtl.
template <typename W, typename PT, typename GT, int PH>
__global__ __launch_bounds__(SR_WIDE_NT) void scalar_wide_fin(const ScalarRec* __restrict__ recs, int32_t* __restrict__ steps,
                                                              const void* const* __restrict__ grads, int32_t first,
                                                              unsigned char* table, const double* __restrict__ part,
                                                              cresso_hyper h) {
    constexpr int V = PH == 1 ? 2 : (PH == 2 ? 13 : 1);
    __shared__ double red[(SR_WIDE_NT / 64) * V];
    __shared__ int s_step;
    const int tid = threadIdx.x;
    const int ri = first + blockIdx.x;
    const ScalarRec& R = recs[ri];
    const Stream<W, PT, GT> S(R, h, grads[ri], table);
    StreamCtl<W>* cp = reinterpret_cast<StreamCtl<W>*>(table + R.ctl_off);
    StreamCtl<W> c;
    if (PH == 0) {
        S.load_state(c);
        if (tid == 0) {
            const int s = steps[ri] + 1;
            steps[ri] = s;
            s_step = s;
        }
    } else {
        c = *cp;
    }
    double v[V];
    for (int j = 0; j < V; ++j) v[j] = 0.0;
    for (int b = tid; b < R.nblk; b += SR_WIDE_NT)
        for (int j = 0; j < V; ++j) v[j] += part[(size_t)(R.blk0 + b) * 16 + j];
    block_sum<V>(v, red);   // its barriers also publish s_step
    if (PH == 0) {
        c.step = s_step;
        S.finA(c, v[0]);
    } else if (PH == 1) {
        S.finB(c, v[0], v[1]);
    } else if (PH == 2) {
        S.finC(c, v);
    } else {
        S.finD(c, v[0]);
        if (tid == 0) S.store_state(c);
    }
    if (tid == 0) *cp = c;
}

// Wide form, after finish B: block k of each tensor turns its slice of the
// fixed-point axis sums into factors.
template <typename W, typename PT, typename GT>
__global__ __launch_bounds__(SR_WIDE_NT) void scalar_wide_axes(const ScalarRec* __restrict__ recs,
                                                               const int32_t* __restrict__ bmap,
                                                               const void* const* __restrict__ grads, unsigned char* table,
                                                               cresso_hyper h) {
    const int b = blockIdx.x;
    const int ri = bmap[b];
    const ScalarRec& R = recs[ri];
    if (R.layout != L_GENERIC && R.layout != L_2D) return;
    const Stream<W, PT, GT> S(R, h, grads[ri], table);
    const StreamCtl<W> c = *reinterpret_cast<const StreamCtl<W>*>(table + R.ctl_off);
    S.axis_factors(c, axis_slice(R, b - R.blk0), axis_slice(R, b - R.blk0 + 1), threadIdx.x, SR_WIDE_NT);
}

// ---------------------------------------------------------------------------
// micro-field kernel: the dense per-coordinate route of small tensors
// (micro_field_max_size > 0), cresso_v5.py:1355-1432 (PyTorch-only in the
// reference).  One workgroup per tensor, five streaming passes:
//   A: sum f^2                          -> force-RMS reservoir, scale s
//   B: energy field e <- EMA of rel^p (written back), sum e; instant density,
//      its sum and its per-axis sums    -> metric normaliser, instant metric
//   C: t; refractory and impulse fields (written back); sums of err^2, rat^2,
//      rat*bnd, bnd^2, pred^2, t^2      -> surprise reservoir, shaped-force
//                                          RMS and the three RMS normalisers
//   D: drive; sum drive^2               -> drive-energy reservoir, gain
//   E: param -= lr * cast(drive * gain)
// Per-axis density sums are 64-bit fixed-point integers (order-independent,
// so the result does not depend on atomic order) in LDS when they fit, else
// in the tensor's table scratch; the fixed-point scale comes from an upper
// bound of the largest density, sqrt(sum f^2) >= max |f|.
// ---------------------------------------------------------------------------
constexpr int64_t MF_LDS_AXES = 4096;   // axis-sum entries held in LDS

template <typename W, typename PT, typename GT>
__global__ __launch_bounds__(SR_NT) void micro_kernel(const ScalarRec* __restrict__ recs, int32_t* __restrict__ steps,
                                                      const void* const* __restrict__ grads, int32_t first,
                                                      unsigned char* table, cresso_hyper h) {
    __shared__ double red[16 * 6];
    __shared__ unsigned long long s_ax[MF_LDS_AXES];
    __shared__ int s_step;
    const int tid = threadIdx.x;
    const int ri = first + blockIdx.x;
    const ScalarRec& R = recs[ri];
    const int64_t n = R.d.numel;
    const int nd = R.d.ndim;
    const int layout = R.layout;
    const W eps = (W)h.eps;
    W* __restrict__ en = reinterpret_cast<W*>(R.d.state[0]);   // micro_energy
    W* __restrict__ im = reinterpret_cast<W*>(R.d.state[1]);   // micro_impulse
    W* __restrict__ rf = reinterpret_cast<W*>(R.d.state[2]);   // micro_refractory
    W* const st_fr = reinterpret_cast<W*>(R.d.state[3]);
    W* const st_de = reinterpret_cast<W*>(R.d.state[4]);
    W* const st_su = reinterpret_cast<W*>(R.d.state[5]);
    W fr = *st_fr, de = *st_de, sur = *st_su;
    if (tid == 0) {
        const int s = steps[ri] + 1;
        steps[ri] = s;
        s_step = s;
    }
    const GT* __restrict__ g = reinterpret_cast<const GT*>(grads[ri]);
    PT* __restrict__ p = reinterpret_cast<PT*>(R.d.param);
    const bool wd_on = h.weight_decay != 0.0;
    const W wd = (W)h.weight_decay;
    const bool neg = h.maximize != 0;
    auto force = [&](int64_t i) -> W {
        W f = ldw<W>(g, i);
        if (neg) f = -f;
        if (wd_on) f = f + wd * ldw<W>(p, i);
        return f;
    };
    unsigned long long* ax = R.sum_dims <= MF_LDS_AXES ? s_ax : reinterpret_cast<unsigned long long*>(table + R.scratch_off);
    const double dn = (double)n;

    // ---- pass A ----
    W a = 0;
    for (int64_t i = tid; i < n; i += SR_NT) {
        const W f = force(i);
        a += f * f;
    }
    if (layout == L_GENERIC) {
        for (int64_t k = tid; k < R.sum_dims; k += SR_NT) ax[k] = 0ull;
        __threadfence();   // zeros reach L2 before any wave's atomics
    }
    __syncthreads();
    const int step = s_step;
    double sumsq;
    {
        double v[1] = {(double)a};
        block_sum<1>(v, red);
        sumsq = v[0];
        fr = reservoir(fr, (W)sqrt((double)((W)(v[0] / dn) + eps)), h.reservoir_decay, step);
    }
    const W scale = fr > eps ? fr : eps;

    // ---- pass B ----
    const W pw = (W)h.energy_power;
    const W md = (W)h.micro_decay, md1 = (W)(1.0 - h.micro_decay);
    const double ipw_d = fmax(h.instant_metric_power, 0.25);
    const W ipw = (W)ipw_d;
    // cresso_v5.py:1390-1392: the instant-metric coupling is capped at 0.35
    const W kappa = nd > 0 ? (W)(fmin(0.35, h.instant_metric_coupling) / ((double)nd * ipw_d)) : (W)0;
    auto rel_of = [&](W f) -> W {
        const W r = (f < 0 ? -f : f) / scale + eps;
        return r < (W)1e4 ? r : (W)1e4;
    };
    auto density = [&](W rel) -> W {   // cresso_v5.py:243-262
        const W r = rel > eps ? rel : eps;
        const W d = ipw == (W)1 ? r : fpow(r, ipw);
        return d < (W)1e6 ? d : (W)1e6;
    };
    int64_t maxcnt = 1;
    for (int k = 0; k < nd; ++k) maxcnt = n / R.d.shape[k] > maxcnt ? n / R.d.shape[k] : maxcnt;
    double fx_scale = 1.0;
    if (layout == L_GENERIC) {
        // every |f| <= sqrt(sum f^2), so every density <= dens_b: the fixed-point
        // axis sums stay below 2^62
        double rb = sqrt(sumsq) / (double)scale + (double)eps;
        rb = fmax(fmin(rb, 1e4), (double)eps);
        const double dens_b = fmin(pow(rb, ipw_d), 1e6) * (1.0 + 1e-6);
        const double lg = log2(fmax(dens_b, 1e-300) * (double)maxcnt);
        int fb = isfinite(lg) ? (int)floor(62.0 - lg) : 0;
        fb = fb < 0 ? 0 : (fb > 900 ? 900 : fb);
        fx_scale = ldexp(1.0, fb);
    }
    W aE = 0, aD = 0;
    for (int64_t i = tid; i < n; i += SR_NT) {
        const W rel = rel_of(force(i));
        const W src = pw == (W)1 ? rel : fpow(rel, pw);
        const W e = step <= 1 ? src : en[i] * md + md1 * src;
        en[i] = e;
        aE += e;
        if (layout != L_NONE) {
            const W d = density(rel);
            aD += d;
            if (layout == L_GENERIC) {
                const unsigned long long v = (unsigned long long)llrint((double)d * fx_scale);
                for (int k = 0; k < nd; ++k) atomicAdd(&ax[R.axis_off[k] + (i / R.stride[k]) % R.d.shape[k]], v);
            }
        }
    }
    if (layout == L_GENERIC) __threadfence();
    W emean, gden;
    {
        double v[2] = {(double)aE, (double)aD};
        block_sum<2>(v, red);
        emean = (W)(v[0] / dn);
        emean = emean > eps ? emean : eps;
        gden = (W)(v[1] / dn);
        gden = gden > eps ? gden : eps;
    }
    // per-axis log factors kappa * log(max(marginal mean / mean, eps)), in
    // place; agent-scope atomic accesses keep the table-scratch case off the L1
    double* axf = reinterpret_cast<double*>(ax);
    if (layout == L_GENERIC) {
        for (int64_t k = tid; k < R.sum_dims; k += SR_NT) {
            int a_ = 0;
            while (a_ + 1 < nd && k >= R.axis_off[a_ + 1]) ++a_;
            const unsigned long long raw = __hip_atomic_load(&ax[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const W mean = (W)((double)(long long)raw / fx_scale / (dn / (double)R.d.shape[a_]));
            const W r = mean / gden;
            __hip_atomic_store(&axf[k], (double)(kappa * flog(r > eps ? r : eps)), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
        __threadfence();
        __syncthreads();
    }
    const bool metric_on = h.hash_metric_coupling != 0.0;
    const W mpow = (W)(h.hash_metric_coupling / fmax(0.25, h.energy_power));
    auto tangent = [&](W f, int64_t i) -> W {
        W metric = 1;
        if (metric_on) {
            metric = fpow(en[i] / emean, mpow);
            metric = metric < (W)0.08 ? (W)0.08 : (metric > (W)12 ? (W)12 : metric);
        }
        W inst = 1;
        if (layout == L_1D) {
            const W r = density(rel_of(f)) / gden;
            inst = fexp(kappa * flog(r > eps ? r : eps));
        } else if (layout == L_GENERIC) {
            W s = 0;
            for (int k = 0; k < nd; ++k)
                s += (W)__hip_atomic_load(&axf[R.axis_off[k] + (i / R.stride[k]) % R.d.shape[k]], __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
            inst = fexp(s);
        }
        if (layout != L_NONE) inst = inst < (W)0.08 ? (W)0.08 : (inst > (W)12 ? (W)12 : inst);
        const W t = f / (scale * metric * inst + eps);
        return t < (W)-1e4 ? (W)-1e4 : (t > (W)1e4 ? (W)1e4 : t);
    };
    const W clip = (W)h.drive_clip, iclip = (W)1 / clip, clip2 = clip * clip;

    // ---- pass C ----
    const W rd = (W)h.refractory_decay, rd1 = (W)(1.0 - h.refractory_decay), rg = (W)h.refractory_gain;
    const W idk = (W)h.micro_impulse_decay, idk1 = (W)(1.0 - h.micro_impulse_decay);
    W m[6] = {0, 0, 0, 0, 0, 0};
    for (int64_t i = tid; i < n; i += SR_NT) {
        const W t = tangent(force(i), i);
        const W r = rf[i] * rd + rd1 * (t < 0 ? -t : t);
        rf[i] = r;
        const W gate = (W)1 / ((W)1 + rg * r);
        const W pr = im[i] * idk + idk1 * (t * gate);
        im[i] = pr;
        const W err = t - pr;
        W rat, bnd, root;
        shape3(t, iclip, clip, clip2, eps, rat, bnd, root);
        m[0] += err * err; m[1] += rat * rat; m[2] += rat * bnd;
        m[3] += bnd * bnd; m[4] += pr * pr; m[5] += t * t;
    }
    double M[6];
    for (int j = 0; j < 6; ++j) M[j] = (double)m[j];
    block_sum<6>(M, red);
    // cresso_v5.py:1406-1425 with every mean(x^2) taken from the sums above;
    // mean(shaped^2) expands over rat^2, rat*bnd and bnd^2.
    const W sur_now = (W)sqrt((double)((W)(M[0] / dn) + eps));
    sur = reservoir(sur, sur_now, h.surprise_decay, step);
    const W spike = (W)h.spike_mix / ((W)1 + sur);
    const W a1 = (W)1 - spike;
    const W ssq = (W)(((double)(a1 * a1) * M[1] + 2.0 * (double)(a1 * spike) * M[2] + (double)(spike * spike) * M[3]) / dn);
    const W target = (W)sqrt((double)(ssq + eps));
    const W rms_p = (W)sqrt((double)((W)(M[4] / dn) + eps));
    const W rms_t = (W)sqrt((double)((W)(M[5] / dn) + eps));
    const W kp = target / (rms_p > eps ? rms_p : eps);
    const W kt = target / (rms_t > eps ? rms_t : eps);
    const W ke = target / (sur_now > eps ? sur_now : eps);
    const W dmix = (W)h.direct_force_mix / ((W)1 + (W)0.35 * sur);
    const W mmix = (W)h.micro_drive_mix / ((W)1 + (W)0.25 * sur);
    const W rmix = (W)h.residual_feedback_mix / ((W)1 + sur);
    W cw = (W)1 - dmix - (W)0.5 * mmix;
    cw = cw < (W)0 ? (W)0 : (cw > (W)1 ? (W)1 : cw);
    const W cR = cw * a1, cBn = cw * spike, cT = dmix * kt, cP = mmix * kp, cE = rmix * ke;
    auto drive = [&](W t, W pr) -> W {
        W rat, bnd, root;
        shape3(t, iclip, clip, clip2, eps, rat, bnd, root);
        return cR * rat + cBn * bnd + cT * t + cP * pr + cE * (t - pr);
    };

    // ---- pass D ----
    W add = 0;
    for (int64_t i = tid; i < n; i += SR_NT) {
        const W d = drive(tangent(force(i), i), im[i]);
        add += d * d;
    }
    {
        double v[1] = {(double)add};
        block_sum<1>(v, red);
        de = reservoir(de, (W)(v[0] / dn), h.reservoir_decay, step);
    }
    W gain = (W)h.target_update_rms / (W)sqrt((double)(de + eps));
    gain = gain < (W)h.min_gain ? (W)h.min_gain : (gain > (W)h.max_gain ? (W)h.max_gain : gain);

    // ---- pass E ---- (force is recomputed before any param store of this thread)
    const W nlr = (W)update_alpha<PT>(-h.lr);
    for (int64_t i = tid; i < n; i += SR_NT) {
        const W d = drive(tangent(force(i), i), im[i]);
        const W u = to_w<W>(from_wd<PT>((double)(d * gain)));
        p[i] = from_wd<PT>((double)(ldw<W>(p, i) + nlr * u));
    }
    if (tid == 0) {
        *st_fr = fr; *st_de = de; *st_su = sur;
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
bool is_pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

struct Variant {
    int pt, gt, kind;   // kind: 0 stream, 1 resident (row-group or column-block layout), 2 wide stream, 3 micro field
    bool full;          // resident with numel == SR_RESIDENT_MAX: eligible for the FAST kernel
    bool operator==(const Variant& o) const { return pt == o.pt && gt == o.gt && kind == o.kind && full == o.full; }
};

// The FAST resident kernel skips the per-element work of these options.
bool fast_hyper(const cresso_hyper& h) {
    return h.weight_decay == 0.0 && h.local_sharpness == 0.0 && (float)fmax(h.instant_metric_power, 0.25) == 1.0f;
}

int dtype_bytes(int t) { return t == CRESSO_F64 ? 8 : (t == CRESSO_F32 ? 4 : 2); }

// Fills r (except scratch_off) and returns the generic scratch bytes needed.
int32_t plan_desc(const cresso_scalar_desc& d, const cresso_hyper& h, ScalarRec& r, Variant& v, size_t& lds,
                  size_t& scratch) {
    if (d.ndim < 0 || d.ndim > 8) return fail(CRESSO_E_INVALID, "scalar route: ndim %d outside 0..8", d.ndim);
    int64_t n = 1;
    for (int a = 0; a < d.ndim; ++a) {
        if (d.shape[a] <= 0)
            return fail(CRESSO_E_INVALID, "scalar route: shape[%d]=%lld must be positive", a, (long long)d.shape[a]);
        n *= d.shape[a];
    }
    if (n != d.numel)
        return fail(CRESSO_E_INVALID, "scalar route: numel %lld != product of shape %lld", (long long)d.numel, (long long)n);
    if (!d.param || !d.grad) return fail(CRESSO_E_INVALID, "scalar route: null param or grad pointer");
    if (d.route != 0 && d.route != 1) return fail(CRESSO_E_INVALID, "scalar route: unknown route %d", d.route);
    const int nstate = d.route == 1 ? 7 : 8;
    for (int i = 0; i < nstate; ++i)
        if (!d.state[i]) return fail(CRESSO_E_INVALID, "scalar route: null state pointer %d", i);
    if (d.route == 1 && d.ndim == 0) return fail(CRESSO_E_INVALID, "micro route: 0-dim tensors use the scalar route");
    auto okdt = [](int t) { return t == CRESSO_F32 || t == CRESSO_F16 || t == CRESSO_BF16 || t == CRESSO_F64; };
    if (!okdt(d.param_dtype) || !okdt(d.grad_dtype)) return fail(CRESSO_E_INVALID, "scalar route: unknown dtype code");
    if ((d.param_dtype == CRESSO_F64) != (d.grad_dtype == CRESSO_F64))
        return fail(CRESSO_E_UNSUPPORTED, "scalar route: float64 params need float64 grads");
    std::memset(&r, 0, sizeof(r));
    r.d = d;
    lds = 0;
    scratch = 0;
    const bool aligned = ((uintptr_t)d.param % (uintptr_t)(4 * dtype_bytes(d.param_dtype))) == 0 &&
                         ((uintptr_t)d.grad % (uintptr_t)(4 * dtype_bytes(d.grad_dtype))) == 0;
    const bool same = d.param_dtype == d.grad_dtype;
    if (d.route == 1) {
        // micro field: streaming kernel; axis sums in LDS up to MF_LDS_AXES entries
        if (h.instant_metric_coupling == 0.0 || n <= 1) {
            r.layout = L_NONE;
        } else if (d.ndim == 1) {
            r.layout = L_1D;
        } else {
            int64_t sum = 0, st = 1;
            for (int a = d.ndim - 1; a >= 0; --a) {
                r.stride[a] = st;
                st *= d.shape[a];
            }
            for (int a = 0; a < d.ndim; ++a) {
                r.axis_off[a] = sum;
                sum += d.shape[a];
            }
            r.layout = L_GENERIC;
            r.sum_dims = sum;
            if (sum > MF_LDS_AXES) scratch = ((size_t)sum * sizeof(unsigned long long) + 255) & ~(size_t)255;
        }
        v = Variant{d.param_dtype, d.grad_dtype, 3, false};
        return CRESSO_OK;
    }
    int kind = 0;
    if (h.instant_metric_coupling == 0.0 || d.ndim == 0 || n <= 1) {
        r.layout = L_NONE;
    } else if (d.ndim == 1) {
        r.layout = L_1D;
    } else {
        const int64_t C0 = d.ndim == 2 ? d.shape[1] : 0;
        const bool res_ok = d.ndim == 2 && same && d.param_dtype != CRESSO_F64 && aligned && n <= SR_RESIDENT_MAX && C0 % 4 == 0;
        // resident layouts: LDS slots first, then row factors / column partials
        const size_t rg_lds = C0 > 0 ? SR_XLDS + ((sizeof(float) * (size_t)d.shape[0] + 15) & ~(size_t)15) +
                                           sizeof(double) * 16 * (size_t)C0 + sizeof(float) * (size_t)C0
                                     : 0;
        if (res_ok && is_pow2(C0 / 4) && C0 / 4 <= 64 && rg_lds <= SR_LDS_MAX) {
            r.layout = L_ROWGROUP;
            r.group = (int32_t)(C0 / 4);
            r.rows = d.shape[0];
            r.cols = C0;
            kind = 1;
            lds = rg_lds;
        } else if (res_ok && C0 == (int64_t)SR_NT * 4) {
            r.layout = L_COLBLOCK;
            r.rows = d.shape[0];
            r.cols = C0;
            kind = 1;
            lds = SR_XLDS + sizeof(float) * SR_SLOTS;
        } else {
            int64_t sum = 0, maxcnt = 1, st = 1;
            for (int a = d.ndim - 1; a >= 0; --a) {
                r.stride[a] = st;
                st *= d.shape[a];
            }
            for (int a = 0; a < d.ndim; ++a) {
                r.axis_off[a] = sum;
                sum += d.shape[a];
                maxcnt = std::max<int64_t>(maxcnt, n / d.shape[a]);
            }
            // 2-D: row/column coordinates advanced incrementally and the axis
            // sums pre-aggregated per wave, lane group or thread (L_2D)
            r.layout = d.ndim == 2 && n < ((int64_t)1 << 31) ? L_2D : L_GENERIC;
            r.rows = d.shape[0];
            r.cols = d.ndim == 2 ? d.shape[1] : 0;
            r.sum_dims = sum;
            // density <= 1e6 per element: every fixed-point axis sum stays below 2^62
            r.frac_bits = (int32_t)std::floor(62.0 - std::log2(1.0e6 * (double)maxcnt));
            scratch = (size_t)sum * (sizeof(unsigned long long) + sizeof(double));   // fixed-point sums, factors in W
            scratch = (scratch + 255) & ~(size_t)255;
        }
    }
    if (kind == 0 && n >= SR_WIDE_MIN) kind = 2;
    r.resident = kind == 1;
    v = Variant{d.param_dtype, d.grad_dtype, kind, kind == 1 && n == SR_RESIDENT_MAX};
    return CRESSO_OK;
}

// The resident kernels use more than 64 KiB of dynamic LDS: raise the
// function's limit once (thread-safe static initialisation).
template <typename PT, typename GT, bool FAST>
hipError_t allow_resident_lds() {
    static const hipError_t e =
        hipFuncSetAttribute(reinterpret_cast<const void*>(&scalar_resident_kernel<PT, GT, FAST>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)SR_LDS_MAX);
    return e;
}

template <typename PT, typename GT, bool FAST>
hipError_t launch_resident_v(const ScalarRec* recs, int32_t* steps, const void* const* grads, int32_t first, int32_t cnt,
                             size_t lds, const cresso_hyper& h, hipStream_t s) {
    const hipError_t e = allow_resident_lds<PT, GT, FAST>();
    if (e != hipSuccess) return e;
    // one resident workgroup per CU: a launch of more workgroups than CUs runs
    // in rounds, staggered (see Stagger); 35 us is about 40 % of one 64 Ki-element
    // tensor's time, the best of the offsets measured on MI355X
    Stagger sg{0, 0, 0u};
    int dev = 0, cus = 0;
    if (FAST && hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 1 && cnt > cus)
        sg = Stagger{cus / 2, cus, 3500u};
    hipLaunchKernelGGL((scalar_resident_kernel<PT, GT, FAST>), dim3(cnt), dim3(SR_NT), lds, s, recs, steps, grads, first, h,
                       sg);
    return hipGetLastError();
}

template <typename PT, typename GT>
hipError_t launch_resident(bool fast, const ScalarRec* recs, int32_t* steps, const void* const* grads, int32_t first,
                           int32_t cnt, size_t lds, const cresso_hyper& h, hipStream_t s) {
    if (lds > SR_LDS_MAX) return hipErrorInvalidValue;
    return fast ? launch_resident_v<PT, GT, true>(recs, steps, grads, first, cnt, lds, h, s)
                : launch_resident_v<PT, GT, false>(recs, steps, grads, first, cnt, lds, h, s);
}

template <typename W, typename PT, typename GT>
hipError_t launch_stream(bool micro, const ScalarRec* recs, int32_t* steps, const void* const* grads, int32_t first,
                         int32_t cnt, unsigned char* table, const cresso_hyper& h, hipStream_t s) {
    if (micro)
        hipLaunchKernelGGL((micro_kernel<W, PT, GT>), dim3(cnt), dim3(SR_NT), 0, s, recs, steps, grads, first, table, h);
    else
        hipLaunchKernelGGL((scalar_stream_kernel<W, PT, GT>), dim3(cnt), dim3(SR_NT), 0, s, recs, steps, grads, first,
                           table, h);
    return hipGetLastError();
}

// The wide form's ten launches: pass A, finish A, pass B, finish B, axis
// factors, pass C, finish C, pass D, finish D, pass E.
template <typename W, typename PT, typename GT>
hipError_t launch_wide(const ScalarRec* recs, int32_t* steps, const void* const* grads, int32_t first, int32_t cnt,
                       int32_t nblocks, const int32_t* bmap, unsigned char* table, double* part, const cresso_hyper& h,
                       hipStream_t s) {
    const dim3 pb(SR_WIDE_NT);
    hipLaunchKernelGGL((scalar_wide_pass<W, PT, GT, 0>), dim3(nblocks), pb, 0, s, recs, bmap, grads, table, part, h);
    hipLaunchKernelGGL((scalar_wide_fin<W, PT, GT, 0>), dim3(cnt), pb, 0, s, recs, steps, grads, first, table, part, h);
    hipLaunchKernelGGL((scalar_wide_pass<W, PT, GT, 1>), dim3(nblocks), pb, 0, s, recs, bmap, grads, table, part, h);
    hipLaunchKernelGGL((scalar_wide_fin<W, PT, GT, 1>), dim3(cnt), pb, 0, s, recs, steps, grads, first, table, part, h);
    hipLaunchKernelGGL((scalar_wide_axes<W, PT, GT>), dim3(nblocks), pb, 0, s, recs, bmap, grads, table, h);
    hipLaunchKernelGGL((scalar_wide_pass<W, PT, GT, 2>), dim3(nblocks), pb, 0, s, recs, bmap, grads, table, part, h);
    hipLaunchKernelGGL((scalar_wide_fin<W, PT, GT, 2>), dim3(cnt), pb, 0, s, recs, steps, grads, first, table, part, h);
    hipLaunchKernelGGL((scalar_wide_pass<W, PT, GT, 3>), dim3(nblocks), pb, 0, s, recs, bmap, grads, table, part, h);
    hipLaunchKernelGGL((scalar_wide_fin<W, PT, GT, 3>), dim3(cnt), pb, 0, s, recs, steps, grads, first, table, part, h);
    hipLaunchKernelGGL((scalar_wide_pass<W, PT, GT, 4>), dim3(nblocks), pb, 0, s, recs, bmap, grads, table, part, h);
    return hipGetLastError();
}

// Launch geometry of a wide group: its block count and block map (in the table).
struct WideGeom {
    int32_t nblocks;
    const int32_t* bmap;
    double* part;
};

hipError_t dispatch(const Variant& v, const ScalarRec* recs, int32_t* steps, const void* const* grads, int32_t first,
                    int32_t cnt, size_t lds, unsigned char* table, const WideGeom& wg, const cresso_hyper& h,
                    hipStream_t s) {
    if (v.kind == 1) {
        const bool fast = v.full && fast_hyper(h);
        if (v.pt == CRESSO_F32) return launch_resident<float, float>(fast, recs, steps, grads, first, cnt, lds, h, s);
        if (v.pt == CRESSO_BF16)
            return launch_resident<__hip_bfloat16, __hip_bfloat16>(fast, recs, steps, grads, first, cnt, lds, h, s);
        if (v.pt == CRESSO_F16) return launch_resident<__half, __half>(fast, recs, steps, grads, first, cnt, lds, h, s);
        return hipErrorInvalidValue;
    }
#define CRESSO_SR_CASE(PC, GC, W, PT, GT)                                                                            \
    if (v.pt == PC && v.gt == GC)                                                                                    \
        return v.kind == 2 ? launch_wide<W, PT, GT>(recs, steps, grads, first, cnt, wg.nblocks, wg.bmap, table, wg.part, h, s) \
                           : launch_stream<W, PT, GT>(v.kind == 3, recs, steps, grads, first, cnt, table, h, s);
    CRESSO_SR_CASE(CRESSO_F32, CRESSO_F32, float, float, float)
    CRESSO_SR_CASE(CRESSO_BF16, CRESSO_BF16, float, __hip_bfloat16, __hip_bfloat16)
    CRESSO_SR_CASE(CRESSO_F16, CRESSO_F16, float, __half, __half)
    CRESSO_SR_CASE(CRESSO_F64, CRESSO_F64, double, double, double)
    CRESSO_SR_CASE(CRESSO_BF16, CRESSO_F32, float, __hip_bfloat16, float)
    CRESSO_SR_CASE(CRESSO_F16, CRESSO_F32, float, __half, float)
    CRESSO_SR_CASE(CRESSO_F32, CRESSO_BF16, float, float, __hip_bfloat16)
    CRESSO_SR_CASE(CRESSO_F32, CRESSO_F16, float, float, __half)
#undef CRESSO_SR_CASE
    return hipErrorInvalidValue;
}

}  // namespace
}  // namespace cresso

// Opaque plan: validated, grouped descriptor table plus pinned staging for
// the per-step grad pointers (double-buffered, guarded by events).
struct cresso_scalar_plan {
    std::vector<cresso::ScalarRec> recs;     // grouped order
    std::vector<int32_t> steps;               // grouped order
    std::vector<int32_t> order;               // grouped index -> caller index
    struct Group {
        cresso::Variant v;
        int32_t first, count;
        size_t lds;
        int32_t nblocks;   // wide form: blocks per pass launch
        size_t map_off;    // wide form: table offset of the block map
    };
    std::vector<Group> groups;
    std::vector<int32_t> bmap;                // wide form: block -> tensor, every wide group in turn
    size_t steps_off = 0, grads_off = 0, bmap_off = 0, part_off = 0, total = 0;
    bool no_instant = false;                  // instant_metric_coupling == 0 at planning time
    // per-step grad pointers in pinned, device-mapped, coherent host memory:
    // the kernels read them there (no copy to the table, whose separate
    // small transfer stalled the stream for tens of µs); double-buffered, ev[k]
    // recorded after the last kernels that read staging[k]
    const void** staging[2] = {nullptr, nullptr};
    const void* const* dstaging[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    int flip = 0;
    int cur = -1;   // staging buffer the last step's kernels read (-1: the table)
    // grad pointers the table holds (grouped order), to skip an unchanged upload
    std::vector<const void*> table_grads;
    const void* table_ptr = nullptr;
};

namespace cresso {
namespace {

int32_t build_plan(const cresso_scalar_desc* descs, int32_t count, const cresso_hyper& h, cresso_scalar_plan& P) {
    std::vector<ScalarRec> recs((size_t)count);
    std::vector<Variant> var((size_t)count);
    std::vector<size_t> lds((size_t)count), scr((size_t)count);
    for (int32_t i = 0; i < count; ++i) {
        int32_t rc = plan_desc(descs[i], h, recs[(size_t)i], var[(size_t)i], lds[(size_t)i], scr[(size_t)i]);
        if (rc != CRESSO_OK) return rc;
    }
    // Mid-size streaming tensors (SR_WIDE_MID .. SR_RESIDENT_MAX elements) take
    // the wide form too when they are too few to fill the GPU one workgroup each.
    int32_t mid = 0;
    for (int32_t i = 0; i < count; ++i)
        mid += var[(size_t)i].kind == 0 && descs[i].numel >= SR_WIDE_MID;
    if (mid > 0 && mid < SR_WIDE_FILL)
        for (int32_t i = 0; i < count; ++i)
            if (var[(size_t)i].kind == 0 && descs[i].numel >= SR_WIDE_MID) var[(size_t)i].kind = 2;
    std::vector<Variant> keys;
    for (const Variant& v : var)
        if (std::find(keys.begin(), keys.end(), v) == keys.end()) keys.push_back(v);
    std::vector<int32_t> key((size_t)count);
    for (int32_t i = 0; i < count; ++i)
        key[(size_t)i] = (int32_t)(std::find(keys.begin(), keys.end(), var[(size_t)i]) - keys.begin());
    P.order.resize((size_t)count);
    for (int32_t i = 0; i < count; ++i) P.order[(size_t)i] = i;
    std::stable_sort(P.order.begin(), P.order.end(), [&](int32_t a, int32_t b) { return key[(size_t)a] < key[(size_t)b]; });
    const size_t recs_bytes = (sizeof(ScalarRec) * (size_t)count + 255) & ~(size_t)255;
    P.steps_off = recs_bytes;
    P.grads_off = P.steps_off + ((sizeof(int32_t) * (size_t)count + 255) & ~(size_t)255);
    size_t off = P.grads_off + ((sizeof(void*) * (size_t)count + 255) & ~(size_t)255);
    P.recs.resize((size_t)count);
    P.steps.resize((size_t)count);
    P.groups.clear();
    P.bmap.clear();
    int32_t max_blocks = 0;
    for (int32_t j = 0; j < count; ++j) {
        const int32_t i = P.order[(size_t)j];
        ScalarRec& r = P.recs[(size_t)j];
        r = recs[(size_t)i];
        r.scratch_off = (int64_t)off;
        off += scr[(size_t)i];
        P.steps[(size_t)j] = descs[i].step;
        if (P.groups.empty() || !(P.groups.back().v == var[(size_t)i]))
            P.groups.push_back({var[(size_t)i], j, 0, 0, 0, 0});
        auto& G = P.groups.back();
        G.count += 1;
        G.lds = std::max(G.lds, lds[(size_t)i]);
        if (G.v.kind == 2) {
            r.ctl_off = (int64_t)off;
            off += SR_CTL_BYTES;
            const int64_t nb = (r.d.numel + SR_WIDE_CH - 1) / SR_WIDE_CH;
            if (nb > (int64_t)INT32_MAX - G.nblocks)
                return fail(CRESSO_E_UNSUPPORTED, "scalar route: wide group of more than 2^31 blocks");
            if (G.nblocks == 0) G.map_off = sizeof(int32_t) * P.bmap.size();   // relative until placed below
            r.blk0 = G.nblocks;
            r.nblk = (int32_t)nb;
            G.nblocks += (int32_t)nb;
            P.bmap.insert(P.bmap.end(), (size_t)nb, j);
            max_blocks = std::max(max_blocks, G.nblocks);
        }
    }
    // block maps, then one partials area shared by the wide groups (they run in turn)
    P.bmap_off = off;
    off += (sizeof(int32_t) * P.bmap.size() + 255) & ~(size_t)255;
    for (auto& G : P.groups)
        if (G.v.kind == 2) G.map_off += P.bmap_off;
    P.part_off = off;
    off += sizeof(double) * 16 * (size_t)max_blocks;
    P.total = off;
    P.no_instant = h.instant_metric_coupling == 0.0;
    return CRESSO_OK;
}

}  // namespace
}  // namespace cresso

using namespace cresso;

extern "C" cresso_scalar_plan* cresso_scalar_plan_create(const cresso_scalar_desc* host_descs, int32_t count,
                                                         const cresso_hyper* hyper) {
    if (count <= 0 || !host_descs || !hyper) {
        fail(CRESSO_E_INVALID, "scalar route: plan needs count > 0, descriptors and hyperparameters");
        return nullptr;
    }
    if (!(hyper->drive_clip > 0.0)) {
        fail(CRESSO_E_INVALID, "scalar route: drive_clip must be positive");
        return nullptr;
    }
    cresso_scalar_plan* P = new cresso_scalar_plan();
    if (build_plan(host_descs, count, *hyper, *P) != CRESSO_OK) {
        delete P;
        return nullptr;
    }
    for (int k = 0; k < 2; ++k) {
        hipError_t e = hipHostMalloc((void**)&P->staging[k], sizeof(void*) * (size_t)count,
                                     hipHostMallocMapped | hipHostMallocCoherent);
        if (e == hipSuccess) e = hipHostGetDevicePointer((void**)&P->dstaging[k], (void*)P->staging[k], 0);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&P->ev[k], hipEventDisableTiming);
        if (e != hipSuccess) {
            hip_fail(e, "scalar route: plan staging");
            cresso_scalar_plan_destroy(P);
            return nullptr;
        }
    }
    return P;
}

extern "C" void cresso_scalar_plan_destroy(cresso_scalar_plan* P) {
    if (!P) return;
    for (int k = 0; k < 2; ++k) {
        if (P->ev[k]) {
            (void)hipEventSynchronize(P->ev[k]);
            (void)hipEventDestroy(P->ev[k]);
        }
        if (P->staging[k]) (void)hipHostFree(P->staging[k]);
    }
    delete P;
}

extern "C" size_t cresso_scalar_plan_bytes(const cresso_scalar_plan* P) { return P ? P->total : 0; }

extern "C" int32_t cresso_scalar_plan_upload(cresso_scalar_plan* P, void* dev_table, size_t table_bytes, void* stream) {
    if (!P || !dev_table) return fail(CRESSO_E_INVALID, "scalar route: null plan or table");
    if (table_bytes < P->total)
        return fail(CRESSO_E_INVALID, "scalar route: table of %zu bytes is smaller than the %zu bytes needed", table_bytes, P->total);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    unsigned char* table = reinterpret_cast<unsigned char*>(dev_table);
    const size_t count = P->recs.size();
    hipError_t e = hipMemcpyAsync(table, P->recs.data(), sizeof(ScalarRec) * count, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(table + P->steps_off, P->steps.data(), sizeof(int32_t) * count, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) {
        std::vector<const void*> g(count);
        for (size_t j = 0; j < count; ++j) g[j] = P->recs[j].d.grad;
        e = hipMemcpyAsync(table + P->grads_off, g.data(), sizeof(void*) * count, hipMemcpyHostToDevice, s);
    }
    if (e == hipSuccess && !P->bmap.empty())
        e = hipMemcpyAsync(table + P->bmap_off, P->bmap.data(), sizeof(int32_t) * P->bmap.size(), hipMemcpyHostToDevice, s);
    // pageable sources: make sure the copies have consumed them before returning
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e == hipSuccess) {
        P->table_grads.resize(count);
        for (size_t j = 0; j < count; ++j) P->table_grads[j] = P->recs[j].d.grad;
        P->table_ptr = dev_table;
        P->cur = -1;
    }
    return e == hipSuccess ? CRESSO_OK : hip_fail(e, "scalar route: table upload");
}

extern "C" int32_t cresso_scalar_plan_step(cresso_scalar_plan* P, void* dev_table, const void* const* grads,
                                           const cresso_hyper* hyper, void* stream) {
    if (!P || !dev_table || !hyper) return fail(CRESSO_E_INVALID, "scalar route: null argument");
    const cresso_hyper& h = *hyper;
    if (!(h.drive_clip > 0.0)) return fail(CRESSO_E_INVALID, "scalar route: drive_clip must be positive");
    if ((h.instant_metric_coupling == 0.0) != P->no_instant)
        return fail(CRESSO_E_INVALID, "scalar route: instant_metric_coupling switched between zero and non-zero; re-plan");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    unsigned char* table = reinterpret_cast<unsigned char*>(dev_table);
    const size_t count = P->recs.size();
    int ks = P->cur;   // grads == NULL: the pointers of the previous call
    if (grads) {
        // the table holds these pointers (those of the upload, as when the
        // caching allocator hands the same grad blocks back): read them there
        bool same = P->table_ptr == dev_table && P->table_grads.size() == count;
        for (size_t j = 0; same && j < count; ++j) same = grads[P->order[j]] == P->table_grads[j];
        ks = -1;
        if (!same) {
            const int k = P->flip;
            P->flip ^= 1;
            hipError_t e = hipEventSynchronize(P->ev[k]);   // the kernels that last read staging[k] are done
            if (e != hipSuccess) return hip_fail(e, "scalar route: staging wait");
            for (size_t j = 0; j < count; ++j) {
                const void* gp = grads[P->order[j]];
                if (!gp) return fail(CRESSO_E_INVALID, "scalar route: null grad pointer for tensor %d", P->order[j]);
                P->staging[k][j] = gp;
            }
            ks = k;
        }
    }
    P->cur = ks;
    const ScalarRec* drecs = reinterpret_cast<const ScalarRec*>(table);
    int32_t* dsteps = reinterpret_cast<int32_t*>(table + P->steps_off);
    const void* const* dgrads = ks >= 0 ? P->dstaging[ks] : reinterpret_cast<const void* const*>(table + P->grads_off);
    for (const auto& G : P->groups) {
        const WideGeom wg{G.nblocks, reinterpret_cast<const int32_t*>(table + G.map_off),
                          reinterpret_cast<double*>(table + P->part_off)};
        hipError_t e = dispatch(G.v, drecs, dsteps, dgrads, G.first, G.count, G.lds, table, wg, h, s);
        if (e != hipSuccess) return hip_fail(e, "scalar route: kernel launch");
    }
    if (ks >= 0) {
        const hipError_t e = hipEventRecord(P->ev[ks], s);
        if (e != hipSuccess) return hip_fail(e, "scalar route: staging event");
    }
    return CRESSO_OK;
}
