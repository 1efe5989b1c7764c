// Spectral / coordinate-hash route of CRESSO5 on gfx950 (large tensors): kernels
// and the step sequence (run_step), shared by the route's translation units.
//
// Math: the reference's PyTorch spectral step, cresso_v5.py:945-1353.  The
// fused CUDA path of the reference (cresso_cuda_kernel.cu, ~46 custom + ~40
// eager launches per tensor, fp64 basis evaluation per element) is not
// followed; this is a from-scratch design:
//
// * Field view.  A tensor of shape (d0, d1, ..., dk) is viewed as rows x cols
//   with rows = d0 and cols = d1*...*dk (rows = 1 for 1-D tensors).  Every
//   basis mode is separable across that split (the phase is additive over
//   axes and the window multiplicative), so each normalized carrier is
//       C = a1(row) b1(col) - a2(row) b2(col)   (additive-phase kinds)
//       S = a2(row) b1(col) + a1(row) b2(col)
//   or C = a1 b1, S = a2 b2 (product kind).  The workspace holds, once per
//   (shape, rank, max_frequency): a row table a[rows][2R], a table of the K
//   distinct column carriers b[K][cols] (K <= 2R+1), the normalization stats
//   in closed form (fp64 sums over the two tables), the hash bins of every
//   element (data independent: packed bytes, computed once) and bin counts.
// * Projection of a field x (mean(x C_r)) is a per-lane accumulation
//   Z1_r = sum_rows a1_r x, Z2_r = sum_rows a2_r x over the lane's column,
//   combined with the lane's b values at the end; reconstruction is
//   out = alpha_0(row) + sum_k alpha_k(row) b_k(col) with alpha built per row
//   panel in LDS from the mode coefficients.  On the fast path (MODE 1) sweeps
//   3 and 4 run both as 16x16x4 fp32 MFMA tiles.
// * Step = 5 sweeps over the field, each followed by a one-block finalize
//   (deterministic fixed-order fp64 reductions of per-block partials) that
//   runs the rank-level recurrences and writes the next sweep's coefficients:
//     S1 sum f^2 -> F1 force RMS, scale
//     S2 density: hash histograms (64-bit fixed point, integer atomics),
//        log-density projection, axis density sums -> F2 hash metric tables,
//        metric oscillator, recon coefficients; M1 instant-metric factors
//     S3 tangent t (stored), t projection, port histograms, 13 moments of t
//        -> F3 surprise, port projection (1 + tm) mean(t Xn) - G u_pred from
//        the basis Gram matrix G, hash impulse, confidence, contact
//        oscillator, drive coefficients (every RMS in closed form)
//     S4 drive without the hash term (written over t); sum d^2, sum d h,
//        sum h^2 -> F4 drive energy, gain.  Fast path: F3 already has the
//        hash term's RMS in closed form (bin co-occurrence counts), so S4
//        writes the full drive and sums drive^2
//     S5 param -= lr * cast((d + c5 h) * gain), resp. cast(drive * gain)
#pragma once

// Each translation unit that includes this header uses a subset of it.
#pragma clang diagnostic ignored "-Wunneeded-internal-declaration"
#pragma clang diagnostic ignored "-Wunused-function"

#include "common.hpp"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <type_traits>
#include <cstring>
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

namespace cresso {
namespace {

constexpr int SP_NT = 256;
constexpr int SP_MAXR = 32;
constexpr int SP_MAXT = 8;
constexpr int SP_FIN_NT = 1024;  // workspace set-up kernels
constexpr int SP_FN_NT = 512;    // per-step finalize kernels (room for fp64 accumulators)
constexpr int SP_FN_E = 2048;    // fin2 keeps the new hash energies in LDS up to this many bins (T B)
// Fast-path histograms keep SP_NHIST interleaved copies ([bin][copy], copy =
// lane & 3): lanes of one wave then collide on an address only when both the
// bin and the copy match.  The copies are summed (integers: any order) before
// the block's global atomics.  LDS is sized for the copies in every mode.
constexpr int SP_NHIST = 4;
// Copies of the global histogram (hist[copy][T*B]) that part_reduce's blocks
// spread their atomics over; the finish kernels read their sum.
constexpr int SP_HCOPIES = 8;
// Closed-form hash term with four tables: 6 table pairs x (B / 16) row chunks
// of co-occurrence counts plus one block of the per-table terms (B <= 256).
constexpr int SP_HHP_MAX = 6 * 16 + 1;

enum ModeType : int32_t { M_ZERO = 0, M_ADD = 1, M_PROD = 2 };

// fp32 constants of one (mode, axis) of the carrier (cast from double exactly
// as the reference's torch expressions cast their Python scalars)
struct AxisConst {
    float pf;     // fl32(pi * f)
    float pc;     // fl32(pi * c * max(1, f)) (chirp kinds)
    float mu;     // fl32(center) (kind 3)
    float sig;    // fl32(width)  (kind 3)
    int32_t f;
    int32_t pad[3];
};

struct ModeMeta {
    int32_t type;   // ModeType
    int32_t kind;   // r % 4 of the reference (0 additive, 1 product, 2 chirp, 3 chirp+window)
    int32_t k1, k2; // column carriers (k2 = -1: identically zero)
};

struct CarrierSrc {  // which mode defines column carrier k and which component (0: b1, 1: b2)
    int32_t mode, comp;
};

struct Geom {
    int64_t n, rows, cols;
    int32_t R, K, T, B;
    int32_t ndim, ntrail;
    int64_t tdim[8];  // dims of the column group, row-major
    int32_t PR, slabs, panels, nblk;   // tiles of the field sweeps
    int32_t nblk1;                     // blocks of the flat force-RMS sweep
    int32_t KA;                        // alpha row width: 2*rmax+1 carriers (zero beyond K) + constant
    int32_t RW;                        // row-table width: 2*rmax (zero beyond 2R)
    int64_t chunk1;                    // elements per block of the flat sweep (multiple of 4)
    double hs_row, hs_col;             // fixed-point scales of the axis density sums
    double shrink;                     // 1/sqrt(max(1, 0.7 log2(R + 1))) (cresso_v5.py:362-376)
    double inv_n;                      // 1/n
    int32_t binbytes, bpb, one_d, nblkg;   // nblkg: blocks of the Gram pair-sum kernel
    int32_t hcopies;                   // copies of the global histogram (SP_HCOPIES for the matrix-core
                                       // sweeps' atomic merges, else 1)
};

// 64-bit words of a plan's global density histogram: hcopies copies of the
// [T][B] low words, then one [T][B] table of high words.
__host__ __device__ inline int64_t hist_words(const Geom& g) { return (int64_t)(g.hcopies + 1) * g.T * g.B; }

struct Offs {
    size_t axc, meta, csrc, rowtab, coltab, stats, bounds, gram, gpart, counts, cooc, bins;   // shape tables
    size_t tbuf, part, part1, sums, hist, hpart, lt, imp, rowfx, colfx, colfac, terms, ctrl, desc;   // per-step scratch
    size_t total;
};

// fp64 constants of one (mode, axis) of the carrier, as the reference's fp64
// work dtype evaluates its Python scalars (cresso_v5.py:272-348)
struct AxisConst64 {
    double pf;    // pi * f
    double pcm;   // (pi * c) * max(1, f) (chirp kinds)
    double mu;    // center (kind 3)
    double sig;   // width  (kind 3)
    int32_t f, kind;
};

// Workspace regions of a plan with the fp64 work dtype (spectral_f64.hip),
// after the fp32 layout (whose bins, counts and bin-count maximum it shares).
struct Offs64 {
    size_t axc, tab, nst, sums, part, hist, lt, marg, terms, ctrl, tbuf;
    int32_t nblk;   // blocks of the element sweeps
    int64_t sumd;   // sum of the dims (axis-table length per mode)
};

// per-step device scalars (written by finalize kernels)
struct Ctrl {
    float scale, inv_s;
    float gden, kappa;
    float rc[4][SP_MAXR][2];  // recon coefficients: 0 metric, 1 pred, 2 pred', 3 echo
    float rconst[4];
    float wpred[2 * SP_MAXR]; // weights of the pre-contact prediction on the normalized carriers
    double hs_ds, hs_P;       // fixed-point scales of the histograms
    double hs_hi;             // weight of one unit of the density histogram's high words
    double cmax;              // largest bin count of any table (data independent, set at workspace init)
    float nscale, srms;
    // drive = k_rat rat + k_ths tanh(t/clip) + k_root root + k_t t + k_pred pred' + k_echo echo
    //         + k_nov tanh(err' nscale) + k_hash hash_pred
    float k_rat, k_ths, k_root, k_t, k_pred, k_echo, k_nov, k_hash, gain;
    float de_prev;            // drive_energy before this step (sweep 5 updates the state)
    float fr_prev;            // force_rms before this step (sweep 2 updates the state)
    int32_t hard_hash;        // four-table closed form: the hard channel's hash term is on (set by fin3)
    int32_t kq;               // 62 - ceil(log2 cmax): limit exponent of the density histogram's low words
    double hh_part[SP_HHP_MAX];   // four-table closed form: partial sums of sum_i hp_i^2 (hh4_kernel)
};

// state pointers of one tensor (kernel argument)
struct SpecState {
    float *force_rms, *drive_energy, *surprise, *action;
    const float* omega;
    float *q_cos, *q_sin, *p_cos, *p_sin, *metric_cos, *metric_sin, *metric_p_cos, *metric_p_sin;
    float *calcium_cos, *calcium_sin, *conf;
    float *hash_energy, *hash_impulse, *hash_refractory;
};

__host__ __device__ inline SpecState spec_state(const cresso_spectral_desc& d) {
    SpecState st;
    st.force_rms = (float*)d.force_rms; st.drive_energy = (float*)d.drive_energy;
    st.surprise = (float*)d.surprise; st.action = (float*)d.action; st.omega = (const float*)d.omega;
    st.q_cos = (float*)d.q_cos; st.q_sin = (float*)d.q_sin; st.p_cos = (float*)d.p_cos; st.p_sin = (float*)d.p_sin;
    st.metric_cos = (float*)d.metric_cos; st.metric_sin = (float*)d.metric_sin;
    st.metric_p_cos = (float*)d.metric_p_cos; st.metric_p_sin = (float*)d.metric_p_sin;
    st.calcium_cos = (float*)d.calcium_cos; st.calcium_sin = (float*)d.calcium_sin; st.conf = (float*)d.mode_confidence;
    st.hash_energy = (float*)d.hash_energy; st.hash_impulse = (float*)d.hash_impulse;
    st.hash_refractory = (float*)d.hash_refractory;
    return st;
}

// Tensors of one step launch.  A batched step runs several tensors of one
// plan in each launch: blockIdx.y picks the tensor, whose per-step scratch
// (tangent field, partials, histograms, control block, and a device copy of
// its descriptor: grad, param, state pointers, step) sits blockIdx.y * ls
// bytes after the first tensor's.  The shape tables (carrier tables, bins,
// counts, closed-form stats) are shared.  A single-tensor launch passes
// dv = nullptr and ls = 0 and takes its pointers from the kernel arguments;
// its grid has one row.
struct Lanes {
    const cresso_spectral_desc* dv;   // the first tensor's descriptor copy, or nullptr
    size_t ls;
};
template <typename T> __device__ __forceinline__ T* lane_at(T* p, const Lanes& L) {
    using C = typename std::conditional<std::is_const<T>::value, const char, char>::type;
    return reinterpret_cast<T*>(reinterpret_cast<C*>(p) + (size_t)blockIdx.y * L.ls);
}
__device__ __forceinline__ const cresso_spectral_desc& lane_desc(const Lanes& L) { return *lane_at(L.dv, L); }

constexpr int NV2 = 2 + 2 * SP_MAXR;            // sum L, sum dens, proj L (C,S)
constexpr int NV3 = 15 + 2 * SP_MAXR;           // see sweep3
constexpr int NV4 = 3;                          // sum d^2, sum d hp, sum hp^2
constexpr int NVMAX = NV3;

#ifdef CRESSO_SPECTRAL_WS_KERNELS
// ---------------------------------------------------------------------------
// workspace construction
// ---------------------------------------------------------------------------
__device__ __forceinline__ float axis_u(int64_t k, int64_t dim) { return ((float)k + 0.5f) / (float)dim; }

// per-axis phase of mode r on one axis (fp32 like cresso_v5.py:272-292)
__device__ __forceinline__ float axis_phase(const AxisConst& a, float u, bool chirp) {
    float ph = a.pf * u;
    if (chirp) {
        const float d = u - 0.5f;
        ph = ph + a.pc * (d * d);
    }
    return ph;
}
__device__ __forceinline__ float axis_window(const AxisConst& a, float u) {
    const float z = (u - a.mu) / a.sig;
    return expf(-0.5f * (z * z));
}

// carriers of mode r over a set of axes given the element coordinates on them
__device__ void group_carrier(const AxisConst* ax, int kind, int naxes, const int64_t* coord, const int64_t* dims,
                              float& c1, float& c2) {
    if (kind == 1) {
        float cp = 1.f, sp = 1.f;
        for (int a = 0; a < naxes; ++a) {
            if (ax[a].f == 0) continue;
            const float ph = ax[a].pf * axis_u(coord[a], dims[a]);
            cp = cp * cosf(ph);
            sp = sp * sinf(ph);
        }
        c1 = cp;
        c2 = sp;
        return;
    }
    const bool chirp = kind != 0;
    float ph = 0.f, w = 1.f;
    bool any = false;
    for (int a = 0; a < naxes; ++a) {
        if (ax[a].f == 0 && !chirp) continue;
        const float u = axis_u(coord[a], dims[a]);
        const float p = axis_phase(ax[a], u, chirp);
        ph = any ? ph + p : p;
        any = true;
        if (kind == 3) w = (a == 0) ? axis_window(ax[a], u) : w * axis_window(ax[a], u);
    }
    c1 = w * cosf(ph);
    c2 = w * sinf(ph);
}

__global__ void ws_rowtab_kernel(Geom g, const AxisConst* __restrict__ axc, const ModeMeta* __restrict__ meta,
                                 float* __restrict__ rowtab) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= g.rows) return;
    for (int r = 0; r < g.R; ++r) {
        float a1 = 1.f, a2 = 0.f;
        const int kind = meta[r].kind;
        if (meta[r].type == M_ZERO) {
            a1 = 1.f;
            a2 = 0.f;
        } else if (g.one_d) {
            // empty leading group: phase 0, window 1 (kinds 0/2/3) or empty products (kind 1)
            a1 = 1.f;
            a2 = kind == 1 ? 1.f : 0.f;
        } else {
            const int64_t coord = i;
            const int64_t dim = g.rows;
            group_carrier(axc + (size_t)r * g.ndim, kind, 1, &coord, &dim, a1, a2);
        }
        rowtab[i * g.RW + 2 * r] = a1;
        rowtab[i * g.RW + 2 * r + 1] = a2;
    }
    for (int j = 2 * g.R; j < g.RW; ++j) rowtab[i * g.RW + j] = 0.f;
}

__global__ void ws_coltab_kernel(Geom g, const AxisConst* __restrict__ axc, const ModeMeta* __restrict__ meta,
                                 const CarrierSrc* __restrict__ csrc, float* __restrict__ coltab) {
    const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= g.cols) return;
    int64_t coord[8];
    int64_t rem = c;
    for (int a = g.ntrail - 1; a >= 0; --a) {
        coord[a] = rem % g.tdim[a];
        rem /= g.tdim[a];
    }
    const int first_axis = g.one_d ? 0 : 1;
    for (int k = 0; k < g.K; ++k) {
        float v = 1.f;
        if (csrc[k].mode >= 0) {
            const int r = csrc[k].mode;
            float b1, b2;
            group_carrier(axc + (size_t)r * g.ndim + first_axis, meta[r].kind, g.ntrail, coord, g.tdim, b1, b2);
            v = csrc[k].comp == 0 ? b1 : b2;
        }
        coltab[(size_t)k * g.cols + c] = v;
    }
    for (int k = g.K; k < g.KA - 1; ++k) coltab[(size_t)k * g.cols + c] = 0.f;
}

// block-wide max of two non-negative values; every thread receives them
__device__ void block_max2(double (&v)[2], double* lds) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    for (int i = 0; i < 2; ++i)
        for (int m = 32; m >= 1; m >>= 1) v[i] = fmax(v[i], __shfl_xor(v[i], m, 64));
    if (lane == 0) {
        lds[2 * wave] = v[0];
        lds[2 * wave + 1] = v[1];
    }
    __syncthreads();
    double a = 0.0, b = 0.0;
    for (int w = 0; w < nw; ++w) {
        a = fmax(a, lds[2 * w]);
        b = fmax(b, lds[2 * w + 1]);
    }
    v[0] = a;
    v[1] = b;
    __syncthreads();
}

// Closed-form normalization stats (cresso_v5.py:138-142 over the separable
// carriers): per mode (mu_c, 1/max(sqrt(var_c+1e-12),1e-6), mu_s, ...) and a
// bound of max|C_n|, max|S_n| used to size fixed-point histograms.  One
// block per mode.
__global__ __launch_bounds__(SP_FIN_NT) void ws_stats_kernel(Geom g, const ModeMeta* __restrict__ meta,
                                                             const float* __restrict__ rowtab,
                                                             const float* __restrict__ coltab, double* __restrict__ stats,
                                                             double* __restrict__ bounds) {
    __shared__ double red[16 * 8];
    const int tid = threadIdx.x;
    {
        const int r = blockIdx.x;   // one block per mode
        // row sums of this mode
        double v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int64_t i = tid; i < g.rows; i += SP_FIN_NT) {
            const double a1 = rowtab[i * g.RW + 2 * r], a2 = rowtab[i * g.RW + 2 * r + 1];
            v[0] += a1; v[1] += a2; v[2] += a1 * a1; v[3] += a1 * a2; v[4] += a2 * a2;
            v[5] = fmax(v[5], fabs(a1)); v[6] = fmax(v[6], fabs(a2));
        }
        double mx[2] = {v[5], v[6]};
        v[5] = v[6] = 0.0;
        block_sum<8>(v, red);
        block_max2(mx, red);
        const double Sa1 = v[0], Sa2 = v[1], Sa11 = v[2], Sa12 = v[3], Sa22 = v[4];
        const double ma1 = mx[0], ma2 = mx[1];
        const int k1 = meta[r].k1, k2 = meta[r].k2;
        double u[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        double bm1 = 0.0, bm2 = 0.0;
        for (int64_t c = tid; c < g.cols; c += SP_FIN_NT) {
            const double b1 = coltab[(size_t)k1 * g.cols + c];
            const double b2 = k2 >= 0 ? (double)coltab[(size_t)k2 * g.cols + c] : 0.0;
            u[0] += b1; u[1] += b2; u[2] += b1 * b1; u[3] += b1 * b2; u[4] += b2 * b2;
            bm1 = fmax(bm1, fabs(b1)); bm2 = fmax(bm2, fabs(b2));
        }
        block_sum<8>(u, red);
        double bm[2] = {bm1, bm2};
        block_max2(bm, red);
        if (tid == 0) {
            const double Sb1 = u[0], Sb2 = u[1], Sb11 = u[2], Sb12 = u[3], Sb22 = u[4];
            const double mb1 = bm[0], mb2 = bm[1];
            const double n = (double)g.n;
            double sc, scc, ss, sss, mc, ms;
            if (meta[r].type == M_ZERO) {
                stats[4 * r + 0] = 0.0; stats[4 * r + 1] = 1.0;  // C = 1, unnormalized
                stats[4 * r + 2] = 0.0; stats[4 * r + 3] = 0.0;  // S = 0
                bounds[2 * r] = 1.0; bounds[2 * r + 1] = 0.0;
            } else {
                if (meta[r].type == M_ADD) {
                    sc = Sa1 * Sb1 - Sa2 * Sb2;
                    scc = Sa11 * Sb11 - 2.0 * Sa12 * Sb12 + Sa22 * Sb22;
                    ss = Sa2 * Sb1 + Sa1 * Sb2;
                    sss = Sa22 * Sb11 + 2.0 * Sa12 * Sb12 + Sa11 * Sb22;
                    mc = ma1 * mb1 + ma2 * mb2;
                    ms = ma2 * mb1 + ma1 * mb2;
                } else {
                    sc = Sa1 * Sb1; scc = Sa11 * Sb11; ss = Sa2 * Sb2; sss = Sa22 * Sb22;
                    mc = ma1 * mb1; ms = ma2 * mb2;
                }
                const double muc = sc / n, mus = ss / n;
                const double vc = fmax(scc / n - muc * muc, 0.0), vs = fmax(sss / n - mus * mus, 0.0);
                const double ic = 1.0 / fmax(sqrt(vc + 1e-12), 1e-6), is = 1.0 / fmax(sqrt(vs + 1e-12), 1e-6);
                stats[4 * r + 0] = muc; stats[4 * r + 1] = ic; stats[4 * r + 2] = mus; stats[4 * r + 3] = is;
                bounds[2 * r] = (mc + fabs(muc)) * ic;
                bounds[2 * r + 1] = (ms + fabs(mus)) * is;
            }
        }
    }
}

// Gram matrix of the normalized basis, G[v][w] = mean over elements of
// Xn_v Xn_w (v = 2r: C_r, v = 2r + 1: S_r), in closed form from the separable
// tables: each raw carrier is a sum of at most two (row factor x column
// carrier) terms, so sum_i X_v X_w is a combination of the row pair sums
// sum_rows a_x a_y (x, y < 2R) and the column pair sums sum_cols b_k b_l
// (k, l < K).  Pair sums are split over nblkg blocks (fixed-order partials).
__global__ __launch_bounds__(256) void ws_pairsum_kernel(Geom g, const float* __restrict__ rowtab,
                                                         const float* __restrict__ coltab, double* __restrict__ gpart) {
    const int V = 2 * g.R, NA = V * V, NB = g.K * g.K;
    const int nb = g.nblkg;
    const int64_t r0 = g.rows * blockIdx.x / nb, r1 = g.rows * (blockIdx.x + 1) / nb;
    const int64_t c0 = g.cols * blockIdx.x / nb, c1 = g.cols * (blockIdx.x + 1) / nb;
    for (int p = threadIdx.x; p < NA + NB; p += blockDim.x) {
        double s = 0.0;
        if (p < NA) {
            const int x = p / V, y = p - x * V;
            for (int64_t i = r0; i < r1; ++i) s += (double)rowtab[i * g.RW + x] * (double)rowtab[i * g.RW + y];
        } else {
            const int q = p - NA, k = q / g.K, l = q - k * g.K;
            for (int64_t c = c0; c < c1; ++c)
                s += (double)coltab[(size_t)k * g.cols + c] * (double)coltab[(size_t)l * g.cols + c];
        }
        gpart[(size_t)blockIdx.x * (NA + NB) + p] = s;
    }
}

// terms (sign, row factor x, column carrier k) of raw carrier v; returns the count
__device__ int carrier_terms(const ModeMeta& m, int v, float* sg, int* x, int* k) {
    const int r = v >> 1, c = v & 1;
    int n = 0;
    auto add = [&](float s_, int x_, int k_) {
        if (k_ >= 0) { sg[n] = s_; x[n] = x_; k[n] = k_; ++n; }
    };
    if (m.type == M_ZERO) {
        if (c == 0) add(1.f, 2 * r, m.k1);
    } else if (m.type == M_ADD) {
        if (c == 0) { add(1.f, 2 * r, m.k1); add(-1.f, 2 * r + 1, m.k2); }
        else { add(1.f, 2 * r + 1, m.k1); add(1.f, 2 * r, m.k2); }
    } else {
        if (c == 0) add(1.f, 2 * r, m.k1);
        else add(1.f, 2 * r + 1, m.k2);
    }
    return n;
}

__global__ __launch_bounds__(SP_FIN_NT) void ws_gram_kernel(Geom g, const ModeMeta* __restrict__ meta,
                                                            const double* __restrict__ stats,
                                                            const double* __restrict__ gpart, double* __restrict__ gram) {
    const int V = 2 * g.R, NA = V * V, NB = g.K * g.K;
    extern __shared__ double s_pair[];   // [NA + NB]
    for (int p = threadIdx.x; p < NA + NB; p += SP_FIN_NT) {
        double s = 0.0;
        for (int b = 0; b < g.nblkg; ++b) s += gpart[(size_t)b * (NA + NB) + p];
        s_pair[p] = s;
    }
    __syncthreads();
    const double n = (double)g.n;
    for (int p = threadIdx.x; p < V * V; p += SP_FIN_NT) {
        const int v = p / V, w = p - v * V;
        float sv[2], sw[2];
        int xv[2], xw[2], kv[2], kw[2];
        const int nv = carrier_terms(meta[v >> 1], v, sv, xv, kv);
        const int nw = carrier_terms(meta[w >> 1], w, sw, xw, kw);
        double sum = 0.0;
        for (int i = 0; i < nv; ++i)
            for (int j = 0; j < nw; ++j)
                sum += (double)(sv[i] * sw[j]) * s_pair[xv[i] * V + xw[j]] * s_pair[NA + kv[i] * g.K + kw[j]];
        // Xn = (X - mu) ic with mu the normalization shift and m the true mean
        // of X (equal, except the constant carrier: mu = 0, m = 1):
        // mean(Xn_v Xn_w) = ic_v ic_w (mean(X_v X_w) - mu_v m_w - mu_w m_v + mu_v mu_w)
        const double muv = stats[4 * (v >> 1) + 2 * (v & 1)], icv = stats[4 * (v >> 1) + 2 * (v & 1) + 1];
        const double muw = stats[4 * (w >> 1) + 2 * (w & 1)], icw = stats[4 * (w >> 1) + 2 * (w & 1) + 1];
        const double mv = (meta[v >> 1].type == M_ZERO && (v & 1) == 0) ? 1.0 : muv;
        const double mw = (meta[w >> 1].type == M_ZERO && (w & 1) == 0) ? 1.0 : muw;
        gram[p] = icv * icw * (sum / n - muv * mw - muw * mv + muv * muw);
    }
}

// Packed bins of every element (data independent; computed once per shape)
// and exact bin counts: per-block u32 counts in LDS when the [T][B] table
// fits (integer adds, so the totals do not depend on arrival order), merged
// into the u64 totals with one global atomic per non-empty bin.
constexpr int WS_BINS_LDS = 8192;  // u32 counters privatised per block
__global__ __launch_bounds__(256) void ws_bins_kernel(Geom g, unsigned char* __restrict__ bins,
                                                      unsigned long long* __restrict__ counts) {
    __shared__ unsigned int s_cnt[WS_BINS_LDS];
    const int TB = g.T * g.B;
    const bool priv = TB <= WS_BINS_LDS;
    if (priv)
        for (int i = threadIdx.x; i < TB; i += blockDim.x) s_cnt[i] = 0u;
    __syncthreads();
    const int64_t mask = (g.B & (g.B - 1)) == 0 ? (int64_t)g.B - 1 : -1;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < g.n; i += stride) {
        uint64_t packed = 0;
        for (int t = 0; t < g.T; ++t) {
            const HashSalt s = hash_salt(t);
            const int b = hash_bin((uint64_t)i, s, g.B, mask);
            packed |= (uint64_t)b << (8 * g.bpb * t);
            if (priv)
                atomicAdd(&s_cnt[t * g.B + b], 1u);
            else
                atomicAdd(&counts[(size_t)t * g.B + b], 1ull);
        }
        switch (g.binbytes) {
            case 1: bins[i] = (unsigned char)packed; break;
            case 2: reinterpret_cast<uint16_t*>(bins)[i] = (uint16_t)packed; break;
            case 4: reinterpret_cast<uint32_t*>(bins)[i] = (uint32_t)packed; break;
            default: reinterpret_cast<uint64_t*>(bins)[i] = packed; break;
        }
    }
    __syncthreads();
    if (priv)
        for (int i = threadIdx.x; i < TB; i += blockDim.x)
            if (s_cnt[i]) atomicAdd(&counts[i], (unsigned long long)s_cnt[i]);
}

#endif  // CRESSO_SPECTRAL_WS_KERNELS

// Co-occurrence counts of the tables' bins, cooc[pair][b][b'] = #{i : bin_t(i)
// = b, bin_t'(i) = b'} for each table pair t < t' (data independent, once per
// shape).  With them the hash prediction's sum of squares is a closed form
// over the impulse tables:
//   sum_i ((1/T) sum_t imp_t[b_t(i)])^2
//     = (sum_t sum_b cnt_t imp_t^2 + 2 sum_{t<t'} sum_{b,b'} cooc_tt' imp_t imp_t') / T^2.
// Used with two or four tables of one-byte bins (the matrix-core sweeps):
// one pair (fin3 evaluates the form) or six (hh4_kernel, many blocks).
__host__ __device__ inline bool cooc_closed(const Geom& g) {
    return (g.T == 2 || g.T == 4) && g.bpb == 1 && g.binbytes == g.T && g.B <= 256;
}
__host__ __device__ inline int cooc_pairs(const Geom& g) { return g.T * (g.T - 1) / 2; }
// tables of pair p of four: (0,1) (0,2) (0,3) (1,2) (1,3) (2,3)
__host__ __device__ inline void cooc_pair(int p, int& t0, int& t1) {
    t0 = p < 3 ? 0 : (p < 5 ? 1 : 2);
    t1 = p < 3 ? p + 1 : (p < 5 ? p - 1 : 3);
}
__host__ __device__ inline int hh4_chunks(const Geom& g) { return (g.B + 15) / 16; }
__host__ __device__ inline int hh4_blocks(const Geom& g) { return 6 * hh4_chunks(g) + 1; }
#ifdef CRESSO_SPECTRAL_WS_KERNELS
constexpr int WS_COOC_LDS = 16384;  // u32 counters privatised per block (B <= 128)
__global__ __launch_bounds__(256) void ws_cooc_kernel(Geom g, const uint16_t* __restrict__ bins,
                                                      unsigned long long* __restrict__ cooc) {
    __shared__ unsigned int s_cnt[WS_COOC_LDS];
    const int BB = g.B * g.B;
    const bool priv = BB <= WS_COOC_LDS;
    if (priv)
        for (int i = threadIdx.x; i < BB; i += blockDim.x) s_cnt[i] = 0u;
    __syncthreads();
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < g.n; i += stride) {
        const unsigned v = bins[i];
        const int k = (int)(v & 0xffu) * g.B + (int)(v >> 8);
        if (priv)
            atomicAdd(&s_cnt[k], 1u);
        else
            atomicAdd(&cooc[k], 1ull);
    }
    __syncthreads();
    if (priv)
        for (int i = threadIdx.x; i < BB; i += blockDim.x)
            if (s_cnt[i]) atomicAdd(&cooc[i], (unsigned long long)s_cnt[i]);
}

// Four tables of one-byte bins (packed 32-bit): the six pairs' counts, with
// 64-bit global atomics (6 x B^2 counters do not fit in LDS).
__global__ __launch_bounds__(256) void ws_cooc4_kernel(Geom g, const uint32_t* __restrict__ bins,
                                                       unsigned long long* __restrict__ cooc) {
    const int64_t BB = (int64_t)g.B * g.B;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < g.n; i += stride) {
        const uint32_t v = bins[i];
#pragma unroll
        for (int p = 0; p < 6; ++p) {
            int t0, t1;
            cooc_pair(p, t0, t1);
            const int b0 = (int)((v >> (8 * t0)) & 0xffu), b1 = (int)((v >> (8 * t1)) & 0xffu);
            atomicAdd(&cooc[p * BB + (int64_t)b0 * g.B + b1], 1ull);
        }
    }
}

// The same counts without global atomics per element: each block counts a
// contiguous chunk of elements into LDS, one table pair and one half of the
// B x B cells (32768 u32 counters, 128 KiB of dynamic LDS) at a time, and
// writes the chunk's whole table part[block][pair][cell]; ws_cooc4_sum_kernel
// adds the blocks' tables in block order (integers: exact).  The chunk is read
// once per (pair, half), from the cache after the first.
constexpr int WS_COOC4_NT = 1024;
constexpr int WS_COOC4_HALF = 32768;
__global__ __launch_bounds__(WS_COOC4_NT) void ws_cooc4_part_kernel(Geom g, const uint32_t* __restrict__ bins,
                                                                    unsigned int* __restrict__ part) {
    extern __shared__ unsigned int s_cnt[];
    const int BB = g.B * g.B;
    const int halves = (BB + WS_COOC4_HALF - 1) / WS_COOC4_HALF;
    const int64_t per = (g.n + gridDim.x - 1) / gridDim.x;
    const int64_t i0 = (int64_t)blockIdx.x * per, i1 = i0 + per < g.n ? i0 + per : g.n;
    for (int c = 0; c < 6 * halves; ++c) {
        const int p = c / halves, h = c % halves;
        int t0, t1;
        cooc_pair(p, t0, t1);
        const int lo = h * WS_COOC4_HALF, len = BB - lo < WS_COOC4_HALF ? BB - lo : WS_COOC4_HALF;
        for (int i = threadIdx.x; i < len; i += WS_COOC4_NT) s_cnt[i] = 0u;
        __syncthreads();
        // sixteen loads in flight per thread before their counts
        constexpr int U = 16;
        for (int64_t base = i0 + threadIdx.x; base < i1; base += (int64_t)U * WS_COOC4_NT) {
            uint32_t v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int64_t i = base + (int64_t)u * WS_COOC4_NT;
                v[u] = bins[i < i1 ? i : i0];
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int k = (int)((v[u] >> (8 * t0)) & 0xffu) * g.B + (int)((v[u] >> (8 * t1)) & 0xffu) - lo;
                if (base + (int64_t)u * WS_COOC4_NT < i1 && (unsigned)k < (unsigned)len) atomicAdd(&s_cnt[k], 1u);
            }
        }
        __syncthreads();
        unsigned int* dst = part + ((size_t)blockIdx.x * 6 + p) * (size_t)BB + lo;
        for (int i = threadIdx.x; i < len; i += WS_COOC4_NT) dst[i] = s_cnt[i];
        __syncthreads();
    }
}
__global__ __launch_bounds__(256) void ws_cooc4_sum_kernel(const unsigned int* __restrict__ part, int nblk, int64_t cells,
                                                           unsigned long long* __restrict__ cooc) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= cells) return;
    unsigned long long a = 0ull;
    for (int b = 0; b < nblk; ++b) a += part[(size_t)b * cells + i];
    cooc[i] = a;
}

#endif  // CRESSO_SPECTRAL_WS_KERNELS

__device__ __forceinline__ uint64_t load_bins(const unsigned char* __restrict__ bins, int64_t e, int binbytes) {
    switch (binbytes) {
        case 1: return bins[e];
        case 2: return reinterpret_cast<const uint16_t*>(bins)[e];
        case 4: return reinterpret_cast<const uint32_t*>(bins)[e];
        default: return reinterpret_cast<const uint64_t*>(bins)[e];
    }
}
__device__ __forceinline__ int bin_of(uint64_t packed, int t, int bpb) {
    return (int)((packed >> (8 * bpb * t)) & (bpb == 1 ? 0xffull : 0xffffull));
}

#ifdef CRESSO_SPECTRAL_WS_KERNELS
// ---------------------------------------------------------------------------
// workspace inspection (parity checks of what the sweeps consume)
// ---------------------------------------------------------------------------
// Bin of every element for every table, int32 [T][n].
__global__ void ws_unpack_bins_kernel(Geom g, const unsigned char* __restrict__ bins, int32_t* __restrict__ out) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < g.n; i += stride) {
        const uint64_t pk = load_bins(bins, i, g.binbytes);
        for (int t = 0; t < g.T; ++t) out[(size_t)t * g.n + i] = bin_of(pk, t, g.bpb);
    }
}

// Normalized carriers C_r, S_r of mode r at every element, formed from the
// row table, the column table and the closed-form stats exactly as the
// sweeps' reconstruction coefficients combine them.
__global__ void ws_basis_kernel(Geom g, const ModeMeta* __restrict__ meta, const float* __restrict__ rowtab,
                                const float* __restrict__ coltab, const double* __restrict__ stats, int r,
                                float* __restrict__ cout, float* __restrict__ sout) {
    const ModeMeta m = meta[r];
    const double muc = stats[4 * r], ic = stats[4 * r + 1], mus = stats[4 * r + 2], is = stats[4 * r + 3];
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < g.n; i += stride) {
        const int64_t row = i / g.cols, col = i - row * g.cols;
        const float a1 = rowtab[row * g.RW + 2 * r], a2 = rowtab[row * g.RW + 2 * r + 1];
        const float b1 = coltab[(size_t)m.k1 * g.cols + col];
        const float b2 = m.k2 >= 0 ? coltab[(size_t)m.k2 * g.cols + col] : 0.f;
        const float craw = m.type == M_ADD ? a1 * b1 - a2 * b2 : a1 * b1;
        const float sraw = m.type == M_ADD ? a2 * b1 + a1 * b2 : a2 * b2;
        cout[i] = (float)(((double)craw - muc) * ic);
        sout[i] = (float)(((double)sraw - mus) * is);
    }
}

// Unit entry points of the basis algebra (cresso_v5.py:351-376) on the
// workspace's separable tables, for parity checks and callers that want the
// reference's project/reconstruct: the normalized carriers of
// ws_basis_kernel, evaluated per element.
__device__ __forceinline__ void carrier_pair_n(const Geom& g, const ModeMeta& m, const float* __restrict__ rowtab,
                                               const float* __restrict__ coltab, const double* __restrict__ stats,
                                               int r, int64_t row, int64_t col, float& cn, float& sn) {
    const float a1 = rowtab[row * g.RW + 2 * r], a2 = rowtab[row * g.RW + 2 * r + 1];
    const float b1 = coltab[(size_t)m.k1 * g.cols + col];
    const float b2 = m.k2 >= 0 ? coltab[(size_t)m.k2 * g.cols + col] : 0.f;
    const float craw = m.type == M_ADD ? a1 * b1 - a2 * b2 : a1 * b1;
    const float sraw = m.type == M_ADD ? a2 * b1 + a1 * b2 : a2 * b2;
    cn = (float)(((double)craw - stats[4 * r]) * stats[4 * r + 1]);
    sn = (float)(((double)sraw - stats[4 * r + 2]) * stats[4 * r + 3]);
}

// sum_i x_i C_r(i), sum_i x_i S_r(i) (fp32 products, fp64 sums), value-major
// block partials part[2r + c][block]
__global__ __launch_bounds__(256) void ws_project_kernel(Geom g, const ModeMeta* __restrict__ meta,
                                                         const float* __restrict__ rowtab,
                                                         const float* __restrict__ coltab,
                                                         const double* __restrict__ stats, const float* __restrict__ x,
                                                         double* __restrict__ part) {
    __shared__ double lds[4 * 2 * SP_MAXR];
    double acc[2 * SP_MAXR];
#pragma unroll
    for (int v = 0; v < 2 * SP_MAXR; ++v) acc[v] = 0.0;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < g.n; i += stride) {
        const int64_t row = i / g.cols, col = i - row * g.cols;
        const float xv = x[i];
#pragma unroll
        for (int r = 0; r < SP_MAXR; ++r) {
            if (r < g.R) {
                float cn, sn;
                carrier_pair_n(g, meta[r], rowtab, coltab, stats, r, row, col, cn, sn);
                acc[2 * r] += (double)(xv * cn);
                acc[2 * r + 1] += (double)(xv * sn);
            }
        }
    }
    block_sum<2 * SP_MAXR>(acc, lds);
    for (int v = threadIdx.x; v < 2 * g.R; v += blockDim.x) part[(size_t)blockIdx.x * (2 * g.R) + v] = acc[v];
}

__global__ void ws_mean_kernel(const double* __restrict__ sums, int V, double inv_n, double* __restrict__ out) {
    const int v = threadIdx.x;
    if (v < V) out[v] = sums[v] * inv_n;
}

// shrink * sum_r g_r (cc_r C_r + sc_r S_r) in mode order, a gate of exactly 0
// skipping the mode (fp32 accumulation like the reference's add_(alpha))
__global__ __launch_bounds__(256) void ws_reconstruct_kernel(Geom g, const ModeMeta* __restrict__ meta,
                                                             const float* __restrict__ rowtab,
                                                             const float* __restrict__ coltab,
                                                             const double* __restrict__ stats,
                                                             const float* __restrict__ cc, const float* __restrict__ sc,
                                                             const float* __restrict__ gates, double shrink,
                                                             float* __restrict__ out) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < g.n; i += stride) {
        const int64_t row = i / g.cols, col = i - row * g.cols;
        float o = 0.f;
        for (int r = 0; r < g.R; ++r) {
            const double gr = gates ? (double)gates[r] : 1.0;
            if (gr == 0.0) continue;
            float cn, sn;
            carrier_pair_n(g, meta[r], rowtab, coltab, stats, r, row, col, cn, sn);
            o = o + (float)((double)cc[r] * shrink * gr) * cn;
            o = o + (float)((double)sc[r] * shrink * gr) * sn;
        }
        out[i] = o;
    }
}

#endif  // CRESSO_SPECTRAL_WS_KERNELS

// ---------------------------------------------------------------------------
// sweep helpers
// ---------------------------------------------------------------------------
template <typename T> __device__ __forceinline__ float ld(const T* p, int64_t i) { return to_f(p[i]); }

// 4 consecutive elements at e (e multiple of 4, base aligned to 4 elements)
template <typename T> struct Ld4;
template <> struct Ld4<float> {
    __device__ static void go(const float* p, int64_t e, float* o) {
        const float4 v = *reinterpret_cast<const float4*>(p + e);
        o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
    }
};
template <typename T> struct Ld4h {
    __device__ static void go(const T* p, int64_t e, float* o) {
        const uint2 raw = *reinterpret_cast<const uint2*>(p + e);
        const T* h = reinterpret_cast<const T*>(&raw);
        o[0] = to_f(h[0]); o[1] = to_f(h[1]); o[2] = to_f(h[2]); o[3] = to_f(h[3]);
    }
};
template <> struct Ld4<__half> : Ld4h<__half> {};
template <> struct Ld4<__hip_bfloat16> : Ld4h<__hip_bfloat16> {};
template <> struct Ld4<double> {
    __device__ static void go(const double* p, int64_t e, float* o) {
        const double2 a = *reinterpret_cast<const double2*>(p + e);
        const double2 b = *reinterpret_cast<const double2*>(p + e + 2);
        o[0] = (float)a.x; o[1] = (float)a.y; o[2] = (float)b.x; o[3] = (float)b.y;
    }
};

// VW = 4 or 8 consecutive elements from e (8: 16-byte loads of 2-byte types,
// two float4 loads of 4-byte ones)
template <typename T, int VW> struct LdV;
template <typename T> struct LdV<T, 4> : Ld4<T> {};
template <typename T> struct LdV<T, 8> {
    __device__ static void go(const T* p, int64_t e, float* o) {
        if constexpr (sizeof(T) == 2) {
            const uint4 raw = *reinterpret_cast<const uint4*>(p + e);
            const T* h = reinterpret_cast<const T*>(&raw);
#pragma unroll
            for (int c = 0; c < 8; ++c) o[c] = to_f(h[c]);
        } else {
            Ld4<T>::go(p, e, o);
            Ld4<T>::go(p, e + 4, o + 4);
        }
    }
};

// 4 consecutive elements stored at e, rounded to the storage dtype
template <typename T> struct St4;
template <> struct St4<float> {
    __device__ static void go(float* p, int64_t e, const float* v) {
        *reinterpret_cast<float4*>(p + e) = make_float4(v[0], v[1], v[2], v[3]);
    }
};
template <typename T> struct St4h {
    __device__ static void go(T* p, int64_t e, const float* v) {
        uint2 raw;
        T* q = reinterpret_cast<T*>(&raw);
        q[0] = from_w<T>(v[0]); q[1] = from_w<T>(v[1]); q[2] = from_w<T>(v[2]); q[3] = from_w<T>(v[3]);
        *reinterpret_cast<uint2*>(p + e) = raw;
    }
};
template <> struct St4<__half> : St4h<__half> {};
template <> struct St4<__hip_bfloat16> : St4h<__hip_bfloat16> {};

struct Tile {
    int slab, panel;
    int64_t col, r0, r1;
    bool colok;
};
__device__ __forceinline__ Tile tile_of(const Geom& g) {
    Tile t;
    t.slab = blockIdx.x % g.slabs;
    t.panel = blockIdx.x / g.slabs;
    t.col = (int64_t)t.slab * SP_NT + threadIdx.x;
    t.colok = t.col < g.cols;
    t.r0 = (int64_t)t.panel * g.PR;
    t.r1 = t.r0 + g.PR < g.rows ? t.r0 + g.PR : g.rows;
    return t;
}

// Block partials, one value at a time: DPP wave totals into LDS [wave][V],
// then a fixed-order sum over the block's waves, written block-major
// part[block][VS]: a block's values are one contiguous row, written as whole
// cache lines.  (Value-major rows, part[v][block], put 8 bytes of 16 blocks
// spread over all XCDs in every line: the partial-line writebacks cost sweeps
// 2 and 3 about 4 us each at C2.)
struct Partials {
    float* lds;
    int V;
    int VS;   // values written (the consumer's fixed width; slots V..VS-1 zero)
    __device__ __forceinline__ void add(int idx, float x) {
        const float w = wave_total(x);
        if ((threadIdx.x & 63) == 63) lds[(threadIdx.x >> 6) * V + idx] = w;
    }
    // block-major: part[block][stride], slots V..VS-1 zero (stride >= VS, default VS)
    __device__ __forceinline__ void flush(double* part, int stride = 0) {
        __syncthreads();
        const size_t row = (size_t)blockIdx.x * (stride > 0 ? stride : VS);
        for (int v = threadIdx.x; v < VS; v += SP_NT) {
            double s = 0.0;
            if (v < V)
                for (int w = 0; w < SP_NT / 64; ++w) s += (double)lds[w * V + v];
            part[row + v] = s;
        }
    }
};

__device__ __forceinline__ float reservoir_f(float old, float cur, double decay, int step) {
    if (step <= 1) return cur;
    return old * (float)decay + (float)(1.0 - decay) * cur;
}

// Histogram partials merged by part_reduce_kernel's blocks after the values:
// small merges (64-bin groups x partial rows <= 4096, e.g. C2's 128 bins x
// 1024 rows) take one bin per block over every row (pr_hist_rows = 0); larger
// ones blocks of 64 bins x pr_hist_rows partial rows (each wave reads 512
// contiguous bytes of a row), whose bin strides would otherwise make every
// load its own cache line.  A block covers at least 1/64 of the rows (8 to
// 64 rows: C5's 1024 bins x 4096 rows take 1024 blocks of 64, C4's 128 bins
// x 4000 rows 128 blocks of 63), so a bin receives at most 64 of the blocks'
// 64-bit atomic adds, spread over SP_HCOPIES copies of the histogram (same-
// address atomics from many CUs serialize; the finish kernels add the copies).
constexpr int PR_HB = 64;
constexpr int PR_U = 8;   // rows whose loads one part_reduce thread has in flight together
__host__ __device__ inline int pr_hist_rows(int TB, int nblk) {
    const int ng = (TB + PR_HB - 1) / PR_HB;
    if ((int64_t)ng * nblk <= 4096) return 0;
    const int r = (nblk + 63) / 64;
    return r < 8 ? 8 : (r > 64 ? 64 : r);
}
__host__ __device__ inline int pr_hist_blocks(int TB, int nblk) {
    const int hr = pr_hist_rows(TB, nblk);
    return hr == 0 ? TB : ((TB + PR_HB - 1) / PR_HB) * ((nblk + hr - 1) / hr);
}

// Cross-block merge of a sweep's partials spread over many CUs: block v < VS
// sums value v of every block's row part[block][VS] (thread j: blocks j,
// j + 256, ... in order; then a fixed-order DPP wave tree and the four wave
// totals in order) into sums[v].  The pr_hist_blocks(TB, nblk) blocks after
// them merge the matrix-core sweeps' per-block histogram partials
// (hpart[block][bin], 64-bit fixed point): one bin over every row each, or
// 64 bins of pr_hist_rows partial rows adding their integer sums into
// copy (row group mod SP_HCOPIES) of hist[bin] with 64-bit atomics (integer
// sums: the same in any order).  Every copy is zero on entry (the finish
// kernels clear them after reading).
__global__ __launch_bounds__(256) void part_reduce_kernel(
    const double* __restrict__ part, int nblk, int VS, double* __restrict__ sums,
    const unsigned long long* __restrict__ hpart, unsigned long long* __restrict__ hist, int TB, Lanes L) {
    part = lane_at(part, L); sums = lane_at(sums, L); hpart = lane_at(hpart, L); hist = lane_at(hist, L);
    __shared__ double s_w[4];
    __shared__ unsigned long long s_h[4][PR_HB];
    const int v = blockIdx.x;
    const int hr = pr_hist_rows(TB, nblk);
    // Each thread issues the loads of PR_U rows before adding any of them (a
    // loop of one load and one add per row waits one memory latency per row:
    // 34 us for 4096 rows), and adds them in row order, as one load per
    // iteration would.
    if (v >= VS && hr == 0) {
        // one bin, every block's row
        const int i = v - VS;
        unsigned long long a = 0ull;
        for (int b = threadIdx.x; b < nblk; b += 256 * PR_U) {
            unsigned long long x[PR_U];
#pragma unroll
            for (int u = 0; u < PR_U; ++u) x[u] = b + 256 * u < nblk ? hpart[(size_t)(b + 256 * u) * TB + i] : 0ull;
#pragma unroll
            for (int u = 0; u < PR_U; ++u) a += x[u];
        }
        for (int o = 32; o > 0; o >>= 1) a += __shfl_xor(a, o);
        if ((threadIdx.x & 63) == 0) s_h[threadIdx.x >> 6][0] = a;
        __syncthreads();
        if (threadIdx.x == 0) hist[i] = s_h[0][0] + s_h[1][0] + s_h[2][0] + s_h[3][0];
        return;
    }
    if (v >= VS) {
        const int hb = v - VS, ng = (TB + PR_HB - 1) / PR_HB;
        const int bin = (hb % ng) * PR_HB + (threadIdx.x & (PR_HB - 1));
        const int b0 = (hb / ng) * hr, b1 = b0 + hr < nblk ? b0 + hr : nblk;
        unsigned long long a = 0ull;
        if (bin < TB)
            for (int b = b0 + (int)(threadIdx.x >> 6); b < b1; b += 4 * PR_U) {
                unsigned long long x[PR_U];
#pragma unroll
                for (int u = 0; u < PR_U; ++u) x[u] = b + 4 * u < b1 ? hpart[(size_t)(b + 4 * u) * TB + bin] : 0ull;
#pragma unroll
                for (int u = 0; u < PR_U; ++u) a += x[u];
            }
        s_h[threadIdx.x >> 6][threadIdx.x & (PR_HB - 1)] = a;
        __syncthreads();
        if (threadIdx.x < PR_HB && bin < TB) {
            const unsigned long long t = s_h[0][threadIdx.x] + s_h[1][threadIdx.x] + s_h[2][threadIdx.x] + s_h[3][threadIdx.x];
            atomicAdd(&hist[(size_t)((hb / ng) % SP_HCOPIES) * TB + bin], t);
        }
        return;
    }
    // (+0.0 for the rows past nblk leaves the sum unchanged: a starts at +0.0,
    // so it is never -0.0)
    double a = 0.0;
    for (int b = threadIdx.x; b < nblk; b += 256 * PR_U) {
        double x[PR_U];
#pragma unroll
        for (int u = 0; u < PR_U; ++u) x[u] = b + 256 * u < nblk ? part[(size_t)(b + 256 * u) * VS + v] : 0.0;
#pragma unroll
        for (int u = 0; u < PR_U; ++u) a += x[u];
    }
    a = wave_total_d(a);
    if ((threadIdx.x & 63) == 63) s_w[threadIdx.x >> 6] = a;
    __syncthreads();
    if (threadIdx.x == 0) sums[v] = ((s_w[0] + s_w[1]) + s_w[2]) + s_w[3];
}



// ---------------------------------------------------------------------------
// S1: sum f^2 over contiguous chunks (float4 loads when aligned)
// ---------------------------------------------------------------------------
// Each block also clears its slice of the axis density sums (rows, then
// columns) for this step's sweep 2.
template <typename PT, typename GT, bool V4>
__global__ __launch_bounds__(SP_NT) void sweep1_kernel(
    Geom g, const GT* __restrict__ grad, const PT* __restrict__ param, double* __restrict__ part,
    unsigned long long* __restrict__ rowfx, unsigned long long* __restrict__ colfx, Ctrl* __restrict__ ctrl,
    const float* __restrict__ fr_state, Lanes L, cresso_hyper h) {
    if (L.dv) {
        const cresso_spectral_desc& d = lane_desc(L);
        grad = (const GT*)d.grad; param = (const PT*)d.param; fr_state = (const float*)d.force_rms;
    }
    part = lane_at(part, L); rowfx = lane_at(rowfx, L); colfx = lane_at(colfx, L); ctrl = lane_at(ctrl, L);
    __shared__ float red[4];
    if (blockIdx.x == 0 && threadIdx.x == 0) ctrl->fr_prev = *fr_state;   // every block of sweep 2 reads the old value
    {
        const int64_t na = g.rows + g.cols, per = (na + g.nblk1 - 1) / g.nblk1;
        const int64_t a0 = (int64_t)blockIdx.x * per, a1 = a0 + per < na ? a0 + per : na;
        for (int64_t i = a0 + threadIdx.x; i < a1; i += SP_NT) {
            if (i < g.rows)
                rowfx[i] = 0ull;
            else
                colfx[i - g.rows] = 0ull;
        }
    }
    const float wd = (float)h.weight_decay;
    const bool wd_on = h.weight_decay != 0.0;
    const int64_t beg = (int64_t)blockIdx.x * g.chunk1;
    const int64_t end = beg + g.chunk1 < g.n ? beg + g.chunk1 : g.n;
    const float sg = h.maximize ? -1.f : 1.f;
    float a = 0.f, m = 0.f;   // sum of f^2, max |f|
    // 64 elements per thread per iteration in flight: 16 float4 loads, or, for
    // 2-byte grads on a 16-byte aligned base, 8 16-byte loads (8 elements each)
    auto vec_loop = [&](auto vw) -> int64_t {
        constexpr int VW = decltype(vw)::value;
        constexpr int UN = 64 / VW;
        const int64_t vend = beg + ((end - beg) & ~(int64_t)(VW - 1));
        const int64_t st = VW * (int64_t)SP_NT;
        int64_t e = beg + VW * (int64_t)threadIdx.x;
        for (; e + (UN - 1) * st < vend; e += UN * st) {
            float f[UN][VW];
#pragma unroll
            for (int u = 0; u < UN; ++u) LdV<GT, VW>::go(grad, e + u * st, f[u]);
            if (wd_on) {
                float pv[UN][VW];
#pragma unroll
                for (int u = 0; u < UN; ++u) LdV<PT, VW>::go(param, e + u * st, pv[u]);
#pragma unroll
                for (int u = 0; u < UN; ++u)
#pragma unroll
                    for (int c = 0; c < VW; ++c) f[u][c] = sg * f[u][c] + wd * pv[u][c];
            }
#pragma unroll
            for (int u = 0; u < UN; ++u)
#pragma unroll
                for (int c = 0; c < VW; ++c) {
                    a += f[u][c] * f[u][c];
                    m = fmaxf(m, fabsf(f[u][c]));
                }
        }
        for (; e < vend; e += st) {
            float f[VW];
            LdV<GT, VW>::go(grad, e, f);
            if (wd_on) {
                float pv[VW];
                LdV<PT, VW>::go(param, e, pv);
#pragma unroll
                for (int c = 0; c < VW; ++c) f[c] = sg * f[c] + wd * pv[c];
            }
#pragma unroll
            for (int c = 0; c < VW; ++c) {
                a += f[c] * f[c];
                m = fmaxf(m, fabsf(f[c]));
            }
        }
        return vend;
    };
    int64_t vend = beg;
    if constexpr (V4) {
        // (chunks start at multiples of 8 elements)
        if (sizeof(GT) == 2 && ((uintptr_t)grad & 15) == 0 &&
            (!wd_on || sizeof(PT) != 2 || ((uintptr_t)param & 15) == 0))
            vend = vec_loop(std::integral_constant<int, 8>{});
        else
            vend = vec_loop(std::integral_constant<int, 4>{});
    }
    // scalar elements: the tail of a vectorized chunk, or the whole chunk
    for (int64_t i = vend + threadIdx.x; i < end; i += SP_NT) {
        float f = sg * ld(grad, i);
        if (wd_on) f = f + wd * ld(param, i);
        a += f * f;
        m = fmaxf(m, fabsf(f));
    }
    Partials P{red, 1, 1};
    P.add(0, a);
    P.flush(part, 2);
    // block max |f| after the block's sum (part[block][1]): max is order independent
    __shared__ float smax[SP_NT / 64];
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((threadIdx.x & 63) == 0) smax[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        float mm = smax[0];
        for (int i = 1; i < SP_NT / 64; ++i) mm = fmaxf(mm, smax[i]);
        part[(size_t)blockIdx.x * 2 + 1] = (double)mm;
    }
}



// F1, in every block of sweep 2: sweep 1's block partials summed in a fixed
// order (so every block gets the same values), then the force-RMS reservoir
// and the scale.  Block 0 stores the new force RMS and the values later
// kernels read from ctrl; the reservoir starts from ctrl->fr_prev (stashed by
// sweep 1), so no block reads a value another block of this launch writes.
// The density histogram's fixed-point scales come from sweep 1's block sums
// and maxima of f^2, |f| (each block's row of part1 holds its sum, then its
// maximum).
//
// Density histogram: every bin holds a low and a high 64-bit word, value =
// (low + high 2^k) / 2^F, each element adding y = rel^p 2^F.  Elements with
// y < 2^k add rint(y) to the low word (one LDS atomic per table, the common
// case); larger ones add floor(rel^p 2^-j) (j = k - F) to the high word and
// the exact remainder to the low word.  (The sweeps' loops add min(y, 2^k);
// a high-word pass, in the blocks hi_block finds can hold such an element,
// adds the rest: HiSplit.)  F, k, j are chosen so that
//   - the low words cannot overflow: either every element's y stays below
//     2^k <= 2^(62 - ceil log2 cmax) (cmax elements per bin at most), or F
//     is the single-word scale F0 for which a bin's whole sum stays below
//     2^61 (bounds below);
//   - the high words cannot overflow: sum rel^p 2^-j <= 2^60;
//   - ordinary elements stay in the low word: 2^j >= 2^16 times a typical
//     rel^p, from the mean of f^2 without each sweep-1 block's largest
//     element (so that a few spikes near the rel clamp, at a large energy
//     power, do not set the resolution of every other bin, as they do F0).
// F is never below F0, so the resolution is never coarser than one word's.
// When F0 alone resolves densities near 1 to 2^-36 (no large element set
// it), the high words stay off and the step pays nothing for them.
struct F1Values {
    float inv_s;
    double hs_ds;   // 2^F
    float yk, hq;   // 2^k, 2^-j
    float kmf;      // k - F
    bool hi_on;     // some element may reach the high words (rmax^p >= 2^(k - F))
};
// Sweep 1's block partials (sum, max) of one thread, blocks threadIdx.x +
// i SP_NT: the first N loaded at once (indices clamped, so that no branch
// separates the loads), summed later in block order.
template <int N>
struct F1Part {
    double s[N > 0 ? N : 1], m[N > 0 ? N : 1];
    __device__ __forceinline__ void load(const Geom& g, const double* __restrict__ part1) {
#pragma unroll
        for (int i = 0; i < N; ++i) {
            int b = (int)threadIdx.x + i * SP_NT;
            b = b < g.nblk1 ? b : g.nblk1 - 1;
            s[i] = part1[(size_t)b * 2];
            m[i] = part1[(size_t)b * 2 + 1];
        }
    }
};
template <int N>
__device__ F1Values fin1_values(const Geom& g, const F1Part<N>& fp, const double* __restrict__ part1,
                                Ctrl* __restrict__ ctrl, float* __restrict__ fr_state, int step, const cresso_hyper& h) {
    __shared__ double s_w[SP_NT / 64], s_m[SP_NT / 64];
    double a = 0.0, mx = 0.0;
#pragma unroll
    for (int i = 0; i < N; ++i)
        if ((int)threadIdx.x + i * SP_NT < g.nblk1) {
            a += fp.s[i];
            mx = fmax(mx, fp.m[i]);
        }
    for (int b = threadIdx.x + N * SP_NT; b < g.nblk1; b += SP_NT) {
        a += part1[(size_t)b * 2];
        mx = fmax(mx, part1[(size_t)b * 2 + 1]);
    }
    const double w = wave_total_d(a);
    for (int o = 32; o > 0; o >>= 1) mx = fmax(mx, __shfl_xor(mx, o));
    if ((threadIdx.x & 63) == 63) s_w[threadIdx.x >> 6] = w;
    if ((threadIdx.x & 63) == 0) s_m[threadIdx.x >> 6] = mx;
    __syncthreads();
    double sum = 0.0;
    for (int i = 0; i < SP_NT / 64; ++i) {
        sum += s_w[i];
        mx = fmax(mx, s_m[i]);
    }
    const float eps = (float)h.eps;
    const float now = sqrtf((float)(sum / (double)g.n) + eps);
    const float fr = reservoir_f(ctrl->fr_prev, now, h.reservoir_decay, step);
    const float sc = fmaxf(fr, eps);
    F1Values v;
    v.inv_s = 1.0f / sc;
    // Single-word scale F0: every bin's sum of ds = rel^p, rel = min(|f|/s +
    // eps, 1e4), times 2^F0 stays below 2^61 (rounding adds at most half a
    // unit per element).  A bin's sum is at most the smaller of
    //   cmax rmax^p                                 (cmax elements, each <= rmax^p)
    //   sum_i rel_i^p <= rmax^(p-2) S2              (p >= 2)
    //                 <= n^(1-p/2) S2^(p/2)         (p < 2, power means)
    // with S2 = sum_i rel_i^2 <= sum f^2/s^2 + 2 eps sqrt(n sum f^2)/s + n eps^2
    // from sweep 1's sums; the smaller bound (l2b, log2) also bounds the
    // whole histogram's sum, which sizes the high words.
    // (fp32 hardware log2 with margins for it and for the sweep's exp2/log2 of
    // rel^p; every block computes the same values)
    const float rmax = fminf(fmaf((float)mx, v.inv_s, eps), 1.0e4f);
    const float pw = (float)h.energy_power;
    const float lr = flog2(rmax);
    const double is = (double)v.inv_s, dn = (double)g.n;
    const double s2 = (sum * is * is + 2.0 * (double)eps * is * sqrt(dn * sum) + dn * (double)eps * (double)eps) * 1.001;
    const float l2s = flog2((float)s2 + 1.0e-30f);
    const float l2tot = pw >= 2.0f ? (pw - 2.0f) * lr + l2s : (1.0f - 0.5f * pw) * flog2((float)dn) + 0.5f * pw * l2s;
    const float l2bin = pw * lr + flog2((float)ctrl->cmax);
    const float l2b = fminf(l2bin, l2tot);
    // (exponents clamped as floats, so that infinite or NaN bounds convert)
    const int f0 = (int)fminf(fmaxf(floorf(61.0f - l2b - 0.05f), -120.0f), 120.0f);
    // The single word keeps 2^-36 resolution at ds = 1 or finer (rel is
    // normalized by the force RMS, so ordinary densities are near 1): high
    // words off (k = 62, which no element reaches under F0).  A coarser F0
    // means a large element set it: the two-word scale, with the low words'
    // limit 2^kq and the high words' weight 2^j.  (f0 is the same in every
    // block, so every block takes the same branch.)
    int F = f0, k = 62, j = 62 - f0;
    if (f0 < 36) {
        // sum f^2 without each sweep-1 block's largest element, in block order
        __shared__ double s_x[SP_NT / 64];
        double ax = 0.0;
#pragma unroll
        for (int i = 0; i < N; ++i)
            if ((int)threadIdx.x + i * SP_NT < g.nblk1) ax += fmax(fp.s[i] - fp.m[i] * fp.m[i], 0.0);
        for (int b = threadIdx.x + N * SP_NT; b < g.nblk1; b += SP_NT) {
            const double mb = part1[(size_t)b * 2 + 1];
            ax += fmax(part1[(size_t)b * 2] - mb * mb, 0.0);
        }
        const double wx = wave_total_d(ax);
        if ((threadIdx.x & 63) == 63) s_x[threadIdx.x >> 6] = wx;
        __syncthreads();
        double sumx = 0.0;
        for (int i = 0; i < SP_NT / 64; ++i) sumx += s_x[i];
        const int kq = ctrl->kq;
        const float rtyp = sqrtf((float)(sumx * g.inv_n)) * v.inv_s + eps;   // typical rel
        j = (int)fminf(fmaxf(ceilf(fmaxf(pw * flog2(rtyp) + 16.0f, l2b - 60.0f + 0.05f)), -100.0f), 100.0f);
        F = kq - j > f0 ? kq - j : f0;
        F = F < 120 ? F : 120;   // 2^F stays a finite fp32 value
        k = F + j < 62 ? F + j : 62;
    }
    v.hs_ds = ldexp(1.0, F);
    v.yk = ldexpf(1.0f, k);
    v.hq = ldexpf(1.0f, -j);
    // the sweeps test elements against 2^k only when the largest one can
    // reach it (margin 0.05 in log2 units for the hardware log2/exp2 of rel^p)
    v.kmf = (float)(k - F);
    v.hi_on = pw * lr + 0.05f >= v.kmf;
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        *fr_state = fr;
        ctrl->scale = sc;
        ctrl->inv_s = v.inv_s;
        ctrl->hs_ds = v.hs_ds;   // fin2 converts the histogram back with these
        ctrl->hs_hi = ldexp(1.0, j);
    }
    return v;
}
__device__ __forceinline__ F1Values fin1_values(const Geom& g, const double* __restrict__ part1, Ctrl* __restrict__ ctrl,
                                                float* __restrict__ fr_state, int step, const cresso_hyper& h) {
    return fin1_values<0>(g, F1Part<0>{}, part1, ctrl, fr_state, step, h);
}

// ---------------------------------------------------------------------------
// reconstruction weights of a lane's column
// ---------------------------------------------------------------------------
// A reconstruction sum_r (wc_r Craw_r + ws_r Sraw_r) + const equals
// sum_x a_x(row) gam_x(col) + const with the row factors a_{2r} = a1_r,
// a_{2r+1} = a2_r of the row table and, per column,
//   additive kinds:     gam_{2r} = wc b_k1 + ws b_k2, gam_{2r+1} = ws b_k1 - wc b_k2
//   product / constant: gam_{2r} = wc b_k1,           gam_{2r+1} = ws b_k2
// (C = a1 b1 - a2 b2, S = a2 b1 + a1 b2, resp. C = a1 b1, S = a2 b2).
// The sweeps read the row factors of the row all lanes share as scalars.
template <int RM, int KC>
__device__ __forceinline__ void recon_weights(const Geom& g, const ModeMeta* __restrict__ meta, const float (&b)[KC],
                                              const float (*rc)[2], float (&gam)[2 * RM]) {
#pragma unroll
    for (int r = 0; r < RM; ++r) {
        float g1 = 0.f, g2 = 0.f;
        if (r < g.R) {
            const ModeMeta m = meta[r];
            float b1 = 0.f, b2 = 0.f;
#pragma unroll
            for (int k = 0; k < KC; ++k) {
                if (k == m.k1) b1 = b[k];
                if (k == m.k2) b2 = b[k];
            }
            const float wc = rc[r][0], ws = rc[r][1];
            if (m.type == M_ADD) {
                g1 = wc * b1 + ws * b2;
                g2 = ws * b1 - wc * b2;
            } else {
                g1 = wc * b1;
                g2 = ws * b2;
            }
        }
        gam[2 * r] = g1;
        gam[2 * r + 1] = g2;
    }
}

// Lane's column carriers (the table has 2*rmax+1 rows, zero beyond K).
template <int KC>
__device__ __forceinline__ void load_cols(const Geom& g, const float* __restrict__ coltab, const Tile& t, float (&b)[KC]) {
#pragma unroll
    for (int k = 0; k < KC; ++k) b[k] = t.colok ? coltab[(size_t)k * g.cols + t.col] : 0.f;
}

// Row coefficients of two reconstructions in the column-carrier form
//   recon(row, col) = c + sum_k alpha_k(row) b_k(col)
// (b_k: the lane's column carriers, b_0 = 1), for the block's nr rows: the
// per-lane form sum_q a_q(row) gamma_q(col) has 2R terms, this one K.  Set
// j's mode coefficients are w0[j] rc0[j] + w1[j] rc1[j] (rc1 may be null).
// The block's row factors arrive staged in LDS (s_rows[lr][q], q < 2 RM).
// Loops of dependent reads per entry (global or LDS) cost microseconds per
// block at the start of a sweep, so the computation is a small dense product
// with independent reads.  Ends with a barrier.
// Out: s_al[lr][j][k], row stride 2 * KCP (KCP = KC rounded up to 4).
template <int KC> constexpr int kcp() { return (KC + 3) & ~3; }
// byte offset of sweep 3's row coefficients in its dynamic LDS
__host__ __device__ inline size_t lds_al_off(const Geom& g) {
    const size_t head = (sizeof(unsigned long long) * SP_NHIST + sizeof(float)) * (size_t)g.T * g.B +
                        sizeof(float) * (size_t)g.PR;
    return (head + 15) & ~(size_t)15;
}
// The reconstruction coefficients alpha_rows builds from: every Cm entry a
// thread writes has the same q = threadIdx.x mod 2 RM (blocks of SP_NT
// threads, a multiple of 2 RM), so the thread needs one mode-table entry and
// the weights of mode q / 2 in both sets.  Loaded first thing, with the
// block's other set-up loads, so that they return in one round trip.
struct CmSrc {
    int on, add, k1, k2;
    float wc[2], ws[2];
};
template <int RM>
__device__ __forceinline__ CmSrc cm_src(const Geom& g, const ModeMeta* __restrict__ meta,
                                        const float (*const rc0[2])[2], const float w0[2],
                                        const float (*const rc1[2])[2], const float w1[2]) {
    constexpr int RW = 2 * RM;
    static_assert(SP_NT % RW == 0, "one projection row per thread residue");
    const int r = (int)(threadIdx.x % RW) >> 1;
    const int rr = r < g.R ? r : 0;
    CmSrc c;
    const ModeMeta m = meta[rr];
    c.on = r < g.R;
    c.add = m.type == M_ADD;
    c.k1 = m.k1;
    c.k2 = m.k2;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        // the second set's loads are issued either way (from the first set,
        // weighted 0, where it is absent: the coefficients are finite): a
        // load inside a branch would wait at once for every load before it
        const float (*const p1)[2] = rc1[j] ? rc1[j] : rc0[j];
        const float v1 = rc1[j] ? w1[j] : 0.f;
        c.wc[j] = fmaf(v1, p1[rr][0], w0[j] * rc0[j][rr][0]);
        c.ws[j] = fmaf(v1, p1[rr][1], w0[j] * rc0[j][rr][1]);
    }
    return c;
}

template <int RM, int KC>
__device__ void alpha_rows(const Geom& g, const CmSrc& cs, const float* __restrict__ s_rows, int nr,
                           float* __restrict__ s_al) {
    // alpha = rows x Cm^T: Cm[j][k][q] is the coefficient of the row factor
    // a_q (q = 2r + c: component c of mode r) in alpha_k of set j.  Every Cm
    // entry is built by its own thread from the mode table; each (row, set)
    // pair is then 2 RM x KP branch-free FMAs on values held in registers.
    constexpr int KP = kcp<KC>();
    constexpr int RW = 2 * RM;
    constexpr int NE = 2 * KP * RW;
    __shared__ __align__(16) float s_cm[2][KP][RW];
    const int q = (int)(threadIdx.x % RW), c = q & 1;
#pragma unroll
    for (int i = 0; i < (NE + SP_NT - 1) / SP_NT; ++i) {
        const int e = (int)threadIdx.x + i * SP_NT;
        if (e < NE) {
            const int j = e / (KP * RW), k = (e - j * (KP * RW)) / RW;
            const float wc = j ? cs.wc[1] : cs.wc[0], ws = j ? cs.ws[1] : cs.ws[0];
            float v = 0.f;
            if (cs.on && k < KC) {
                if (cs.add) {   // alpha_k1 += wc a1 + ws a2, alpha_k2 += ws a1 - wc a2
                    if (cs.k1 == k) v += c == 0 ? wc : ws;
                    if (cs.k2 == k) v += c == 0 ? ws : -wc;
                } else {        // alpha_k1 += wc a1, alpha_k2 += ws a2
                    if (cs.k1 == k && c == 0) v += wc;
                    if (cs.k2 == k && c == 1) v += ws;
                }
            }
            s_cm[j][k][q] = v;
        }
    }
    __syncthreads();   // Cm and the caller's staged rows are complete
    // (row, set, half of the carriers) per thread: 4 nr items, all threads busy
    constexpr int KH = KP / 2;
    for (int p = threadIdx.x; p < 4 * nr; p += blockDim.x) {
        const int lr = p >> 2, j = (p >> 1) & 1, k0 = (p & 1) * KH;
        float row[RW];
#pragma unroll
        for (int q = 0; q < RW; ++q) row[q] = s_rows[lr * RW + q];
        float* __restrict__ out = s_al + lr * (2 * KP) + j * KP + k0;
#pragma unroll
        for (int k = 0; k < KH; ++k) {
            float a = 0.f;
#pragma unroll
            for (int q = 0; q < RW; ++q) a = fmaf(s_cm[j][k0 + k][q], row[q], a);
            out[k] = a;
        }
    }
    __syncthreads();
}
template <int RM, int KC>
__device__ void alpha_rows(const Geom& g, const ModeMeta* __restrict__ meta, const float* __restrict__ s_rows, int nr,
                           const float (*const rc0[2])[2], const float w0[2], const float (*const rc1[2])[2],
                           const float w1[2], float* __restrict__ s_al) {
    alpha_rows<RM, KC>(g, cm_src<RM>(g, meta, rc0, w0, rc1, w1), s_rows, nr, s_al);
}

// alpha on the matrix cores (the matrix-core sweeps):
//   alpha[j][row][k] = sum_q rows[row][q] Cm[j][k][q]
// as v_mfma_f32_16x16x4f32 over 16-row and 16-carrier tiles.  In step s of a
// tile, lane (li, lg) holds q = QPL lg + s (QPL = 2 RM / 4 values of q a
// lane): A[i][k] = rows[16 rt + li][q], B[k][j] = Cm[j][16 kt + li][q] built
// in registers from the lane's modes q / 2 (CmLane, loaded with the block's
// other set-up loads), so the Cm table needs no LDS and no barrier.
typedef float f32x4m __attribute__((ext_vector_type(4)));
template <int RM>
struct CmLane {
    static constexpr int QPL = RM / 2;
    static constexpr int NM = QPL / 2;   // modes a lane (QPL is even: RM >= 4)
    int on[NM], add[NM], k1[NM], k2[NM];
    float wc[NM][2], ws[NM][2];
};
template <int RM>
__device__ __forceinline__ CmLane<RM> cm_lane(const Geom& g, const ModeMeta* __restrict__ meta,
                                              const float (*const rc0[2])[2], const float w0[2],
                                              const float (*const rc1[2])[2], const float w1[2]) {
    constexpr int QPL = CmLane<RM>::QPL, NM = CmLane<RM>::NM;
    static_assert(RM >= 4 && RM % 4 == 0, "even q count a lane");
    const int lg = (int)(threadIdx.x & 63) >> 4;
    CmLane<RM> c;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        const int r = (QPL * lg) / 2 + m;
        const int rr = r < g.R ? r : 0;
        const ModeMeta mm = meta[rr];
        c.on[m] = r < g.R;
        c.add[m] = mm.type == M_ADD;
        c.k1[m] = mm.k1;
        c.k2[m] = mm.k2;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            // as cm_src: the second set's loads issued either way
            const float (*const p1)[2] = rc1[j] ? rc1[j] : rc0[j];
            const float v1 = rc1[j] ? w1[j] : 0.f;
            c.wc[m][j] = fmaf(v1, p1[rr][0], w0[j] * rc0[j][rr][0]);
            c.ws[m][j] = fmaf(v1, p1[rr][1], w0[j] * rc0[j][rr][1]);
        }
    }
    return c;
}
template <int RM, int KC>
__device__ void alpha_rows_m(const Geom& g, const CmLane<RM>& cl, const float* __restrict__ s_rows, int nr,
                             float* __restrict__ s_al) {
    constexpr int KP = kcp<KC>();
    constexpr int RW = 2 * RM;
    constexpr int QPL = CmLane<RM>::QPL;
    constexpr int NKT = (KP + 15) / 16;
    __syncthreads();   // the staged rows are complete
    const int l = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int li = l & 15, lg = l >> 4;
    const int ntr = nr / 16;
    // (row tile, set) items over the block's waves (wave-uniform loop)
    for (int it = wv; it < 2 * ntr; it += SP_NT / 64) {
        const int rt = it >> 1, j = it & 1;
        float a[QPL];
#pragma unroll
        for (int s = 0; s < QPL; ++s) a[s] = s_rows[(16 * rt + li) * RW + QPL * lg + s];
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt) {
            const int k = 16 * kt + li;
            f32x4m d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < QPL; ++s) {
                const int m = s >> 1, c = s & 1;
                const float wc = j ? cl.wc[m][1] : cl.wc[m][0], ws = j ? cl.ws[m][1] : cl.ws[m][0];
                float v = 0.f;
                if (cl.on[m] && k < KC) {
                    if (cl.add[m]) {   // alpha_k1 += wc a1 + ws a2, alpha_k2 += ws a1 - wc a2
                        if (cl.k1[m] == k) v += c == 0 ? wc : ws;
                        if (cl.k2[m] == k) v += c == 0 ? ws : -wc;
                    } else {           // alpha_k1 += wc a1, alpha_k2 += ws a2
                        if (cl.k1[m] == k && c == 0) v += wc;
                        if (cl.k2[m] == k && c == 1) v += ws;
                    }
                }
                d = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], v, d, 0, 0, 0);
            }
            // D[i][j'] in lane j' = li (carrier k), register r: row 16 rt + 4 lg + r
            if (k < KP) {
#pragma unroll
                for (int r = 0; r < 4; ++r) s_al[(16 * rt + 4 * lg + r) * (2 * KP) + j * KP + k] = d[r];
            }
        }
    }
    __syncthreads();
}

// The block's rows of the row-factor table into LDS: s_rows[lr][q], q < 2 RM
// (the table's rows have g.RW >= 2 RM entries).  No barrier.
template <int RM>
__device__ __forceinline__ void stage_rows(const Geom& g, const float* __restrict__ rowtab, int64_t r0, int nr,
                                           float* __restrict__ s_rows) {
    constexpr int RW = 2 * RM;
    for (int e = threadIdx.x; e < nr * RW; e += blockDim.x) {
        const int lr = e / RW, q = e - lr * RW;
        s_rows[e] = rowtab[(r0 + lr) * g.RW + q];
    }
}

// Set-up loads of the matrix-core sweeps, in two halves: load() issues every
// global load of a staged table at once (addresses clamped into the table,
// so that no branch separates them and one wait covers them all), store()
// writes the values to LDS.  Up to N values per thread; a larger table takes
// its remainder in a loop (never on the matrix-core path: panels of 32 or 64
// rows, at most 4 tables of 256 bins).
template <int N>
struct Staged {
    float v[N];
    __device__ __forceinline__ void load(const float* __restrict__ src, int n) {
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const int e = (int)threadIdx.x + i * SP_NT;
            v[i] = src[e < n ? e : n - 1];
        }
    }
    // row lr of the row-factor table: 2 RM entries of a row of g.RW
    template <int RM>
    __device__ __forceinline__ void load_rows(const Geom& g, const float* __restrict__ rowtab, int64_t r0, int nr) {
        constexpr int RW = 2 * RM;
        const int n = nr * RW;
#pragma unroll
        for (int i = 0; i < N; ++i) {
            int e = (int)threadIdx.x + i * SP_NT;
            e = e < n ? e : n - 1;
            const int lr = e / RW, q = e - lr * RW;
            v[i] = rowtab[(r0 + lr) * g.RW + q];
        }
    }
    template <typename F>
    __device__ __forceinline__ void store(float* __restrict__ dst, int n, F&& f) const {
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const int e = (int)threadIdx.x + i * SP_NT;
            if (e < n) dst[e] = f(v[i]);
        }
    }
    __device__ __forceinline__ void store(float* __restrict__ dst, int n) const {
        store(dst, n, [](float x) { return x; });
    }
};
// the remainder of a table longer than N values a thread
template <int N, typename F>
__device__ __forceinline__ void stage_rest(float* __restrict__ dst, const float* __restrict__ src, int n, F&& f) {
    for (int e = (int)threadIdx.x + N * SP_NT; e < n; e += SP_NT) dst[e] = f(src[e]);
}
template <int RM, int N>
__device__ __forceinline__ void stage_rows_rest(const Geom& g, const float* __restrict__ rowtab, int64_t r0, int nr,
                                                float* __restrict__ s_rows) {
    constexpr int RW = 2 * RM;
    for (int e = (int)threadIdx.x + N * SP_NT; e < nr * RW; e += SP_NT) {
        const int lr = e / RW, q = e - lr * RW;
        s_rows[e] = rowtab[(r0 + lr) * g.RW + q];
    }
}

// Lane contribution of a projection: Z[2q] = sum over the lane's rows of
// a1_q(row) x, Z[2q+1] = the same with a2_q; combined with the lane's column
// carriers into the raw C/S projections of every mode, partial slots
// base + 2r (C) and base + 2r + 1 (S).
template <int RM, int KC>
__device__ __forceinline__ void proj_finish(const Geom& g, const ModeMeta* __restrict__ meta, const float (&Z)[2 * RM],
                                            const float (&b)[KC], Partials& P, int base) {
#pragma unroll
    for (int r = 0; r < RM; ++r) {
        if (r < g.R) {
            const ModeMeta m = meta[r];
            float b1 = 0.f, b2 = 0.f;
#pragma unroll
            for (int k = 0; k < KC; ++k) {
                if (k == m.k1) b1 = b[k];
                if (k == m.k2) b2 = b[k];
            }
            float c, sn;
            if (m.type == M_ADD) {
                c = b1 * Z[2 * r] - b2 * Z[2 * r + 1];
                sn = b1 * Z[2 * r + 1] + b2 * Z[2 * r];
            } else {
                c = b1 * Z[2 * r];
                sn = b2 * Z[2 * r + 1];
            }
            P.add(base + 2 * r, c);
            P.add(base + 2 * r + 1, sn);
        }
    }
}

// Instant-metric factor of an axis marginal (cresso_v5.py:243-262):
// exp(kappa * log(max(mean/gden, eps))), mean from a fixed-point sum;
// inv_hc = 1 / (hs * count), hs the sum's power-of-two scale.
__device__ __forceinline__ float marg_factor(unsigned long long fx, double inv_hc, float gden, float kappa, float eps) {
    const float mean = (float)((double)fx * inv_hc);
    return fexp2(kappa * flog2(fmaxf(mean / gden, eps)));
}

constexpr int SP_U = 8;  // rows whose loads are in flight together

// Keeps the scheduler from interleaving the arithmetic of consecutive
// elements (their loads are already in flight): bounds register pressure.
__device__ __forceinline__ void elem_fence() { __builtin_amdgcn_sched_barrier(0); }

// Element addressing inside a block's panel: the element index of the panel's
// first element (row r0, first column of the slab) is uniform, so each array
// is addressed as (uniform base pointer) + (32-bit lane offset lr * cols +
// lane); the planner keeps PR * cols below 2^29.
__device__ __forceinline__ int64_t panel_base(const Geom& g, const Tile& t) { return t.r0 * g.cols + (int64_t)t.slab * SP_NT; }
// The tangent / drive field after the matrix-core sweeps, 4-row interleaved:
// element (R, C) at 4 ((R / 4) cols + C) + R % 4 (rows are a multiple of 4 on
// that path).  A block's elements (r0 + i, c0 + j) then sit at
// q4_base + 4 ((i / 4) cols + j) + i % 4, and the four rows 4 lg + r of a
// lane's tile column are one float4.
__device__ __forceinline__ int64_t q4_base(const Geom& g, const Tile& t) {
    return t.r0 * g.cols + 4 * (int64_t)t.slab * SP_NT;
}
__device__ __forceinline__ uint32_t q4_lane_bytes(uint32_t cols, int lg, int wv, int li) {
    return 16u * ((uint32_t)lg * cols + 64u * (uint32_t)wv + (uint32_t)li);
}
__device__ __forceinline__ uint32_t q4_tile_bytes(uint32_t cols, int tr, int tc) {
    return 16u * (4u * (uint32_t)tr * cols + 16u * (uint32_t)tc);
}
__device__ __forceinline__ uint32_t panel_off(const Geom& g, int lr) { return (uint32_t)lr * (uint32_t)g.cols + threadIdx.x; }
__device__ __forceinline__ uint64_t load_bins_at(const unsigned char* __restrict__ bins, int64_t base, uint32_t off,
                                                 int binbytes) {
    switch (binbytes) {
        case 1: return (bins + base)[off];
        case 2: return (reinterpret_cast<const uint16_t*>(bins) + base)[off];
        case 4: return (reinterpret_cast<const uint32_t*>(bins) + base)[off];
        default: return (reinterpret_cast<const uint64_t*>(bins) + base)[off];
    }
}

// A value every thread of the wave holds, moved to a scalar register.
__device__ __forceinline__ float uniform_f(float x) {
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x)));
}
// Density of one element: rel = min(|f|/s + eps, 1e4), f = sign grad (+
// weight decay param), and ds = rel^p.  The full-tile form (no weight decay,
// instant-metric power 1) writes rel with one fma.  A sweep computes an
// element's density with the same helpers in its loop and again in its
// high-word pass, which must reproduce the loop's values exactly.
__device__ __forceinline__ float force_of(float gv, float pv, float sg, float wd, bool wd_on) {
    float f = sg * gv;
    if (wd_on) f = f + wd * pv;
    return f;
}
__device__ __forceinline__ float rel_gen(float f, float inv_s, float eps) { return fminf(fabsf(f) * inv_s + eps, 1.0e4f); }
__device__ __forceinline__ float rel_full(float x, float inv_s, float eps) { return fminf(fmaf(fabsf(x), inv_s, eps), 1.0e4f); }
// An element whose y = ds 2^F reached 2^k: the sweep's loop added 2^k
// (lo_k, y clamped) to its low word; the high-word pass adds the high word
// floor(q), q = ds 2^-j, and (q - floor q) 2^k - 2^k to the low word (mod
// 2^64: the bin's final low sum is in range, so the wrapped partial sums
// come out exact).  Both parts are exact in fp32 (scalings by powers of two,
// the fraction of q).
struct HiSplit {
    unsigned long long hi, lo;
};
__device__ __forceinline__ HiSplit hi_split(float ds, float hq, float yk, unsigned long long lo_k) {
    const float q = ds * hq, qi = floorf(q);
    return HiSplit{to_fixed_u(qi), to_fixed_u((q - qi) * yk) - lo_k};
}

// Whether a block's elements may include one whose y reached 2^k: sweep 1's
// maxima of |f| over the chunks that the block's flat index range [base,
// base + (nr - 1) cols + SP_NT) touches, with hi_on's margin.  A spike thus
// sends the blocks of its panel rows (not every block) through the
// high-word pass.  Every thread of the block calls it (a barrier).
__device__ __forceinline__ bool hi_block(const Geom& g, const double* __restrict__ part1, int64_t base, int nr,
                                         float inv_s, float eps, float pw, float kmf) {
    const int64_t c0 = base / g.chunk1;
    int64_t c1 = (base + (int64_t)(nr - 1) * g.cols + SP_NT - 1) / g.chunk1;
    c1 = c1 < g.nblk1 - 1 ? c1 : g.nblk1 - 1;
    int hit = 0;
    for (int64_t c = c0 + threadIdx.x; c <= c1; c += SP_NT)
        hit |= pw * flog2(rel_full((float)part1[c * 2 + 1], inv_s, eps)) + 0.05f >= kmf ? 1 : 0;
    return __syncthreads_or(hit) != 0;
}

// Panel arrays of a full tile as buffer views: one descriptor per array (the
// panel's first element as base), the lane's column as the VGPR offset and the
// row as a uniform SGPR offset, so the row loop needs no address arithmetic.
// Byte sizes stay below 2^31 (the planner keeps PR * cols below 2^29).
struct PanelBuf {
    __amdgpu_buffer_rsrc_t r;
    uint32_t lane;   // byte offset of the lane's column
    uint32_t row;    // bytes per row
};
template <typename T>
__device__ __forceinline__ PanelBuf panel_buf(const T* panel0, const Geom& g, int nr) {
    PanelBuf b;
    b.r = make_rsrc(panel0, (uint32_t)((int64_t)nr * g.cols * (int64_t)sizeof(T)));
    b.lane = (uint32_t)(threadIdx.x * sizeof(T));
    b.row = (uint32_t)(g.cols * sizeof(T));
    return b;
}
template <typename T> __device__ __forceinline__ float ldb_lane(const PanelBuf& b, int lr);
template <> __device__ __forceinline__ float ldb_lane<float>(const PanelBuf& b, int lr) {
    return bload1(b.r, b.lane, (uint32_t)lr * b.row);
}
template <> __device__ __forceinline__ float ldb_lane<__half>(const PanelBuf& b, int lr) {
    return to_f(__builtin_bit_cast(__half, (unsigned short)bload1u16(b.r, b.lane, (uint32_t)lr * b.row)));
}
template <> __device__ __forceinline__ float ldb_lane<__hip_bfloat16>(const PanelBuf& b, int lr) {
    return to_f(__builtin_bit_cast(__hip_bfloat16, (unsigned short)bload1u16(b.r, b.lane, (uint32_t)lr * b.row)));
}
template <> __device__ __forceinline__ float ldb_lane<double>(const PanelBuf& b, int lr) {
    return (float)__builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(b.r, b.lane, (uint32_t)lr * b.row, 0));
}
__device__ __forceinline__ uint32_t ldb_bins16(const PanelBuf& b, int lr) {
    return bload1u16(b.r, b.lane, (uint32_t)lr * b.row);
}
__device__ __forceinline__ void stb_lane(const PanelBuf& b, int lr, float v) {
    bstore1(b.r, b.lane, (uint32_t)lr * b.row, v);
}

// Rows of a full panel in batches of U: the loads of batch i+1 are issued
// before batch i is processed (two register sets, no copies).  nr is a
// multiple of 2U.  load(lr, x, b) loads row lr's lane values, body(lr, x, b)
// processes them.
// The same with a per-batch body: batch(i0, x[U], b[U]) processes rows i0..i0+U-1.
// xa/ba hold the first batch, loaded by the caller (at the top of the kernel,
// so that its latency overlaps the block's set-up).
template <int U, typename Load, typename Batch>
__device__ __forceinline__ void pipelined_batches(int nr, Load&& load, Batch&& batch, float (&xa)[U],
                                                  uint32_t (&ba)[U]) {
    float xb[U];
    uint32_t bb[U];
    for (int i0 = 0; i0 < nr; i0 += 2 * U) {
#pragma unroll
        for (int u = 0; u < U; ++u) load(i0 + U + u, xb[u], bb[u]);
        batch(i0, xa, ba);
        if (i0 + 2 * U < nr) {
#pragma unroll
            for (int u = 0; u < U; ++u) load(i0 + 2 * U + u, xa[u], ba[u]);
        }
        batch(i0 + U, xb, bb);
    }
}
template <int U, typename Load, typename Body>
__device__ __forceinline__ void pipelined_rows(int nr, Load&& load, Body&& body, float (&xa)[U], uint32_t (&ba)[U]) {
    pipelined_batches<U>(
        nr, load,
        [&](int i0, const float* x, const uint32_t* b) {
#pragma unroll
            for (int u = 0; u < U; ++u) body(i0 + u, x[u], b[u]);
        },
        xa, ba);
}

// Sums of 8 per-lane values (rows i0..i0+7 of the lane's column) over the 16
// lanes of each DPP row: lane l returns row (l & 7)'s partial (lanes l and
// l ^ 8 hold the same sum).  Lanes pair xor 1, 2, 4 while the values halve
// (each lane keeps the rows of its own bit and receives them from its
// partner), then xor 8: 25 instructions instead of 8 full wave reductions.
// DPP row_ror:n reads lane (l - n) mod 16, so xor 4 is ror 4 for lanes with
// bit 2 set and ror 12 for the others.
template <int CTRL> __device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float rows8_lanesum16(const float (&v)[8]) {
    const int l = threadIdx.x & 63;
    const bool b0 = (l & 1) != 0, b1 = (l & 2) != 0, b2 = (l & 4) != 0;
    float w4[4], w2[2];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float keep = b0 ? v[2 * j + 1] : v[2 * j], give = b0 ? v[2 * j] : v[2 * j + 1];
        w4[j] = keep + dpp_mov<0xB1>(give);   // quad_perm [1,0,3,2]: xor 1
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const float keep = b1 ? w4[2 * j + 1] : w4[2 * j], give = b1 ? w4[2 * j] : w4[2 * j + 1];
        w2[j] = keep + dpp_mov<0x4E>(give);   // quad_perm [2,3,0,1]: xor 2
    }
    const float keep = b2 ? w2[1] : w2[0], give = b2 ? w2[0] : w2[1];
    const float from_below = dpp_mov<0x124>(give);   // row_ror:4  -> lane l - 4
    const float from_above = dpp_mov<0x12C>(give);   // row_ror:12 -> lane l + 4
    float w1 = keep + (b2 ? from_below : from_above);
    w1 += dpp_mov<0x128>(w1);                        // row_ror:8: xor 8
    return w1;
}

// Sweep variants: MODE 1 is the common large-matrix case with every option
// fixed at compile time (2-D tensor, instant metric on, two hash tables of at
// most 256 bins, no weight decay, no local sharpness); MODE 0 handles every
// other combination with runtime flags.
struct SweepFlags {
    bool hash_on, axes_on, wd_on, ls_on;
    int T, bpb, binbytes;
};
template <int MODE>
__device__ __forceinline__ SweepFlags sweep_flags(const Geom& g, int hash_arg, int axes_arg, const cresso_hyper& h) {
    SweepFlags f;
    if (MODE == 1) {
        f.hash_on = true; f.axes_on = true; f.wd_on = false; f.ls_on = false;
        f.T = 2; f.bpb = 1; f.binbytes = 2;
    } else {
        f.hash_on = hash_arg != 0; f.axes_on = axes_arg != 0;
        f.wd_on = h.weight_decay != 0.0; f.ls_on = h.local_sharpness != 0.0;
        f.T = g.T; f.bpb = g.bpb; f.binbytes = g.binbytes;
    }
    return f;
}
// whether a tensor's step can use MODE 1 (host side)
// (MODE 1 also needs full tiles: every row of every panel and every lane's
// column valid, and panels of a multiple of 4 SP_U rows for the row pipelines.)
inline bool fast_mode(const Geom& g, int hash_on, int axes_on, const cresso_hyper& h) {
    return hash_on && axes_on && g.T == 2 && g.bpb == 1 && g.binbytes == 2 && !g.one_d && h.weight_decay == 0.0 &&
           h.local_sharpness == 0.0 && (float)fmax(h.instant_metric_power, 0.25) == 1.0f && g.rows % g.PR == 0 &&
           g.cols % SP_NT == 0 && g.PR % (4 * SP_U) == 0;
}
// tables the matrix-core sweeps take: 2 or 4 tables of one-byte bins, packed
__host__ __device__ inline bool mtables(const Geom& g) {
    return (g.T == 2 || g.T == 4) && g.bpb == 1 && g.binbytes == g.T;
}
// The environment variable CRESSO_SPECTRAL_MATRIX_CORES=0 turns the
// matrix-core sweeps off (the general sweeps run instead, same results within
// rounding): a measurement switch for comparing the two forms on one build.
inline bool matrix_cores_enabled() {
    static const bool on = [] {
        const char* v = std::getenv("CRESSO_SPECTRAL_MATRIX_CORES");
        return !(v && v[0] == '0' && v[1] == 0);
    }();
    return on;
}
// whether a tensor's step can use the matrix-core sweeps (host side): MODE 1's
// conditions with 2 or 4 tables
inline bool mfast_mode(const Geom& g, int hash_on, int axes_on, const cresso_hyper& h) {
    return hash_on && axes_on && mtables(g) && !g.one_d && h.weight_decay == 0.0 && h.local_sharpness == 0.0 &&
           (float)fmax(h.instant_metric_power, 0.25) == 1.0f && g.rows % g.PR == 0 && g.cols % SP_NT == 0 &&
           g.PR % (4 * SP_U) == 0 && matrix_cores_enabled();
}

// ---------------------------------------------------------------------------
// S2: density field
// ---------------------------------------------------------------------------
template <int RM, int KC, typename PT, typename GT, int MODE>
__global__ __launch_bounds__(SP_NT, RM >= 16 ? 2 : 4) void sweep2_kernel(
    Geom g, const GT* __restrict__ grad, const PT* __restrict__ param, const float* __restrict__ rowtab,
    const float* __restrict__ coltab, const ModeMeta* __restrict__ meta, const unsigned char* __restrict__ bins,
    Ctrl* __restrict__ ctrl, double* __restrict__ part, unsigned long long* __restrict__ hist,
    unsigned long long* __restrict__ rowfx, unsigned long long* __restrict__ colfx, int hash_arg, int axes_arg,
    const double* __restrict__ part1, float* __restrict__ fr_state, int step, Lanes L, cresso_hyper h) {
    if (L.dv) {
        const cresso_spectral_desc& d = lane_desc(L);
        grad = (const GT*)d.grad; param = (const PT*)d.param; fr_state = (float*)d.force_rms; step = d.step;
    }
    ctrl = lane_at(ctrl, L); part = lane_at(part, L); hist = lane_at(hist, L);
    rowfx = lane_at(rowfx, L); colfx = lane_at(colfx, L); part1 = lane_at(part1, L);
    constexpr int RW = 2 * RM;
    extern __shared__ __align__(16) unsigned char dyn[];
    __shared__ float red[4 * NV2];
    const SweepFlags F = sweep_flags<MODE>(g, hash_arg, axes_arg, h);
    const Tile t = tile_of(g);
    const int B = g.B;
    const int TB = F.T * B;
    const int nr = (int)(t.r1 - t.r0);
    const int64_t base = panel_base(g, t);
    const GT* __restrict__ gb = grad + base;
    // MODE 1: the first batch's loads go out before the set-up below
    PanelBuf gbv, bnv;
    float x0[SP_U];
    uint32_t b0[SP_U];
    if constexpr (MODE == 1) {
        gbv = panel_buf(gb, g, nr);
        bnv = panel_buf(reinterpret_cast<const uint16_t*>(bins) + base, g, nr);
#pragma unroll
        for (int u = 0; u < SP_U; ++u) {
            x0[u] = ldb_lane<GT>(gbv, u);
            b0[u] = ldb_bins16(bnv, u);
        }
    }
    // LDS: histogram [T][B] u64 (low words; MODE 1: [T][B][SP_NHIST] copies) |
    // row-sum partials [16][PR] (MODE 0: [4 waves][PR]; MODE 1: [4 waves][4
    // DPP rows][PR]) | MODE 1 row factors [PR][RW]
    unsigned long long* s_hist = reinterpret_cast<unsigned long long*>(dyn);
    float* s_wrow = reinterpret_cast<float*>(dyn + sizeof(unsigned long long) * SP_NHIST * (size_t)TB);
    constexpr int NH = MODE == 1 ? SP_NHIST : 1;   // histogram copies in use
    float* s_ar = s_wrow + 16 * g.PR;
    if (F.hash_on)
        for (int i = threadIdx.x; i < NH * TB; i += SP_NT) s_hist[i] = 0ull;
    if (MODE == 1) stage_rows<RM>(g, rowtab, t.r0, nr, s_ar);
    __syncthreads();
    const PT* __restrict__ pb = param + base;
    const float* __restrict__ rt = rowtab + t.r0 * g.RW;
    const F1Values f1 = fin1_values(g, part1, ctrl, fr_state, step, h);
    const float inv_s = f1.inv_s;
    const float eps = (float)h.eps;
    const float pw = (float)h.energy_power;
    const float ipw = (float)fmax(h.instant_metric_power, 0.25);
    const bool ip_one = ipw == 1.0f;
    const float wd = (float)h.weight_decay;
    const float sg = h.maximize ? -1.f : 1.f;
    // (every thread holds the same values: scalar registers)
    const float hs = (float)f1.hs_ds, yk = uniform_f(f1.yk), hq = uniform_f(f1.hq), kmf = uniform_f(f1.kmf);
    const bool hi_on = __builtin_amdgcn_readfirstlane((int)f1.hi_on) != 0;   // uniform: a scalar branch
    float Z[RW];
#pragma unroll
    for (int q = 0; q < RW; ++q) Z[q] = 0.f;
    float aL = 0.f, aD = 0.f;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // Sums of log(1 + ds) are kept in log2 units (fin2 scales them by ln 2).
    if constexpr (MODE == 1) {
        // full tile: rel >= eps and instant-metric power 1, so the density is rel
        constexpr int U = SP_U;
        const int hc = threadIdx.x & (SP_NHIST - 1);
        pipelined_batches<U>(
            nr,
            [&](int lr, float& x, uint32_t& b) {
                x = ldb_lane<GT>(gbv, lr);
                b = ldb_bins16(bnv, lr);
            },
            [&](int i0, const float* x, const uint32_t* bv) {
#pragma unroll
                for (int h8 = 0; h8 < U / 8; ++h8) {
                    float dn[8];
#pragma unroll
                    for (int v8 = 0; v8 < 8; ++v8) {
                        const int u = 8 * h8 + v8;
                        const float rel = rel_full(x[u], inv_s, eps);
                        const float ds = fexp2(pw * flog2(rel));
                        const float L = flog2(1.0f + ds);
                        dn[v8] = rel;
                        aL += L;
                        aD += rel;
                        const float* __restrict__ ar = s_ar + (i0 + u) * RW;
#pragma unroll
                        for (int q = 0; q < RW; ++q) Z[q] = fmaf(ar[q], L, Z[q]);
                        const unsigned long long v = to_fixed_u(fminf(ds * hs, yk));   // high words: hi_pass
                        atomicAdd(&s_hist[bin_of(bv[u], 0, 1) * NH + hc], v);
                        atomicAdd(&s_hist[(B + bin_of(bv[u], 1, 1)) * NH + hc], v);
#pragma unroll
                        for (int q = 0; q < RW; ++q) pin1(Z[q]);
                        pin1(aL);
                        pin1(aD);
                        pin1(dn[v8]);
                        elem_fence();
                    }
                    const float rs = rows8_lanesum16(dn);
                    if ((lane & 8) == 0) s_wrow[((wave << 2) + (lane >> 4)) * g.PR + i0 + 8 * h8 + (lane & 7)] = rs;
                }
            },
            x0, b0);
    } else
    for (int i0 = 0; i0 < nr; i0 += SP_U) {
        float gv[SP_U], pv[SP_U];
        uint64_t bv[SP_U];
#pragma unroll
        for (int u = 0; u < SP_U; ++u) {
            gv[u] = 0.f;
            pv[u] = 0.f;
            bv[u] = 0;
            if (i0 + u < nr && t.colok) {
                const uint32_t o = panel_off(g, i0 + u);
                gv[u] = to_f(gb[o]);
                if (F.wd_on) pv[u] = to_f(pb[o]);
                if (F.hash_on) bv[u] = load_bins_at(bins, base, o, F.binbytes);
            }
        }
#pragma unroll
        for (int u = 0; u < SP_U; ++u) {
            const int lr = i0 + u;
            if (lr >= nr) break;
            float dens = 0.f;
            if (t.colok) {
                const float rel = rel_gen(force_of(gv[u], pv[u], sg, wd, F.wd_on), inv_s, eps);
                const float ds = fpow(rel, pw);
                const float L = flog2(1.0f + ds);
                const float rl = fmaxf(rel, eps);
                dens = fminf(ip_one ? rl : fpow(rl, ipw), 1.0e6f);
                aL += L;
                aD += dens;
                const float* __restrict__ ar = rt + lr * g.RW;
#pragma unroll
                for (int q = 0; q < RW; ++q) Z[q] += ar[q] * L;
                if (F.hash_on) {
                    const unsigned long long v = to_fixed_u(fminf(ds * hs, yk));   // high words: hi_pass
#pragma unroll
                    for (int tt = 0; tt < SP_MAXT; ++tt) {
                        if (tt >= F.T) break;
                        atomicAdd(&s_hist[tt * B + bin_of(bv[u], tt, F.bpb)], v);
                    }
                }
            }
            if (F.axes_on) {
                const float ws = wave_total(dens);
                if (lane == 63) s_wrow[wave * g.PR + lr] = ws;
            }
            if (MODE == 0) elem_fence();
        }
    }
    if (F.hash_on && hi_on && hi_block(g, part1, base, nr, inv_s, eps, pw, kmf) && t.colok) {
        // high-word pass: the thread's elements again
        const unsigned long long lo_k = to_fixed_u(yk);   // what the loop added for y >= 2^k
        for (int lr = 0; lr < nr; ++lr) {
            const uint32_t o = panel_off(g, lr);
            float ds;
            if constexpr (MODE == 1) {
                ds = fexp2(pw * flog2(rel_full(to_f(gb[o]), inv_s, eps)));
            } else {
                const float pvv = F.wd_on ? to_f(pb[o]) : 0.f;
                ds = fpow(rel_gen(force_of(to_f(gb[o]), pvv, sg, wd, F.wd_on), inv_s, eps), pw);
            }
            if (ds * hs >= yk) {
                // MODE 1: two tables of one-byte bins, histogram copy threadIdx.x mod SP_NHIST
                const uint64_t bb = MODE == 1 ? (uint64_t)(reinterpret_cast<const uint16_t*>(bins) + base)[o]
                                              : load_bins_at(bins, base, o, F.binbytes);
                const int nt = MODE == 1 ? 2 : F.T, bpb = MODE == 1 ? 1 : F.bpb;
                const int hcm = MODE == 1 ? (int)(threadIdx.x & (SP_NHIST - 1)) : 0;
                const HiSplit sp = hi_split(ds, hq, yk, lo_k);
                for (int tt = 0; tt < nt; ++tt) {
                    const int bin = tt * B + bin_of(bb, tt, bpb);
                    atomicAdd(&hist[(size_t)g.hcopies * TB + bin], sp.hi);   // the high-word table
                    atomicAdd(&s_hist[bin * NH + hcm], sp.lo);
                }
            }
        }
    }
    __syncthreads();
    if (F.axes_on) {
        // axis density sums: one fixed-point atomic per row of this slab and per column of this panel
        for (int lr = threadIdx.x; lr < nr; lr += SP_NT) {
            float s = 0.f;
            for (int w = 0; w < (MODE == 1 ? 16 : SP_NT / 64); ++w) s += s_wrow[w * g.PR + lr];
            atomicAdd(&rowfx[t.r0 + lr], to_fixed_u(s * (float)g.hs_row));
        }
        if (t.colok) atomicAdd(&colfx[t.col], to_fixed_u(aD * (float)g.hs_col));
    }
    if (F.hash_on)
        for (int i = threadIdx.x; i < TB; i += SP_NT) {
            unsigned long long v = 0ull;
#pragma unroll
            for (int c = 0; c < NH; ++c) v += s_hist[i * NH + c];
            if (v) atomicAdd(&hist[i], v);
        }
    float b[KC];
    load_cols<KC>(g, coltab, t, b);
    Partials P{red, 2 + 2 * g.R, NV2};
    P.add(0, aL);
    P.add(1, aD);
    proj_finish<RM, KC>(g, meta, Z, b, P, 2);
    P.flush(part);
}



// Helpers of the matrix-core sweeps.
constexpr int SP_BQS = SP_NT + 16;   // row stride of sweep3m's LDS carrier table
template <typename GT> __device__ __forceinline__ float ldg_el(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff);
template <> __device__ __forceinline__ float ldg_el<float>(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return bload1(r, voff, soff);
}
template <> __device__ __forceinline__ float ldg_el<__half>(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return to_f(__builtin_bit_cast(__half, (unsigned short)bload1u16(r, voff, soff)));
}
template <>
__device__ __forceinline__ float ldg_el<__hip_bfloat16>(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return to_f(__builtin_bit_cast(__hip_bfloat16, (unsigned short)bload1u16(r, voff, soff)));
}
template <> __device__ __forceinline__ float ldg_el<double>(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return (float)__builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
}

// Sum over each 16-lane DPP row (every lane of the row gets its row's total,
// in a fixed order).
__device__ __forceinline__ float row16_total(float v) {
    v = dpp_add<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
    v = dpp_add<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
    v = dpp_add<0x124, 0xF>(v);  // row_ror:4
    v = dpp_add<0x128, 0xF>(v);  // row_ror:8
    return v;
}

// The matrix-core sweeps take TT = 2 or 4 tables of one-byte bins, packed in
// TT bytes per element (table t in byte t).
template <int TT> __device__ __forceinline__ uint32_t ldg_bins(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    static_assert(TT == 2 || TT == 4, "two or four tables of one-byte bins");
    if constexpr (TT == 2)
        return bload1u16(r, voff, soff);
    else
        return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}
template <int TT> __device__ __forceinline__ uint32_t bin_byte(uint32_t b, int tt) {
    return tt == TT - 1 ? (b >> (8 * tt)) : ((b >> (8 * tt)) & 0xffu);
}
// projection rows of rank RM in 16-row tiles; carriers in chunks of 4
template <int RM> constexpr int nqt() { return (2 * RM + 15) / 16; }


// Inputs of a matrix-core sweep's projection finish: lane group lg's modes
// r = 8 qt + 2 lg + h (h = 0, 1) and their column carriers b1, b2 at the
// lane's 4 columns.  Fetched in the prologue, so that the finish after the
// last tile is not a dependent global round trip (mode table, then carriers).
template <int NQ>
struct ProjCols {
    int on[NQ][2], add[NQ][2], k1[NQ][2], k2[NQ][2];
    float b1[NQ][2][4], b2[NQ][2][4];
    // modes, first thing in the kernel
    __device__ __forceinline__ void modes(const Geom& g, const ModeMeta* __restrict__ meta, int lg, int KC) {
#pragma unroll
        for (int qt = 0; qt < NQ; ++qt)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int r = 8 * qt + 2 * lg + hh;
                const ModeMeta m = meta[r < g.R ? r : 0];
                on[qt][hh] = r < g.R;
                add[qt][hh] = m.type == M_ADD;
                // carrier index outside [0, KC) (k2 = -1: identically zero) reads as 0
                k1[qt][hh] = (m.k1 >= 0 && m.k1 < KC) ? m.k1 : -1;
                k2[qt][hh] = (m.k2 >= 0 && m.k2 < KC) ? m.k2 : -1;
            }
    }
    // carriers of the lane's columns colw + 16 tc + li from the column table
    __device__ __forceinline__ void load(const Geom& g, const float* __restrict__ coltab, int64_t colw, int li) {
#pragma unroll
        for (int qt = 0; qt < NQ; ++qt)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                for (int tc = 0; tc < 4; ++tc) {
                    // (row 0 for an absent carrier, then zeroed: no branch between the loads)
                    const int64_t c = colw + 16 * tc + li;
                    const float v1 = coltab[(size_t)(k1[qt][hh] >= 0 ? k1[qt][hh] : 0) * g.cols + c];
                    const float v2 = coltab[(size_t)(k2[qt][hh] >= 0 ? k2[qt][hh] : 0) * g.cols + c];
                    b1[qt][hh][tc] = k1[qt][hh] >= 0 ? v1 : 0.f;
                    b2[qt][hh][tc] = k2[qt][hh] >= 0 ? v2 : 0.f;
                }
    }
    // the same carriers from an LDS copy of the block's column table rows (row stride ls)
    __device__ __forceinline__ void load_lds(const float* __restrict__ s_col, int ls, int wcol, int li) {
#pragma unroll
        for (int qt = 0; qt < NQ; ++qt)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                for (int tc = 0; tc < 4; ++tc) {
                    const int c = wcol + 16 * tc + li;
                    b1[qt][hh][tc] = k1[qt][hh] >= 0 ? s_col[k1[qt][hh] * ls + c] : 0.f;
                    b2[qt][hh][tc] = k2[qt][hh] >= 0 ? s_col[k2[qt][hh] * ls + c] : 0.f;
                }
    }
    // in q-tile qt, lane group lg holds Z_{16 qt + 4 lg + j}(col), j < 4: both
    // components of its two modes for its 4 columns (proj_finish's form); each
    // mode's raw C/S is summed over the columns, then over the 16 lanes of the
    // group, into LDS slots base + 16 qt + 4 lg + j of wave wv's row of red
    __device__ __forceinline__ void finish(const Geom& g, const f32x4m (&zacc)[NQ][4], float* red, int rowV, int base,
                                           int wv, int lg, int li) const {
#pragma unroll
        for (int qt = 0; qt < NQ; ++qt) {
            float cs[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                if (on[qt][hh]) {
#pragma unroll
                    for (int tc = 0; tc < 4; ++tc) {
                        const float z1 = zacc[qt][tc][2 * hh], z2 = zacc[qt][tc][2 * hh + 1];
                        const float c1 = b1[qt][hh][tc], c2 = b2[qt][hh][tc];
                        if (add[qt][hh]) {
                            cs[2 * hh] += c1 * z1 - c2 * z2;
                            cs[2 * hh + 1] += c1 * z2 + c2 * z1;
                        } else {
                            cs[2 * hh] += c1 * z1;
                            cs[2 * hh + 1] += c2 * z2;
                        }
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float sm = row16_total(cs[j]);
                const int slot = 16 * qt + 4 * lg + j;
                if (li == 15 && slot < 2 * g.R) red[wv * rowV + base + slot] = sm;
            }
        }
    }
};
template <int KC> constexpr int kch() { return (KC + 3) / 4; }
// Waves per SIMD (blocks of 256 threads per CU) each matrix-core sweep is
// compiled for: 4 at rank <= 8 with carriers in LDS; sweep 3m holds the
// carriers in registers past three chunks and 256 VGPRs at rank 16 (two
// waves); sweeps 2m and 4m fit in 168 VGPRs at rank 16 (three waves, their
// LDS 44 and 31 KiB a block).
template <int RM, int KC> constexpr int occ2m() { return RM > 8 ? 3 : 4; }
template <int RM, int KC> constexpr int occ3m() { return (RM > 8 || kch<KC>() > 3) ? 2 : 4; }
template <int RM, int KC> constexpr int occ4m() { return (RM > 8 || kch<KC>() > 3) ? 3 : 4; }

// ---------------------------------------------------------------------------
// S2 on the matrix cores (MODE 1 tiles, RM <= 16, TT = 2 or 4 tables of
// one-byte bins): sweep2_kernel's element math in sweep3m_kernel's tile
// layout (lane l: rows 4 lg + r of column li of each 16 x 16 tile, 4 tile
// columns per wave).  The log-density projection Z_q(col) = sum_rows a_q(row)
// L(row, col) is 4 MFMAs per tile and 16-row tile of q (A = the rows' factors,
// B = L).  Row density sums: the lane's 4 tile columns are added in registers,
// then each 16-lane row group sums its columns with DPP; column sums stay per
// lane and tile column until the end.
// ---------------------------------------------------------------------------
template <int RM, int KC, typename GT, int TT>
__global__ __launch_bounds__(SP_NT, (occ2m<RM, KC>())) void sweep2m_kernel(
    Geom g, const GT* __restrict__ grad, const float* __restrict__ rowtab, const float* __restrict__ coltab,
    const ModeMeta* __restrict__ meta, const unsigned char* __restrict__ bins, Ctrl* __restrict__ ctrl,
    double* __restrict__ part, unsigned long long* __restrict__ hist, unsigned long long* __restrict__ hhi,
    unsigned long long* __restrict__ rowfx, unsigned long long* __restrict__ colfx, const double* __restrict__ part1,
    float* __restrict__ fr_state, int step, Lanes L, cresso_hyper h, int one_round, int hdirect) {
    if (L.dv) {
        const cresso_spectral_desc& d = lane_desc(L);
        grad = (const GT*)d.grad; fr_state = (float*)d.force_rms; step = d.step;
    }
    ctrl = lane_at(ctrl, L); part = lane_at(part, L); hist = lane_at(hist, L); hhi = lane_at(hhi, L);
    rowfx = lane_at(rowfx, L); colfx = lane_at(colfx, L); part1 = lane_at(part1, L);
    static_assert(RM <= 16, "two 16-row tiles of projection rows at most");
    constexpr int RW = 2 * RM;
    constexpr int NQ = nqt<RM>();
    extern __shared__ __align__(16) unsigned char dyn[];
    __shared__ float red[4 * NV2];
    const Tile t = tile_of(g);
    const int B = g.B;
    const int TB = TT * B;
    const int nr = g.PR;
    const int l = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int li = l & 15, lg = l >> 4;
    ProjCols<NQ> pc;
    pc.modes(g, meta, lg, KC);
    const int64_t base = panel_base(g, t);
    const uint32_t cols = (uint32_t)g.cols;
    const __amdgpu_buffer_rsrc_t rg = make_rsrc(grad + base, (uint32_t)((int64_t)nr * g.cols * (int64_t)sizeof(GT)));
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(bins + (size_t)TT * base, (uint32_t)((int64_t)nr * g.cols * TT));
    const uint32_t lane_el = 4u * (uint32_t)lg * cols + 64u * (uint32_t)wv + (uint32_t)li;  // element offset
    const uint32_t vg = lane_el * (uint32_t)sizeof(GT), vb = lane_el * (uint32_t)TT;
    auto tile_off = [&](int tr, int tc, int r) -> uint32_t { return (uint32_t)(16 * tr + r) * cols + 16u * tc; };
    // one register set, refilled tile by tile (loads three tiles ahead of use)
    float xv[16];
    uint32_t bv[16];
    auto load_tile = [&](int tr, int tc) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t o = tile_off(tr, tc, r);
            xv[4 * tc + r] = ldg_el<GT>(rg, vg, o * (uint32_t)sizeof(GT));
            bv[4 * tc + r] = ldg_bins<TT>(rb, vb, o * (uint32_t)TT);
        }
    };
#pragma unroll
    for (int tc = 0; tc < 4; ++tc) load_tile(0, tc);
    // LDS: histogram copies [TB][NH] u64 (low words) | row-sum partials [4 waves][PR] | row factors [PR][RW]
    constexpr int NH = SP_NHIST;
    const int hc = (int)(threadIdx.x & (SP_NHIST - 1));
    unsigned long long* s_hist = reinterpret_cast<unsigned long long*>(dyn);
    float* s_wrow = reinterpret_cast<float*>(dyn + sizeof(unsigned long long) * SP_NHIST * (size_t)TB);
    float* s_ar = s_wrow + 16 * g.PR;
    // set-up loads, all issued behind the first tiles': the row factors and
    // sweep 1's block partials
    constexpr int NRW = (64 * RW + SP_NT - 1) / SP_NT;
    Staged<NRW> srw;
    srw.template load_rows<RM>(g, rowtab, t.r0, nr);
    F1Part<4> f1p;
    f1p.load(g, part1);
    for (int i = threadIdx.x; i < NH * TB; i += SP_NT) s_hist[i] = 0ull;
    srw.store(s_ar, nr * RW);
    stage_rows_rest<RM, NRW>(g, rowtab, t.r0, nr, s_ar);
    // the projection finish's carriers (their rows come from the mode table,
    // in registers by now); first used after the loop
    const int64_t colw = (int64_t)t.slab * SP_NT + 64 * wv;
    pc.load(g, coltab, colw, li);
    __syncthreads();
    const F1Values f1 = fin1_values<4>(g, f1p, part1, ctrl, fr_state, step, h);
    const float inv_s = f1.inv_s;
    const float eps = (float)h.eps;
    const float pw = (float)h.energy_power;
    // (every thread holds the same values: scalar registers)
    const float hs = (float)f1.hs_ds, yk = uniform_f(f1.yk), hq = uniform_f(f1.hq), kmf = uniform_f(f1.kmf);
    const bool hi_on = __builtin_amdgcn_readfirstlane((int)f1.hi_on) != 0;   // uniform: a scalar branch
    // the lane's projection A operands, a_{16 qt + li}(row 16 tr + 4 lg + r),
    // held in registers: read from LDS inside the loop they would queue
    // behind the histogram atomics (LDS operations complete in order)
    float aJv[NQ][4][4];
#pragma unroll
    for (int qt = 0; qt < NQ; ++qt)
#pragma unroll
        for (int tr = 0; tr < 4; ++tr)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int q = 16 * qt + li;
                aJv[qt][tr][r] = (q < RW && tr < nr / 16) ? s_ar[(16 * tr + 4 * lg + r) * RW + (q < RW ? q : 0)] : 0.f;
            }
    f32x4m zacc[NQ][4];
#pragma unroll
    for (int qt = 0; qt < NQ; ++qt)
#pragma unroll
        for (int tc = 0; tc < 4; ++tc) zacc[qt][tc] = f32x4m{0.f, 0.f, 0.f, 0.f};
    float aL = 0.f;
    float cD[4] = {0.f, 0.f, 0.f, 0.f};   // column density sums of the lane's 4 tile columns
    // Sums of log(1 + ds) are kept in log2 units (fin2 scales them by ln 2).
    const int ntr = nr / 16;   // 2 or 4 (panels of 32 or 64 rows)
#pragma unroll
    for (int tr = 0; tr < 4; ++tr) {
        if (tr >= ntr) break;
        if (one_round) progress_prio(4 * tr / ntr);
        float rs[4] = {0.f, 0.f, 0.f, 0.f};   // this row of tiles' density, per lane row
#pragma unroll
        for (int tc = 0; tc < 4; ++tc) {
            const float* x = xv + 4 * tc;
            const uint32_t* b = bv + 4 * tc;
            float Ls[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                // full tile: rel >= eps and instant-metric power 1, so the density is rel
                // (|sign x| = |x|)
                const float rel = rel_full(x[r], inv_s, eps);
                const float ds = fexp2(pw * flog2(rel));
                const float L = flog2(1.0f + ds);
                Ls[r] = L;
                aL += L;
                rs[r] += rel;
                cD[tc] += rel;
                const unsigned long long v = to_fixed_u(fminf(ds * hs, yk));   // high words: hi_pass
#pragma unroll
                for (int tt = 0; tt < TT; ++tt) atomicAdd(&s_hist[(tt * B + bin_byte<TT>(b[r], tt)) * NH + hc], v);
            }
            // A of the projection: a_q(row 16 tr + 4 lg + r)
#pragma unroll
            for (int qt = 0; qt < NQ; ++qt)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    zacc[qt][tc] = __builtin_amdgcn_mfma_f32_16x16x4f32(aJv[qt][tr][r], Ls[r], zacc[qt][tc], 0, 0, 0);
            if (tr + 1 < ntr) load_tile(tr + 1, tc);
            pin1(aL);
#pragma unroll
            for (int r = 0; r < 4; ++r) pin1(rs[r]);
#pragma unroll
            for (int c = 0; c < 4; ++c) pin1(cD[c]);
            elem_fence();
        }
        // rows 16 tr + 4 lg + r: the 16 columns of the lane group, lane li = r writes
        float rt[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) rt[r] = row16_total(rs[r]);
        if (li < 4) s_wrow[wv * g.PR + 16 * tr + 4 * lg + li] = li == 0 ? rt[0] : (li == 1 ? rt[1] : (li == 2 ? rt[2] : rt[3]));
    }
    if (hi_on && hi_block(g, part1, base, nr, inv_s, eps, pw, kmf)) {
        // high-word pass: the lane's elements again
        const unsigned long long lo_k = to_fixed_u(yk);   // what the loop added for y >= 2^k
        for (int tr = 0; tr < ntr; ++tr)
            for (int tc = 0; tc < 4; ++tc)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t o = tile_off(tr, tc, r);
                    const float ds = fexp2(pw * flog2(rel_full(ldg_el<GT>(rg, vg, o * (uint32_t)sizeof(GT)), inv_s, eps)));
                    if (ds * hs >= yk) {
                        const uint32_t bb = ldg_bins<TT>(rb, vb, o * (uint32_t)TT);
                        const HiSplit sp = hi_split(ds, hq, yk, lo_k);
#pragma unroll
                        for (int tt = 0; tt < TT; ++tt) {
                            const int bin = tt * B + (int)bin_byte<TT>(bb, tt);
                            atomicAdd(&hhi[bin], sp.hi);   // the high-word table (global)
                            atomicAdd(&s_hist[bin * NH + hc], sp.lo);
                        }
                    }
                }
    }
    __syncthreads();
    // axis density sums: one fixed-point atomic per row of this slab and per column of this panel
    for (int lr = threadIdx.x; lr < nr; lr += SP_NT) {
        float sr = 0.f;
        for (int w = 0; w < SP_NT / 64; ++w) sr += s_wrow[w * g.PR + lr];
        atomicAdd(&rowfx[t.r0 + lr], to_fixed_u(sr * (float)g.hs_row));
    }
    float aD = 0.f;
#pragma unroll
    for (int tc = 0; tc < 4; ++tc) {
        // the column's 4 lane groups, in a fixed order
        float c = cD[tc];
        c += __shfl_xor(c, 16, 64);
        c += __shfl_xor(c, 32, 64);
        if (lg == 0) atomicAdd(&colfx[colw + 16 * tc + li], to_fixed_u(c * (float)g.hs_col));
        aD += cD[tc];
    }
    for (int i = threadIdx.x; i < TB; i += SP_NT) {
        unsigned long long v = 0ull;
#pragma unroll
        for (int c = 0; c < NH; ++c) v += s_hist[i * NH + c];
        if (hdirect) {
            // multi-round launch: blocks end at different times, so they add
            // into the SP_HCOPIES histogram copies directly (integer sums)
            if (v) atomicAdd(&hist[(size_t)(blockIdx.x % SP_HCOPIES) * TB + i], v);
        } else {
            hist[(size_t)blockIdx.x * TB + i] = v;   // this block's partial (hpart[block][bin])
        }
    }
    Partials P{red, 2 + 2 * g.R, NV2};
    P.add(0, aL);
    P.add(1, aD);
    pc.finish(g, zacc, red, P.V, 2, wv, lg, li);
    P.flush(part);
}



// Bin i of a merged histogram: the sum of its nc copies (loads issued
// together), each cleared for the next sweep.
__device__ __forceinline__ unsigned long long take_hist(unsigned long long* __restrict__ hist, int TB, int i, int nc) {
    unsigned long long c[SP_HCOPIES];
#pragma unroll
    for (int k = 0; k < SP_HCOPIES; ++k) c[k] = k < nc ? hist[(size_t)k * TB + i] : 0ull;
    unsigned long long v = 0ull;
#pragma unroll
    for (int k = 0; k < SP_HCOPIES; ++k) {
        if (k >= nc) break;
        v += c[k];
        hist[(size_t)k * TB + i] = 0ull;
    }
    return v;
}

// ---------------------------------------------------------------------------
// finalize helpers: one wave, one lane per mode
// ---------------------------------------------------------------------------
// Mode weights (the coefficient of each normalized carrier) and the
// coefficients (wc, ws) of the raw carriers and the constant of
//   shrink * sum_r g_r (cc_r Cn_r + sc_r Sn_r)  (cresso_v5.py:362-376)
// with Cn = (Craw - mu_c) ic; a gate of exactly 0 drops the mode.  Lane r of
// the calling wave handles mode r; the constant is summed in mode order.
__device__ void set_recon_lanes(const Geom& g, const double* __restrict__ stats, float (*rc)[2], float* rconst,
                                float cc, float sc, float gate, float* s_tmp, float* weights = nullptr) {
    const int r = threadIdx.x & 63;
    const double shrink = g.shrink;
    float kc = 0.f, ks = 0.f, wc = 0.f, ws = 0.f, cterm = 0.f;
    if (r < g.R) {
        if (gate != 0.0f) {
            kc = (float)((double)cc * shrink) * gate;
            ks = (float)((double)sc * shrink) * gate;
            wc = (float)((double)kc * stats[4 * r + 1]);
            ws = (float)((double)ks * stats[4 * r + 3]);
            cterm = (float)((double)wc * stats[4 * r + 0] + (double)ws * stats[4 * r + 2]);
        }
        rc[r][0] = wc;
        rc[r][1] = ws;
        s_tmp[r] = cterm;
        if (weights) {
            weights[2 * r] = kc;
            weights[2 * r + 1] = ks;
        }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup", "local");   // LDS only: pending global stores need not complete
    if (r == 0) {
        float cst = 0.f;
        for (int q = 0; q < g.R; ++q) cst -= s_tmp[q];
        *rconst = cst;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup", "local");   // LDS only: pending global stores need not complete
}

// Sum over lanes 0..R-1 of a fully active wave (fp64), in the fixed order of
// the DPP wave reduction, returned to every lane.
__device__ double lanes_sum(double v, int R) {
    const int r = threadIdx.x & 63;
    const double t = wave_total_d(r < R ? v : 0.0);
    const int lo = __builtin_amdgcn_readlane(__double2loint(t), 63);
    const int hi = __builtin_amdgcn_readlane(__double2hiint(t), 63);
    return __hiloint2double(hi, lo);
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

// Barrier of waves 1.. of a finalize block while wave 0 runs the mode lanes:
// each arriving wave publishes its earlier stores (workgroup-scope release),
// counts itself in an LDS counter and waits until the counter reaches
// `target`.  Every wave 1.. calls each such barrier, so every wait ends;
// targets are cumulative (k-th barrier: k times the number of waves 1..).
__device__ __forceinline__ void waves_sync(unsigned int* cnt, unsigned int target) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    while (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target) __builtin_amdgcn_s_sleep(1);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// ---------------------------------------------------------------------------
// F2: hash metric, metric oscillator, recon coefficients
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(SP_FN_NT) void fin2_kernel(
    Geom g, const ModeMeta* __restrict__ meta, const double* __restrict__ stats, const double* __restrict__ bounds,
    const double* __restrict__ part, unsigned long long* __restrict__ hist,
    const unsigned long long* __restrict__ counts, float* __restrict__ lt, SpecState st, Ctrl* __restrict__ ctrl,
    int step, int hash_on, int hard, int nc, Lanes L, cresso_hyper h) {
    if (L.dv) {
        st = spec_state(lane_desc(L));
        step = lane_desc(L).step;
    }
    part = lane_at(part, L); hist = lane_at(hist, L); lt = lane_at(lt, L); ctrl = lane_at(ctrl, L);
    __shared__ double s_v[NV2];
    __shared__ double s_wsum[SP_MAXT][SP_FN_NT / 64];
    __shared__ float s_emean[SP_MAXT];
    __shared__ float s_e[SP_FN_E];   // this step's hash energy when T B <= SP_FN_E
    __shared__ float s_tmpf[64];
    __shared__ unsigned int s_sync;
    const int tid = threadIdx.x;
    if (tid == 0) s_sync = 0u;   // published by the staging barrier
    const float eps = (float)h.eps;
    __shared__ double s_stats[4 * SP_MAXR], s_bounds[2 * SP_MAXR];
    __shared__ float s_mode[SP_MAXR][9];
    __shared__ int s_zero[SP_MAXR];
    // everything the block reads is loaded first, one value per thread at
    // clamped (in-bounds) indices, so the loads are in flight together; then
    // stored to LDS
    static_assert(9 * SP_MAXR <= SP_FN_NT && NV2 <= SP_FN_NT, "one staged value per thread");
    const int R = g.R, NS = 2 + 2 * R;
    const double v_st = stats[tid < 4 * R ? tid : 0];
    const double v_bd = bounds[tid < 2 * R ? tid : 0];
    const int mi = tid < 9 * R ? tid : 0, mr = mi / 9, mj = mi - 9 * mr;
    const float* src[8] = {st.omega, st.metric_cos, st.metric_p_cos, st.metric_sin, st.metric_p_sin, st.q_cos,
                           st.q_sin, st.conf};
    const float v_md = src[mj < 8 ? mj : 0][mr];
    const int v_zero = meta[mr].type == M_ZERO;
    const double v_sum = part[tid < NS ? tid : 0];
    if (tid < 4 * R) s_stats[tid] = v_st;
    if (tid < 2 * R) s_bounds[tid] = v_bd;
    if (tid < 9 * R) {
        if (mj < 8) s_mode[mr][mj] = v_md;
        else s_zero[mr] = v_zero;
    }
    // sweep 2 sums log(1 + ds) in log2 units
    if (tid < NS) s_v[tid] = tid != 1 ? v_sum * 0.6931471805599453 : v_sum;
    __syncthreads();
    // hash energy per table (cresso_v5.py:1012-1056), on waves 1.. while wave 0
    // runs the mode lanes (which read none of it)
    if (hash_on && tid >= 64) {
        const int TB = g.T * g.B, t1 = tid - 64, n1 = SP_FN_NT - 64;
        constexpr unsigned nw1 = SP_FN_NT / 64 - 1;
        // the means and the log table read the new energies back from LDS
        // (from the state in global memory when the tables are larger)
        const bool el = TB <= SP_FN_E;
        for (int i = t1; i < TB; i += n1) {
            const double cnt = (double)counts[i];
            // low words (every copy) plus the high word, each cleared for the next step
            unsigned long long* hhi = hist + (size_t)g.hcopies * TB + i;
            const unsigned long long hv = *hhi;
            *hhi = 0ull;
            const double lo = (double)(long long)take_hist(hist, TB, i, nc) / ctrl->hs_ds;
            const float cell = (float)(fma((double)hv, ctrl->hs_hi, lo) / fmax(cnt, 1.0));
            float e = st.hash_energy[i];
            e = step <= 1 ? cell : e * (float)h.hash_decay + (float)(1.0 - h.hash_decay) * cell;
            st.hash_energy[i] = e;
            if (el) s_e[i] = e;
        }
        waves_sync(&s_sync, nw1);
        // each table's mean: the waves' fp64 totals added in wave order
        for (int tt = 0; tt < g.T; ++tt) {
            double a = 0.0;
            for (int b = t1; b < g.B; b += n1) a += (double)(el ? s_e[tt * g.B + b] : st.hash_energy[tt * g.B + b]);
            const double w = wave_total_d(a);
            if ((tid & 63) == 63) s_wsum[tt][(tid >> 6) - 1] = w;
        }
        waves_sync(&s_sync, 2 * nw1);
        if (t1 < g.T) {
            double a = 0.0;
            for (int w = 0; w < (int)nw1; ++w) a += s_wsum[t1][w];
            s_emean[t1] = (float)(a / (double)g.B);
        }
        waves_sync(&s_sync, 3 * nw1);
        const float ex = (float)(h.hash_metric_coupling / fmax(0.25, h.energy_power));
        for (int i = t1; i < TB; i += n1) {
            const int tt = i / g.B;
            const float hm = fmaxf((el ? s_e[i] : st.hash_energy[i]) / fmaxf(s_emean[tt], eps), eps);
            lt[i] = logf(fmaxf(clampf(powf(hm, ex), 0.08f, 12.0f), eps));
        }
    }
    if (tid < 64) {
        // lane r: mode r
        const int r = tid;
        const bool on = r < g.R;
        const double sumL = s_v[0], sumD = s_v[1];
        // log-density projections: d = L/max(mean L, eps) - 1, mean(d Cn) = mean(L Cn)/m - mean(Cn)
        const double m = fmax((double)(float)(sumL * g.inv_n), (double)eps);
        float pcos = 0.f, psin = 0.f;
        if (on) {
            const double prc = (s_v[2 + 2 * r] - s_stats[4 * r] * sumL) * s_stats[4 * r + 1] * g.inv_n / m -
                               (s_zero[r] ? 1.0 : 0.0);   // mean(Cn) = 1 for the constant mode
            const double prs = (s_v[3 + 2 * r] - s_stats[4 * r + 2] * sumL) * s_stats[4 * r + 3] * g.inv_n / m;
            pcos = (float)prc;
            psin = (float)prs;
        }
        // metric oscillator (cresso_v5.py:1064-1088)
        const float mdt = (float)h.metric_dt;
        const float damp = (float)fmax(0.0, 1.0 - h.metric_dt * h.metric_friction);
        float mqc = 0.f, mqs = 0.f;
        if (on) {
            const float om = s_mode[r][0];
            const float o2 = om * om;
            float mq = s_mode[r][1], mp = s_mode[r][2];
            mp = mp * damp;
            mp = mp + mdt * (pcos - o2 * mq);
            mq = clampf(mq + mdt * mp, -3.0f, 3.0f);
            st.metric_cos[r] = mq;
            st.metric_p_cos[r] = mp;
            mqc = mq;
            mq = s_mode[r][3];
            mp = s_mode[r][4];
            mp = mp * damp;
            mp = mp + mdt * (psin - o2 * mq);
            mq = clampf(mq + mdt * mp, -3.0f, 3.0f);
            st.metric_sin[r] = mq;
            st.metric_p_sin[r] = mp;
            mqs = mq;
        }
        set_recon_lanes(g, s_stats, ctrl->rc[0], &ctrl->rconst[0], mqc, mqs, 1.0f, s_tmpf);
        // prediction with the pre-contact state and gates
        float qc = 0.f, qs = 0.f, gt = 0.f;
        double pm = 0.0;
        const double shrink = g.shrink;
        if (on) {
            qc = s_mode[r][5];
            qs = s_mode[r][6];
            gt = sigmoidf_((float)h.confidence_gain * s_mode[r][7]);
            pm = shrink * gt * (fabs((double)qc) * s_bounds[2 * r] + fabs((double)qs) * s_bounds[2 * r + 1]);
        }
        set_recon_lanes(g, s_stats, ctrl->rc[1], &ctrl->rconst[1], qc, qs, gt, s_tmpf, ctrl->wpred);
        const double pmax = lanes_sum(pm, g.R);
        if (r == 0) {
            // instant metric: mean density and coupling (cresso_v5.py:243-262)
            ctrl->gden = (float)fmax(sumD * g.inv_n, (double)eps);
            const float icoup = hard ? (float)h.instant_metric_coupling : 0.0f;
            ctrl->kappa = (float)((double)icoup / ((double)g.ndim * fmax(h.instant_metric_power, 0.25)));
            // fixed-point scale of the port histogram: |P| <= (1+tm)*1e4 + max|pred|, <= cmax elements per bin
            const double vmax = (1.0 + h.transport_mix) * 1.0e4 + pmax * 1.01 + 1.0;
            ctrl->hs_P = ldexp(1.0, (int)floor(62.0 - log2(vmax * ctrl->cmax)));
        }
    }
}



// ndim >= 3: the factor of each column of the column group (the trailing
// axes) is the product over those axes of (axis mean / global mean)^kappa.
// marg_terms_kernel: one block per coordinate k of trailing axis a sums the
// column sums that share it (64-bit integers: exact in any order) into the
// axis term kappa log(max(mean / gden, eps)).
constexpr int SP_MARG_NT = 256;
__global__ __launch_bounds__(SP_MARG_NT) void marg_terms_kernel(
    Geom g, const unsigned long long* __restrict__ colfx, float* __restrict__ terms, const Ctrl* __restrict__ ctrl,
    float eps, Lanes L) {
    colfx = lane_at(colfx, L); terms = lane_at(terms, L); ctrl = lane_at(ctrl, L);
    __shared__ unsigned long long red[SP_MARG_NT];
    // block -> (axis a, coordinate k); the axis terms are laid out axis after axis
    int64_t k = blockIdx.x, off = 0;
    int a = 0;
    while (a + 1 < g.ntrail && k >= g.tdim[a]) {
        k -= g.tdim[a];
        off += g.tdim[a];
        ++a;
    }
    int64_t inner = 1;
    for (int b = a + 1; b < g.ntrail; ++b) inner *= g.tdim[b];
    const int64_t dim = g.tdim[a];
    const int64_t m = g.cols / dim;   // columns sharing coordinate k: outer x inner
    unsigned long long s = 0ull;
    for (int64_t j = threadIdx.x; j < m; j += SP_MARG_NT) {
        const int64_t o = j / inner, in = j - o * inner;
        s += colfx[(o * dim + k) * inner + in];
    }
    red[threadIdx.x] = s;
    __syncthreads();
    for (int w = SP_MARG_NT / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const float mean = (float)((double)red[0] / g.hs_col / ((double)g.n / (double)dim));
        terms[off + k] = ctrl->kappa * logf(fmaxf(mean / ctrl->gden, eps));
    }
}



// marg_fac_kernel: one thread per column, exp of the sum of its axis terms.
__global__ __launch_bounds__(SP_MARG_NT) void marg_fac_kernel(
    Geom g, const float* __restrict__ terms, float* __restrict__ colfac, Lanes L) {
    terms = lane_at(terms, L); colfac = lane_at(colfac, L);
    const int64_t c = (int64_t)blockIdx.x * SP_MARG_NT + threadIdx.x;
    if (c >= g.cols) return;
    int64_t off = 0;
    for (int a = 0; a < g.ntrail; ++a) off += g.tdim[a];
    int64_t rem = c;
    float acc = 0.f;
    for (int a = g.ntrail - 1; a >= 0; --a) {
        off -= g.tdim[a];
        const int64_t k = rem % g.tdim[a];
        rem /= g.tdim[a];
        acc += terms[off + k];
    }
    colfac[c] = expf(acc);
}



// ---------------------------------------------------------------------------
// S3: tangent force, prediction error, port projection / histograms, t projection
// ---------------------------------------------------------------------------
template <int RM, int KC, typename PT, typename GT, int MODE>
__global__ __launch_bounds__(SP_NT, RM >= 16 ? 2 : 4) void sweep3_kernel(
    Geom g, const GT* __restrict__ grad, const PT* __restrict__ param, const float* __restrict__ rowtab,
    const float* __restrict__ coltab, const ModeMeta* __restrict__ meta, const unsigned char* __restrict__ bins,
    const Ctrl* __restrict__ ctrl, const float* __restrict__ lt, const unsigned long long* __restrict__ rowfx,
    const unsigned long long* __restrict__ colfx, const float* __restrict__ colfac, float* __restrict__ tbuf,
    double* __restrict__ part, unsigned long long* __restrict__ hist, int hash_arg, Lanes L, cresso_hyper h) {
    if (L.dv) {
        const cresso_spectral_desc& d = lane_desc(L);
        grad = (const GT*)d.grad; param = (const PT*)d.param;
    }
    ctrl = lane_at(ctrl, L); lt = lane_at(lt, L); rowfx = lane_at(rowfx, L); colfx = lane_at(colfx, L);
    colfac = lane_at(colfac, L); tbuf = lane_at(tbuf, L); part = lane_at(part, L); hist = lane_at(hist, L);
    constexpr int RW = 2 * RM;
    extern __shared__ __align__(16) unsigned char dyn[];
    __shared__ float red[4 * NV3];
    const SweepFlags F = sweep_flags<MODE>(g, hash_arg, 1, h);
    const Tile t = tile_of(g);
    const int B = g.B;
    const int TB = F.T * B;
    const int nr = (int)(t.r1 - t.r0);
    const int64_t base = panel_base(g, t);
    const GT* __restrict__ gb = grad + base;
    float* __restrict__ tb = tbuf + base;
    // MODE 1: the first batch's loads go out before the set-up below
    PanelBuf gbv, bnv, tbv;
    float x0[SP_U];
    uint32_t b0[SP_U];
    if constexpr (MODE == 1) {
        gbv = panel_buf(gb, g, nr);
        bnv = panel_buf(reinterpret_cast<const uint16_t*>(bins) + base, g, nr);
        tbv = panel_buf(tb, g, nr);
#pragma unroll
        for (int u = 0; u < SP_U; ++u) {
            x0[u] = ldb_lane<GT>(gbv, u);
            b0[u] = ldb_bins16(bnv, u);
        }
    }
    // LDS: histogram [T][B] u64 | log hash metric [T][B] | row metric factor [PR]
    //      | row reconstruction coefficients [PR][2][KP] (16-byte aligned) | row factors [PR][RW]
    unsigned long long* s_hist = reinterpret_cast<unsigned long long*>(dyn);
    float* s_lt = reinterpret_cast<float*>(dyn + sizeof(unsigned long long) * SP_NHIST * (size_t)TB);
    constexpr int NH = MODE == 1 ? SP_NHIST : 1;   // histogram copies in use
    const int hc = MODE == 1 ? (int)(threadIdx.x & (SP_NHIST - 1)) : 0;
    float* s_rf = s_lt + TB;
    const float eps = (float)h.eps;
    const float kappa = ctrl->kappa, gden = ctrl->gden;
    const bool inst_on = MODE == 1 ? true : kappa != 0.0f;
    if (F.hash_on)
        for (int i = threadIdx.x; i < TB; i += SP_NT) {
            s_lt[i] = lt[i];
#pragma unroll
            for (int c = 0; c < NH; ++c) s_hist[i * NH + c] = 0ull;
        }
    for (int lr = threadIdx.x; lr < nr; lr += SP_NT)
        s_rf[lr] = (inst_on && !g.one_d) ? marg_factor(rowfx[t.r0 + lr], 1.0 / (g.hs_row * (double)g.cols), gden, kappa, eps) : 1.0f;
    // the lane's column carriers and the rows' coefficients of the metric
    // field (set 0) and the prediction (set 1)
    constexpr int KP = kcp<KC>();
    float bc[KC];
    load_cols<KC>(g, coltab, t, bc);
    float* s_al = reinterpret_cast<float*>(dyn + lds_al_off(g));
    // the rows' factors a_q of the t projection, staged with the coefficients
    // (uniform LDS reads in the loop instead of scalar loads of every row)
    float* s_ar = s_al + 2 * KP * g.PR;
    stage_rows<RM>(g, rowtab, t.r0, nr, s_ar);
    {
        const float (*const r0[2])[2] = {ctrl->rc[0], ctrl->rc[1]};
        const float (*const r1[2])[2] = {nullptr, nullptr};
        const float w0[2] = {1.f, 1.f}, w1[2] = {0.f, 0.f};
        alpha_rows<RM, KC>(g, meta, s_ar, nr, r0, w0, r1, w1, s_al);
    }
    const float cM = ctrl->rconst[0], cP = ctrl->rconst[1];
    __syncthreads();
    const PT* __restrict__ pb = param + base;
    const float inv_s = ctrl->inv_s, scale = ctrl->scale;
    const float mcoup = (float)h.metric_coupling;
    const float wd = (float)h.weight_decay;
    const float sg = h.maximize ? -1.f : 1.f;
    const float ls = (float)h.local_sharpness;
    const float ipw = (float)fmax(h.instant_metric_power, 0.25);
    float ec = 1.0f;
    if (inst_on && !g.one_d && t.colok)
        ec = g.ntrail == 1 ? marg_factor(colfx[t.col], 1.0 / (g.hs_col * (double)g.rows), gden, kappa, eps) : colfac[t.col];
    const float invT = 1.0f / (float)F.T;
    const float tm = (float)h.transport_mix;
    const float hs = (float)ctrl->hs_P;
    const float clip = (float)h.drive_clip, iclip = 1.0f / clip, clip2 = clip * clip;
    const float k2 = -2.8853900817779268f * iclip;   // -2 log2(e) / clip
    // Only t is projected: the port P = (1 + tm) t - pred projects to
    // (1 + tm) mean(t Xn) - G u_pred, formed in fin3 from the Gram matrix.
    float ZT[RW];
#pragma unroll
    for (int q = 0; q < RW; ++q) ZT[q] = 0.f;
    float m_ee = 0.f, m_t = 0.f, m_tt = 0.f, m_rr = 0.f, m_bb = 0.f, m_oo = 0.f, m_rb = 0.f, m_ro = 0.f,
          m_bo = 0.f, m_tr = 0.f, m_tb = 0.f, m_to = 0.f;
    // MODE 1 panel views (full tile)
    // one row of the lane's column: f -> t (stored), moments, projection, histogram
    auto row = [&](int lr, float gval, float pval, uint64_t bval) {
                float f = sg * gval;
                if (F.wd_on) f = f + wd * pval;
                const float* __restrict__ ar = s_ar + lr * RW;
                // metric field exp(c * clamp(recon(metric), +-3)) clamped (cresso_v5.py:1090-1093)
                const float* __restrict__ al = s_al + lr * (2 * KP);
                float lm = cM;
#pragma unroll
                for (int k = 0; k < KC; ++k) lm = fmaf(al[k], bc[k], lm);
                lm = med3f(lm, -3.0f, 3.0f);
                const float M = med3f(fexp(mcoup * lm), 0.06f, 16.0f);
                float den = scale * M;
                if (F.ls_on) {
                    const float rel = fminf(fabsf(f) * inv_s + eps, 1.0e4f);
                    den = den * clampf(1.0f + ls * fsqrt(fminf(rel, 100.0f)), 1.0f, 8.0f);
                }
                if (inst_on) {
                    float I;
                    if (MODE == 0 && g.one_d) {
                        const float rel = fmaxf(fminf(fabsf(f) * inv_s + eps, 1.0e4f), eps);
                        const float dens = fminf(ipw == 1.0f ? rel : fpow(rel, ipw), 1.0e6f);
                        I = fexp(kappa * flog(fmaxf(dens / gden, eps)));
                    } else {
                        I = s_rf[lr] * ec;
                    }
                    den = den * med3f(I, 0.08f, 12.0f);
                }
                if (F.hash_on) {
                    float lsum = 0.f;
#pragma unroll
                    for (int tt = 0; tt < SP_MAXT; ++tt) {
                        if (tt >= F.T) break;
                        lsum += s_lt[tt * B + bin_of(bval, tt, F.bpb)];
                    }
                    den = den * med3f(fexp(lsum * invT), 0.08f, 12.0f);
                }
                const float tv = med3f(f * frcp(den + eps), -1.0e4f, 1.0e4f);
                if (MODE == 1)
                    stb_lane(tbv, lr, tv);
                else
                    tb[panel_off(g, lr)] = tv;
                float pred = cP;
#pragma unroll
                for (int k = 0; k < KC; ++k) pred = fmaf(al[KP + k], bc[k], pred);
                const float err = tv - pred;
                const float P = err + tm * tv;
                m_ee += err * err;
                m_t += tv;
                m_tt += tv * tv;
                // |rat|, |tanh|, |root| share the sign of t: the moments take
                // magnitudes, and fin3 scales the tanh ones by clip (bnd = clip tanh)
                const float at = fabsf(tv);
                const Shape3A z = shape3a(at, k2, iclip, clip2, eps);
                m_rr = fmaf(z.rat, z.rat, m_rr); m_bb = fmaf(z.th, z.th, m_bb); m_oo = fmaf(z.root, z.root, m_oo);
                m_rb = fmaf(z.rat, z.th, m_rb); m_ro = fmaf(z.rat, z.root, m_ro); m_bo = fmaf(z.th, z.root, m_bo);
                m_tr = fmaf(at, z.rat, m_tr); m_tb = fmaf(at, z.th, m_tb); m_to = fmaf(at, z.root, m_to);
#pragma unroll
                for (int q = 0; q < RW; ++q) ZT[q] += ar[q] * tv;
                if (F.hash_on) {
                    const unsigned long long v = to_fixed_s(P * hs);
#pragma unroll
                    for (int tt = 0; tt < SP_MAXT; ++tt) {
                        if (tt >= F.T) break;
                        atomicAdd(&s_hist[(tt * B + bin_of(bval, tt, F.bpb)) * NH + hc], v);
                    }
                }
                if (MODE == 1) {
                    // this row's contributions are complete here
#pragma unroll
                    for (int q = 0; q < RW; ++q) pin1(ZT[q]);
                    pin1(m_ee); pin1(m_t); pin1(m_tt); pin1(m_rr); pin1(m_bb); pin1(m_oo);
                    pin1(m_rb); pin1(m_ro); pin1(m_bo); pin1(m_tr); pin1(m_tb); pin1(m_to);
                }
                elem_fence();
    };
    if constexpr (MODE == 1) {
        // full tile: no guards, next rows' loads in flight during these rows
        pipelined_rows<SP_U>(
            nr,
            [&](int lr, float& x, uint32_t& b) {
                x = ldb_lane<GT>(gbv, lr);
                b = ldb_bins16(bnv, lr);
            },
            [&](int lr, float x, uint32_t b) { row(lr, x, 0.f, b); }, x0, b0);
    } else if (t.colok) {
        for (int i0 = 0; i0 < nr; i0 += SP_U) {
            float gv[SP_U], pv[SP_U];
            uint64_t bv[SP_U];
#pragma unroll
            for (int u = 0; u < SP_U; ++u) {
                gv[u] = 0.f;
                pv[u] = 0.f;
                bv[u] = 0;
                if (i0 + u < nr) {
                    const uint32_t o = panel_off(g, i0 + u);
                    gv[u] = to_f(gb[o]);
                    if (F.wd_on) pv[u] = to_f(pb[o]);
                    if (F.hash_on) bv[u] = load_bins_at(bins, base, o, F.binbytes);
                }
            }
#pragma unroll
            for (int u = 0; u < SP_U; ++u) {
                if (i0 + u >= nr) break;
                row(i0 + u, gv[u], pv[u], bv[u]);
            }
        }
    }
    __syncthreads();
    if (F.hash_on)
        for (int i = threadIdx.x; i < TB; i += SP_NT) {
            unsigned long long v = 0ull;
#pragma unroll
            for (int c = 0; c < NH; ++c) v += s_hist[i * NH + c];
            if (v) atomicAdd(&hist[i], v);
        }
    Partials P{red, 15 + 2 * g.R, NV3};
    const float mm[13] = {m_ee, 0.f, m_t, m_tt, m_rr, m_bb, m_oo, m_rb, m_ro, m_bo, m_tr, m_tb, m_to};
#pragma unroll
    for (int k = 0; k < 13; ++k) P.add(k, mm[k]);
    P.add(13, 0.f);
    P.add(14, 0.f);
    proj_finish<RM, KC>(g, meta, ZT, bc, P, 15);
    P.flush(part);
}



// ---------------------------------------------------------------------------
// S3 on the matrix cores (MODE 1 tiles, RM <= 16, TT = 2 or 4 tables of
// one-byte bins).  The element math is sweep3_kernel's; the contractions run
// as v_mfma_f32_16x16x4f32 on 16 x 16 tiles, each wave owning 64 columns of
// the panel as 4 tile columns:
//   metric and prediction fields: 2 KCH MFMAs per tile, KCH = KC / 4 rounded
//     up (column-carrier form, A = the rows' alpha coefficients, B = the
//     columns' carriers);
//   t projection Z_q(col) = sum_rows a_q(row) t(row, col): 4 MFMAs per tile
//     and 16-row tile of q, A[q][k] = a_q(row 4k + r), B[k][col] =
//     t(row 4k + r, col) for the tile's element r of each lane, accumulated
//     over the panel in D[q][col].
// Layouts (lane l, li = l % 16, lg = l / 16): A[i][k] from lane (i = li,
// k = lg), B[k][j] from lane (j = li, k = lg), D[i][j] in lane (j = li),
// register r: i = 4 lg + r.  Lane l processes rows 4 lg + r of column li of
// each tile.  The loads of the next row of tiles are in flight while a row is
// processed.  Up to three chunks of carriers (rank <= 8) the B operands are
// read from an LDS table; more chunks stay in registers (rank 16: 36 per lane,
// within the 256 registers of two waves per SIMD).
// ---------------------------------------------------------------------------
template <int KC> constexpr bool bq_in_regs() { return kch<KC>() > 3; }
template <int RM, int KC, typename GT, int TT>
__global__ __launch_bounds__(SP_NT, (occ3m<RM, KC>())) void sweep3m_kernel(
    Geom g, const GT* __restrict__ grad, const float* __restrict__ rowtab, const float* __restrict__ coltab,
    const ModeMeta* __restrict__ meta, const unsigned char* __restrict__ bins, const Ctrl* __restrict__ ctrl,
    const float* __restrict__ lt, const unsigned long long* __restrict__ rowfx,
    const unsigned long long* __restrict__ colfx, const float* __restrict__ colfac, float* __restrict__ tbuf,
    double* __restrict__ part, unsigned long long* __restrict__ hist, Lanes L, cresso_hyper h, int one_round,
    int hdirect) {
    if (L.dv) grad = (const GT*)lane_desc(L).grad;
    ctrl = lane_at(ctrl, L); lt = lane_at(lt, L); rowfx = lane_at(rowfx, L); colfx = lane_at(colfx, L);
    colfac = lane_at(colfac, L); tbuf = lane_at(tbuf, L); part = lane_at(part, L); hist = lane_at(hist, L);
    static_assert(RM <= 16, "two 16-row tiles of projection rows at most");
    constexpr int RW = 2 * RM;
    constexpr int NQ = nqt<RM>();
    constexpr int KP = kcp<KC>();
    constexpr int KCH = kch<KC>();
    constexpr bool BQR = bq_in_regs<KC>();
    extern __shared__ __align__(16) unsigned char dyn[];
    __shared__ float red[4 * NV3];
    const Tile t = tile_of(g);
    const int B = g.B;
    const int TB = TT * B;
    const int nr = g.PR;
    const int l = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int li = l & 15, lg = l >> 4;
    ProjCols<NQ> pc;
    pc.modes(g, meta, lg, KC);
    const int64_t base = panel_base(g, t);
    const uint32_t cols = (uint32_t)g.cols;
    const __amdgpu_buffer_rsrc_t rg = make_rsrc(grad + base, (uint32_t)((int64_t)nr * g.cols * (int64_t)sizeof(GT)));
    // t goes to the field in the 4-row interleaved layout (q4_base): a lane's
    // four rows of a tile are one float4, and a wave's store writes whole lines
    const __amdgpu_buffer_rsrc_t rt = make_rsrc(tbuf + q4_base(g, t), (uint32_t)((int64_t)nr * g.cols * 4));
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(bins + (size_t)TT * base, (uint32_t)((int64_t)nr * g.cols * TT));
    const uint32_t lane_el = 4u * (uint32_t)lg * cols + 64u * (uint32_t)wv + (uint32_t)li;  // element offset
    const uint32_t vg = lane_el * (uint32_t)sizeof(GT), vb = lane_el * (uint32_t)TT;
    const uint32_t vt = q4_lane_bytes(cols, lg, wv, li);
    // tile (tr, tc), lane element r: panel element (16 tr + 4 lg + r, 64 wv + 16 tc + li)
    auto tile_off = [&](int tr, int tc, int r) -> uint32_t { return (uint32_t)(16 * tr + r) * cols + 16u * tc; };
    // one register set, refilled tile by tile: the loads of tile (tr + 1, tc)
    // go out as soon as tile (tr, tc) is done, three tiles ahead of their use
    float xv[16];
    uint32_t bv[16];
    auto load_tile = [&](int tr, int tc) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t o = tile_off(tr, tc, r);
            xv[4 * tc + r] = ldg_el<GT>(rg, vg, o * (uint32_t)sizeof(GT));
            bv[4 * tc + r] = ldg_bins<TT>(rb, vb, o * (uint32_t)TT);
        }
    };
#pragma unroll
    for (int tc = 0; tc < 4; ++tc) load_tile(0, tc);
    // LDS as sweep3_kernel: histogram copies [TB][NH] u64 | log hash metric [TB]
    //      | row metric factor [PR] | (16-aligned) alpha [PR][2][KP] | row factors [PR][RW]
    constexpr int NH = SP_NHIST;
    const int hc = (int)(threadIdx.x & (SP_NHIST - 1));
    unsigned long long* s_hist = reinterpret_cast<unsigned long long*>(dyn);
    float* s_lt = reinterpret_cast<float*>(dyn + sizeof(unsigned long long) * SP_NHIST * (size_t)TB);
    float* s_rf = s_lt + TB;
    float* s_al = reinterpret_cast<float*>(dyn + lds_al_off(g));
    float* s_ar = s_al + 2 * KP * g.PR;
    const float eps = (float)h.eps;
    const float kappa = ctrl->kappa, gden = ctrl->gden;
    // every set-up load goes out here, behind the first tiles' loads: the
    // coefficient sources, exp(lt / T), the row factors and axis sums, the
    // column carriers (B operands and the projection finish's) and axis sums
    const float (*const rcm0[2])[2] = {ctrl->rc[0], ctrl->rc[1]};
    const float (*const rcm1[2])[2] = {nullptr, nullptr};
    const float wm0[2] = {1.f, 1.f}, wm1[2] = {0.f, 0.f};
    const CmLane<RM> cs = cm_lane<RM>(g, meta, rcm0, wm0, rcm1, wm1);
    constexpr int NLT = TT, NRW = (64 * RW + SP_NT - 1) / SP_NT;
    Staged<NLT> slt;
    slt.load(lt, TB);
    Staged<NRW> srw;
    srw.template load_rows<RM>(g, rowtab, t.r0, nr);
    const unsigned long long rfx = rowfx[t.r0 + ((int)threadIdx.x < nr ? (int)threadIdx.x : nr - 1)];
    const int64_t colw = (int64_t)t.slab * SP_NT + 64 * wv;
    const int64_t c_own = (int64_t)t.slab * SP_NT + threadIdx.x;
    // the column's axis sum (2-D) or factor (more dims): both loads issued,
    // the unused one through an empty buffer range (reads 0, no branch)
    const bool two_d = g.ntrail == 1;
    const u32x2 cfx2 = bload2u(make_rsrc(colfx + (int64_t)t.slab * SP_NT, two_d ? SP_NT * 8u : 0u), threadIdx.x * 8u, 0);
    const float cfac = bload1(make_rsrc(colfac + (int64_t)t.slab * SP_NT, two_d ? 0u : SP_NT * 4u), threadIdx.x * 4u, 0);
    const unsigned long long cfx = ((unsigned long long)cfx2[1] << 32) | cfx2[0];
    float bqr[BQR ? 4 : 1][BQR ? KCH : 1];
    if constexpr (BQR) {
#pragma unroll
        for (int tc = 0; tc < 4; ++tc)
#pragma unroll
            for (int kc = 0; kc < KCH; ++kc) {
                const int k = 4 * kc + lg;
                bqr[tc][kc] = coltab[(size_t)(k < KC ? k : 0) * g.cols + colw + 16 * tc + li];
                if (k >= KC) bqr[tc][kc] = 0.f;
            }
    }
    const float lts = 1.4426950408889634f / (float)TT;
    auto exp_lt = [&](float v) { return fexp2(v * lts); };   // exp(lt / T)
    slt.store(s_lt, TB, exp_lt);
    stage_rest<NLT>(s_lt, lt, TB, exp_lt);
    for (int i = threadIdx.x; i < TB; i += SP_NT) {
#pragma unroll
        for (int c = 0; c < NH; ++c) s_hist[i * NH + c] = 0ull;
    }
    // the projection finish's carriers (their rows come from the mode table,
    // in registers by now); first used after the loop
    if constexpr (BQR) pc.load(g, coltab, colw, li);
    const double irow = 1.0 / (g.hs_row * (double)g.cols);
    if ((int)threadIdx.x < nr) s_rf[threadIdx.x] = marg_factor(rfx, irow, gden, kappa, eps);
    for (int lr = threadIdx.x + SP_NT; lr < nr; lr += SP_NT) s_rf[lr] = marg_factor(rowfx[t.r0 + lr], irow, gden, kappa, eps);
    srw.store(s_ar, nr * RW);
    stage_rows_rest<RM, NRW>(g, rowtab, t.r0, nr, s_ar);
    // the block's column instant-metric factors in LDS [SP_NT], after the
    // column carriers (B operands of the reconstructions) when those are in
    // LDS too: [KP][SP_BQS] (rows padded so that the 4 lane groups of a wave
    // read distinct banks)
    float* s_bq = s_ar + RW * g.PR;
    float* s_ec = s_bq + (BQR ? 0 : KP * SP_BQS);
    if constexpr (!BQR) {
#pragma unroll
        for (int k = 0; k < KP; ++k) s_bq[k * SP_BQS + threadIdx.x] = k < KC ? coltab[(size_t)k * g.cols + c_own] : 0.f;
    }
    s_ec[threadIdx.x] = two_d ? marg_factor(cfx, 1.0 / (g.hs_col * (double)g.rows), gden, kappa, eps) : cfac;
    const float* __restrict__ bql = s_bq + lg * SP_BQS + 64 * wv + li;   // + 4 kc SP_BQS + 16 tc
    const float* __restrict__ ecl = s_ec + 64 * wv + li;                  // + 16 tc
    alpha_rows_m<RM, KC>(g, cs, s_ar, nr, s_al);   // ends with a barrier
    const float cM = ctrl->rconst[0], cP = ctrl->rconst[1];
    // the force's sign (maximize) rides on the denominator: f / den = grad / (sign den)
    const float sg = h.maximize ? -1.f : 1.f;
    const float scale_s = sg * ctrl->scale, eps_s = sg * eps;
    const float kM = (float)h.metric_coupling * 1.4426950408889634f;   // exp(c x) = exp2((c log2 e) x)
    const float tm = (float)h.transport_mix;
    const float hs = (float)ctrl->hs_P;
    const float clip = (float)h.drive_clip, iclip = 1.0f / clip, clip2 = clip * clip;
    const float k2 = -2.8853900817779268f * iclip;   // -2 log2(e) / clip
    f32x4m zacc[NQ][4];
#pragma unroll
    for (int qt = 0; qt < NQ; ++qt)
#pragma unroll
        for (int tc = 0; tc < 4; ++tc) zacc[qt][tc] = f32x4m{0.f, 0.f, 0.f, 0.f};
    float m_ee = 0.f, m_t = 0.f, m_tt = 0.f, m_rr = 0.f, m_bb = 0.f, m_oo = 0.f, m_rb = 0.f, m_ro = 0.f,
          m_bo = 0.f, m_tr = 0.f, m_tb = 0.f, m_to = 0.f;
    // metric and prediction fields of tile column tc of the current row of tiles
    float aM[KCH], aQ[KCH];
    auto recon = [&](int tc, f32x4m& lm, f32x4m& pred) {
        lm = f32x4m{cM, cM, cM, cM};
        pred = f32x4m{cP, cP, cP, cP};
#pragma unroll
        for (int kc = 0; kc < KCH; ++kc) {
            float bq;
            if constexpr (BQR)
                bq = bqr[tc][kc];
            else
                bq = bql[4 * kc * SP_BQS + 16 * tc];
            lm = __builtin_amdgcn_mfma_f32_16x16x4f32(aM[kc], bq, lm, 0, 0, 0);
            pred = __builtin_amdgcn_mfma_f32_16x16x4f32(aQ[kc], bq, pred, 0, 0, 0);
        }
    };
    // A operands of row of tiles tr: alpha_{4 kc + lg}(row 16 tr + li) of both fields
    auto row_alpha = [&](int tr) {
        const float* __restrict__ alr = s_al + (16 * tr + li) * (2 * KP) + lg;
#pragma unroll
        for (int kc = 0; kc < KCH; ++kc) {
            aM[kc] = alr[4 * kc];
            aQ[kc] = alr[KP + 4 * kc];
        }
    };
    // With registers to spare (two waves per SIMD: rank 16, or carriers held in
    // registers) the tile's LDS reads go first: LDS operations complete in
    // order, so a read issued after histogram atomics waits for them.  The
    // atomics then follow the element math that feeds them, and the moments
    // (the tile's longest VALU stretch) come after the atomics, so the next
    // tile's reads find the LDS queue drained.  At four waves per SIMD the
    // extra live registers spill, and the reads stay beside their uses.
    constexpr bool GATHER = RM > 8 || kch<KC>() > 3;
    auto tile = [&](int tr, int tc, const float* x, const uint32_t* b, const f32x4m& lm, const f32x4m& pred) {
        if constexpr (GATHER) {
            const float ec = ecl[16 * tc];
            float rfv[4], hmv[4], aJv[NQ][4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                rfv[r] = s_rf[16 * tr + 4 * lg + r];
                // hash metric exp(mean over tables of lt) as the product of the tables' exp(lt / T)
                float hm = s_lt[bin_byte<TT>(b[r], 0)];
#pragma unroll
                for (int tt = 1; tt < TT; ++tt) hm *= s_lt[tt * B + bin_byte<TT>(b[r], tt)];
                hmv[r] = hm;
            }
            // A of the projection: a_q(row 16 tr + 4 lg + r), q = 16 qt + li
#pragma unroll
            for (int qt = 0; qt < NQ; ++qt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int q = 16 * qt + li;
                    aJv[qt][r] = q < RW ? s_ar[(16 * tr + 4 * lg + r) * RW + (q < RW ? q : 0)] : 0.f;
                }
            float tvs[4];
            unsigned long long vfx[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                // metric field exp(c * clamp(recon(metric), +-3)) clamped (cresso_v5.py:1090-1093)
                const float M = med3f(fexp2(kM * med3f(lm[r], -3.0f, 3.0f)), 0.06f, 16.0f);
                float den = scale_s * M;
                den = den * med3f(rfv[r] * ec, 0.08f, 12.0f);
                den = den * med3f(hmv[r], 0.08f, 12.0f);
                const float tv = med3f(x[r] * frcp(den + eps_s), -1.0e4f, 1.0e4f);
                tvs[r] = tv;
                const float err = tv - pred[r];
                const float P = err + tm * tv;
                m_ee += err * err;
                m_t += tv;
                m_tt += tv * tv;
                vfx[r] = to_fixed_s(P * hs);
            }
            bstore4(rt, vt, q4_tile_bytes(cols, tr, tc), f32x4{tvs[0], tvs[1], tvs[2], tvs[3]});
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int tt = 0; tt < TT; ++tt) atomicAdd(&s_hist[(tt * B + bin_byte<TT>(b[r], tt)) * NH + hc], vfx[r]);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float at = fabsf(tvs[r]);
                const Shape3A z = shape3a(at, k2, iclip, clip2, eps);
                m_rr = fmaf(z.rat, z.rat, m_rr); m_bb = fmaf(z.th, z.th, m_bb); m_oo = fmaf(z.root, z.root, m_oo);
                m_rb = fmaf(z.rat, z.th, m_rb); m_ro = fmaf(z.rat, z.root, m_ro); m_bo = fmaf(z.th, z.root, m_bo);
                m_tr = fmaf(at, z.rat, m_tr); m_tb = fmaf(at, z.th, m_tb); m_to = fmaf(at, z.root, m_to);
            }
#pragma unroll
            for (int qt = 0; qt < NQ; ++qt)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    zacc[qt][tc] = __builtin_amdgcn_mfma_f32_16x16x4f32(aJv[qt][r], tvs[r], zacc[qt][tc], 0, 0, 0);
            pin1(m_ee); pin1(m_t); pin1(m_tt); pin1(m_rr); pin1(m_bb); pin1(m_oo);
            pin1(m_rb); pin1(m_ro); pin1(m_bo); pin1(m_tr); pin1(m_tb); pin1(m_to);
        } else {
            const float ec = ecl[16 * tc];
            float tvs[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                // metric field exp(c * clamp(recon(metric), +-3)) clamped (cresso_v5.py:1090-1093)
                const float M = med3f(fexp2(kM * med3f(lm[r], -3.0f, 3.0f)), 0.06f, 16.0f);
                float den = scale_s * M;
                den = den * med3f(s_rf[16 * tr + 4 * lg + r] * ec, 0.08f, 12.0f);
                // hash metric exp(mean over tables of lt) as the product of the tables' exp(lt / T)
                float hm = s_lt[bin_byte<TT>(b[r], 0)];
#pragma unroll
                for (int tt = 1; tt < TT; ++tt) hm *= s_lt[tt * B + bin_byte<TT>(b[r], tt)];
                den = den * med3f(hm, 0.08f, 12.0f);
                const float tv = med3f(x[r] * frcp(den + eps_s), -1.0e4f, 1.0e4f);
                tvs[r] = tv;
                const float err = tv - pred[r];
                const float P = err + tm * tv;
                m_ee += err * err;
                m_t += tv;
                m_tt += tv * tv;
                const float at = fabsf(tv);
                const Shape3A z = shape3a(at, k2, iclip, clip2, eps);
                m_rr = fmaf(z.rat, z.rat, m_rr); m_bb = fmaf(z.th, z.th, m_bb); m_oo = fmaf(z.root, z.root, m_oo);
                m_rb = fmaf(z.rat, z.th, m_rb); m_ro = fmaf(z.rat, z.root, m_ro); m_bo = fmaf(z.th, z.root, m_bo);
                m_tr = fmaf(at, z.rat, m_tr); m_tb = fmaf(at, z.th, m_tb); m_to = fmaf(at, z.root, m_to);
                const unsigned long long v = to_fixed_s(P * hs);
#pragma unroll
                for (int tt = 0; tt < TT; ++tt) atomicAdd(&s_hist[(tt * B + bin_byte<TT>(b[r], tt)) * NH + hc], v);
            }
            bstore4(rt, vt, q4_tile_bytes(cols, tr, tc), f32x4{tvs[0], tvs[1], tvs[2], tvs[3]});
            // A of the projection: a_q(row 16 tr + 4 lg + r), q = 16 qt + li
#pragma unroll
            for (int qt = 0; qt < NQ; ++qt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int q = 16 * qt + li;
                    const float aJ = q < RW ? s_ar[(16 * tr + 4 * lg + r) * RW + (q < RW ? q : 0)] : 0.f;
                    zacc[qt][tc] = __builtin_amdgcn_mfma_f32_16x16x4f32(aJ, tvs[r], zacc[qt][tc], 0, 0, 0);
                }
            pin1(m_ee); pin1(m_t); pin1(m_tt); pin1(m_rr); pin1(m_bb); pin1(m_oo);
            pin1(m_rb); pin1(m_ro); pin1(m_bo); pin1(m_tr); pin1(m_tb); pin1(m_to);
        }
        elem_fence();
    };
    const int ntr = nr / 16;
    f32x4m lmA, prA, lmB, prB;
    row_alpha(0);
    recon(0, lmA, prA);
    for (int tr = 0; tr < ntr; ++tr) {
        if (one_round) progress_prio(4 * tr / ntr);
        // the fields of tile (tr, tc + 1), or of (tr + 1, 0), go to the matrix
        // cores before tile (tr, tc)'s element math, which reads the fields
        // issued one tile earlier
#pragma unroll
        for (int tc = 0; tc < 4; ++tc) {
            if (tc < 3) {
                recon(tc + 1, lmB, prB);
            } else if (tr + 1 < ntr) {
                row_alpha(tr + 1);
                recon(0, lmB, prB);
            }
            tile(tr, tc, xv + 4 * tc, bv + 4 * tc, lmA, prA);
            if (tr + 1 < ntr) load_tile(tr + 1, tc);
            lmA = lmB;
            prA = prB;
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < TB; i += SP_NT) {
        unsigned long long v = 0ull;
#pragma unroll
        for (int c = 0; c < NH; ++c) v += s_hist[i * NH + c];
        if (hdirect) {
            // multi-round launch: blocks end at different times, so they add
            // into the SP_HCOPIES histogram copies directly (integer sums)
            if (v) atomicAdd(&hist[(size_t)(blockIdx.x % SP_HCOPIES) * TB + i], v);
        } else {
            hist[(size_t)blockIdx.x * TB + i] = v;   // this block's partial (hpart[block][bin])
        }
    }
    Partials P{red, 15 + 2 * g.R, NV3};
    const float mm[13] = {m_ee, 0.f, m_t, m_tt, m_rr, m_bb, m_oo, m_rb, m_ro, m_bo, m_tr, m_tb, m_to};
#pragma unroll
    for (int k = 0; k < 13; ++k) P.add(k, mm[k]);
    P.add(13, 0.f);
    P.add(14, 0.f);
    if constexpr (!BQR) pc.load_lds(s_bq, SP_BQS, 64 * wv, li);
    pc.finish(g, zacc, red, P.V, 15, wv, lg, li);
    P.flush(part);
}



// ---------------------------------------------------------------------------
// F3: surprise, hash impulse, confidence, contact, and every drive-shaping
// coefficient that does not need the hash prediction's rms
// ---------------------------------------------------------------------------
// Contact oscillator (cresso_v5.py:914-943) on bank 0 (cos) then bank 1 (sin)
// with the shared action, lane r = mode r; the energy and power sums over
// modes are summed in mode order.  A bank's sums use its own pre-update p and
// q, so both banks' sums are formed first (the six wave reductions in flight
// together); the action, the friction it sets and each bank's update then run
// in bank order.
__device__ void contact_banks_lanes(float (&q)[2], float (&p)[2], const float (&port)[2], float omega,
                                    float (&calcium)[2], float& action, float S, int R, const cresso_hyper& h) {
    const int r = threadIdx.x & 63;
    const bool on = r < R;
    const float dt = (float)h.dt;
    const float rd = (float)h.refractory_decay;
    const float plast = 1.0f + (float)h.surprise_gain * S / (1.0f + S);
    const float brake = 1.0f / (1.0f + (float)h.surprise_brake * S);
    float gp[2] = {0.f, 0.f};
    double e1[2] = {0.0, 0.0}, e2[2] = {0.0, 0.0}, pw[2] = {0.0, 0.0};
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        if (on) {
            calcium[b] = calcium[b] * rd + (float)(1.0 - h.refractory_decay) * fabsf(port[b]);
            const float gate = 1.0f / (1.0f + (float)h.refractory_gain * calcium[b]);
            gp[b] = port[b] * gate * plast * brake;
            e1[b] = (double)(p[b] * p[b]);
            const float oq = omega * q[b];
            e2[b] = (double)(oq * oq);
            pw[b] = (double)(gp[b] * p[b]);
        }
    }
    double E1[2], E2[2], PW[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        E1[b] = lanes_sum(e1[b], R);
        E2[b] = lanes_sum(e2[b], R);
        PW[b] = lanes_sum(pw[b], R);
    }
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        if (R > 0) {
            const double iR = 1.0 / (double)R;
            const float energy = 0.5f * ((float)(E1[b] * iR) + (float)(E2[b] * iR));
            const float power = (float)(PW[b] * iR);
            action = action * 0.985f + dt * (power - energy);
        }
        const float fric = (float)h.impulse_friction + (float)h.contact_gain * tanhf(fabsf(action));
        const float damp = fmaxf(1.0f - dt * fric, 0.0f);
        if (on) {
            float pr = p[b] * damp;
            const float qq = q[b];
            pr = pr + dt * (gp[b] - (float)h.restoring * (omega * omega) * qq - (float)h.cubic * (qq * qq * qq));
            p[b] = pr;
            q[b] = clampf(qq + dt * pr, -8.0f, 8.0f);
        }
    }
}

// The drive (cresso_v5.py:1303-1353) is
//   c0 core + c1 pred' + c2 nov + c3 err' + c4 echo + c5 hash
// with core = cr rat + cb bnd + co root + ct t.  Every c except c5 depends on
// rms values that are closed forms of this step's sweep-3 sums:
//   * mean(core^2): a quadratic form in the 13 moments of t;
//   * mean(pred'^2), mean(echo^2): u^T G u over the Gram matrix G of the
//     normalized basis (pred' and echo are reconstructions with weights u);
//   * mean(t pred') = sum_v u'_v mean(t Xn_v) (the t projection);
//   * mean(err'^2) = mean(err^2) - 2 mean(err D) + mean(D^2), D = pred' - pred
//     a reconstruction with weights du = u' - u, mean(err Xn_v) =
//     mean(t Xn_v) - (G u)_v: small corrections to a directly summed term.
// So sweep 4 can write the drive without c5; the hash term's rms comes from
// sweep 4's sums and is added in sweep 5.
__global__ __launch_bounds__(SP_FN_NT) void fin3_kernel(
    Geom g, const ModeMeta* __restrict__ meta, const double* __restrict__ stats, const double* __restrict__ gram,
    const double* __restrict__ part, unsigned long long* __restrict__ hist,
    const unsigned long long* __restrict__ counts, float* __restrict__ imp_tab, SpecState st, Ctrl* __restrict__ ctrl,
    const unsigned long long* __restrict__ cooc, int step, int hash_on, int hard, int echo_on, int c5_closed, int nc, Lanes L,
    cresso_hyper h) {
    if (L.dv) {
        st = spec_state(lane_desc(L));
        step = lane_desc(L).step;
    }
    part = lane_at(part, L); hist = lane_at(hist, L); imp_tab = lane_at(imp_tab, L); ctrl = lane_at(ctrl, L);
    if (threadIdx.x == 0) ctrl->de_prev = *st.drive_energy;   // every block of sweep 5 reads the old value
    __shared__ double s_m[NV3];
    __shared__ double s_ec[2 * SP_MAXR];    // mean(t Xn_v)
    __shared__ double s_u[3][2 * SP_MAXR];  // weights of pred, pred', echo
    __shared__ float s_wp[2 * SP_MAXR], s_we[2 * SP_MAXR];
    __shared__ float s_tmpf[64];
    const int tid = threadIdx.x;
    const int R = g.R, V = 2 * g.R;
    // everything the mode lanes read, staged in LDS by all threads (global
    // loads in flight together instead of one round trip per use)
    __shared__ double s_gram[4 * SP_MAXR * SP_MAXR];
    __shared__ double s_stats[4 * SP_MAXR];
    __shared__ float s_mode[SP_MAXR][9];
    __shared__ float s_scal[2];
    __shared__ float s_impv[2 * 256];
    __shared__ double s_hhw[SP_FN_NT / 64];
    __shared__ float s_srms;
    __shared__ unsigned int s_sync;
    if (tid == 0) s_sync = 0u;   // published by the staging barrier
    // every staged value is loaded first (clamped, in-bounds indices: the
    // loads are in flight together), then stored to LDS
    constexpr int NG = 4 * SP_MAXR * SP_MAXR / SP_FN_NT;   // Gram values per thread at most
    static_assert(NG * SP_FN_NT == 4 * SP_MAXR * SP_MAXR && 9 * SP_MAXR <= SP_FN_NT && NV3 <= SP_FN_NT,
                  "staged values per thread");
    const int VV = V * V, NS = 15 + 2 * R;
    double v_gr[NG];
#pragma unroll
    for (int u = 0; u < NG; ++u) {
        const int i = tid + u * SP_FN_NT;
        v_gr[u] = gram[i < VV ? i : 0];
    }
    const double v_st = stats[tid < 4 * R ? tid : 0];
    const int mi = tid < 9 * R ? tid : 0, mr = mi / 9, mj = mi - 9 * mr;
    const float* src[8] = {st.omega, st.q_cos, st.q_sin, st.p_cos, st.p_sin, st.calcium_cos, st.calcium_sin, st.conf};
    const float v_md = src[mj < 8 ? mj : 0][mr];
    const double v_wp = (double)ctrl->wpred[tid < V ? tid : 0];
    const float v_sur = *st.surprise, v_act = *st.action;
    const double v_sum = part[tid < NS ? tid : 0];
#pragma unroll
    for (int u = 0; u < NG; ++u) {
        const int i = tid + u * SP_FN_NT;
        if (i < VV) s_gram[i] = v_gr[u];
    }
    if (tid < 4 * R) s_stats[tid] = v_st;
    if (tid < 9 * R) s_mode[mr][mj] = mj < 8 ? v_md : 0.f;
    if (tid < V) s_u[0][tid] = v_wp;
    if (tid == 0) {
        s_scal[0] = v_sur;
        s_scal[1] = v_act;
    }
    if (tid < NS) s_m[tid] = v_sum;
    __syncthreads();
    const float eps = (float)h.eps;
    __shared__ double s_gu[2 * SP_MAXR];     // G u_pred: mean(pred Xn_v)
    if (tid < 64) {
        const int r = tid;
        const bool on = r < R;
        const double sT = s_m[2];
        // surprise reservoir (cresso_v5.py:1127-1129)
        const float sur = reservoir_f(s_scal[0], sqrtf((float)(s_m[0] * g.inv_n) + eps), h.surprise_decay, step);
        // t projections mean(t Xn) in fp64
        float ecs = 0.f, ess = 0.f;
        if (on) {
            const double mc = s_stats[4 * r], ic = s_stats[4 * r + 1], ms = s_stats[4 * r + 2], is = s_stats[4 * r + 3];
            const double ecd = (s_m[15 + 2 * r] - mc * sT) * ic * g.inv_n;
            const double esd = (s_m[16 + 2 * r] - ms * sT) * is * g.inv_n;
            ecs = (float)ecd;
            ess = (float)esd;
            s_ec[2 * r] = ecd;
            s_ec[2 * r + 1] = esd;
        }
        // mean(pred Xn_v) = (G u_pred)_v, lane v = carrier v
        if (r < V) {
            double gu = 0.0;
#pragma unroll 8
            for (int w = 0; w < V; ++w) gu += s_gram[r * V + w] * s_u[0][w];
            s_gu[r] = gu;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup", "local");   // LDS only: pending global stores need not complete
        // port projections (cresso_v5.py:1136): P = err + tm t = (1 + tm) t - pred
        float pc = 0.f, ps = 0.f;
        if (on) {
            const double k1 = 1.0 + (double)(float)h.transport_mix;
            pc = (float)(k1 * s_ec[2 * r] - s_gu[2 * r]);
            ps = (float)(k1 * s_ec[2 * r + 1] - s_gu[2 * r + 1]);
        }
        float om = 0.f, qc = 0.f, qs = 0.f, pcv = 0.f, psv = 0.f, cac = 0.f, cas = 0.f, conf = 0.f;
        if (on) {
            om = s_mode[r][0]; qc = s_mode[r][1]; qs = s_mode[r][2]; pcv = s_mode[r][3]; psv = s_mode[r][4];
            cac = s_mode[r][5]; cas = s_mode[r][6]; conf = s_mode[r][7];
        }
        // confidence (cresso_v5.py:1199-1202) with the pre-contact q
        float gt = 0.f;
        if (on) {
            const float pe = sqrtf(pc * pc + ps * ps + eps);
            const float sup = (pc * qc + ps * qs) / (pe * sqrtf(qc * qc + qs * qs + eps) + eps);
            const float c = conf * (float)h.confidence_decay + (float)(1.0 - h.confidence_decay) * clampf(sup, -1.0f, 1.0f);
            conf = clampf(c, -4.0f, 4.0f);
            gt = sigmoidf_((float)h.confidence_gain * conf);
        }
        // contact on the cos bank then the sin bank with the shared action
        float action = s_scal[1];
        {
            float qb[2] = {qc, qs}, pb[2] = {pcv, psv}, cb[2] = {cac, cas};
            const float portb[2] = {pc, ps};
            contact_banks_lanes(qb, pb, portb, om, cb, action, sur, R, h);
            qc = qb[0]; qs = qb[1]; pcv = pb[0]; psv = pb[1]; cac = cb[0]; cas = cb[1];
        }
        set_recon_lanes(g, s_stats, ctrl->rc[2], &ctrl->rconst[2], qc, qs, gt, s_tmpf, s_wp);
        if (echo_on) set_recon_lanes(g, s_stats, ctrl->rc[3], &ctrl->rconst[3], ecs, ess, 1.0f, s_tmpf, s_we);
        if (on) {
            st.q_cos[r] = qc; st.q_sin[r] = qs; st.p_cos[r] = pcv; st.p_sin[r] = psv;
            st.calcium_cos[r] = cac; st.calcium_sin[r] = cas; st.conf[r] = conf;
            s_u[1][2 * r] = (double)s_wp[2 * r];
            s_u[1][2 * r + 1] = (double)s_wp[2 * r + 1];
            s_u[2][2 * r] = echo_on ? (double)s_we[2 * r] : 0.0;
            s_u[2][2 * r + 1] = echo_on ? (double)s_we[2 * r + 1] : 0.0;
        }
        if (r == 0) {
            *st.surprise = sur;
            *st.action = action;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup", "local");   // LDS only: pending global stores need not complete
        // Gram products, lane v = carrier v (v < 2R <= 32)
        double q0 = 0.0, q1 = 0.0, q2 = 0.0, q3 = 0.0, q4 = 0.0;
        if (r < V) {
            const int v = r;
            const double gu = s_gu[v];
            double gup = 0.0, gue = 0.0;
#pragma unroll 8
            for (int w = 0; w < V; ++w) {
                const double gvw = s_gram[v * V + w];
                gup += gvw * s_u[1][w];
                gue += gvw * s_u[2][w];
            }
            const double du = s_u[1][v] - s_u[0][v];
            q0 = s_u[1][v] * gup;        // -> mean(pred'^2)
            q1 = s_u[2][v] * gue;        // -> mean(echo^2)
            q2 = du * (gup - gu);        // -> mean(D^2)
            q3 = du * (s_ec[v] - gu);    // -> mean(err D)
            q4 = s_u[1][v] * s_ec[v];    // -> mean(t pred')
        }
        const double Q0 = lanes_sum(q0, V), Q1 = lanes_sum(q1, V), Q2 = lanes_sum(q2, V);
        const double Q3 = lanes_sum(q3, V), Q4 = lanes_sum(q4, V);
        if (r == 0) {
            const float S = sur;
            // shaped / core coefficients from the moments of t (cresso_v5.py:1315-1337)
            // sweep 3 sums |tanh| where the moments use bnd = clip tanh
            const double cl = (double)(float)h.drive_clip;
            const double Stt = s_m[3], Srr = s_m[4], Sbb = s_m[5] * cl * cl, Soo = s_m[6], Srb = s_m[7] * cl;
            const double Sro = s_m[8], Sbo = s_m[9] * cl;
            const double Str = s_m[10], Stb = s_m[11] * cl, Sto = s_m[12];
            const float frms = sqrtf((float)(Stt * g.inv_n) + eps);
            const float rms_rat = sqrtf((float)(Srr * g.inv_n) + eps);
            const float rms_root = sqrtf((float)(Soo * g.inv_n) + eps);
            const float kroot = rms_rat / fmaxf(rms_root, eps);
            const float spike = (float)h.spike_mix / (1.0f + S);
            const float rmix = (hard ? (float)h.root_channel_mix : 0.0f) / (1.0f + 0.5f * S);
            const double ar = (double)((1.0f - rmix) * (1.0f - spike));
            const double ab = (double)((1.0f - rmix) * spike);
            const double ao = (double)(rmix * kroot);
            const double sh2 = ar * ar * Srr + ab * ab * Sbb + ao * ao * Soo + 2.0 * (ar * ab * Srb + ar * ao * Sro + ab * ao * Sbo);
            const float srms = sqrtf((float)(sh2 * g.inv_n) + eps);
            const float dmix = (float)h.direct_force_mix / (1.0f + 0.35f * S);
            const float kdir = srms / fmaxf(frms, eps);
            const double cr = (1.0 - (double)dmix) * ar, cb = (1.0 - (double)dmix) * ab, co = (1.0 - (double)dmix) * ao;
            const double ct = (double)(dmix * kdir);
            const double core2 = cr * cr * Srr + cb * cb * Sbb + co * co * Soo + ct * ct * Stt +
                                 2.0 * (cr * cb * Srb + cr * co * Sro + cb * co * Sbo + ct * cr * Str + ct * cb * Stb + ct * co * Sto);
            // alignment gate and prediction mix (cresso_v5.py:1303-1313)
            const float prms = sqrtf((float)Q0 + eps);
            const float align = clampf((float)Q4 / (frms * prms + eps), -1.0f, 1.0f);
            float agate = clampf((align + 1.0f) * 0.5f, 0.0f, 1.0f);
            // the predicate prms > sqrt(eps) in fp64 (in fp32 it is a rounding
            // tie when mean(pred'^2) is below half an ulp of eps)
            if (!(sqrt(fmax(Q0, 0.0) + h.eps) > sqrt(h.eps))) agate = 0.0f;
            const double warm = h.warmup_steps == 0 ? 1.0 : 1.0 - exp(-(double)step / (double)(h.warmup_steps > 1 ? h.warmup_steps : 1));
            const float mix = (float)(h.prediction_mix * warm) * agate * (1.0f / (1.0f + S));
            // residual feedback: err' rms from the directly summed err rms and the Gram corrections
            const float crms = sqrtf((float)(core2 * g.inv_n) + eps);
            const double ee = fmax(s_m[0] * g.inv_n - 2.0 * Q3 + Q2, 0.0);
            const float erms = sqrtf((float)ee + eps);
            const float kres = crms / fmaxf(erms, eps);
            const float resmix = (float)h.residual_feedback_mix / (1.0f + S);
            float kecho = 0.f;
            if (hard && echo_on) kecho = srms / fmaxf(sqrtf((float)Q1 + eps), eps);
            const double c0 = 1.0 - (double)mix, c1 = mix, c2 = h.novelty_mix, c3 = (double)(resmix * kres);
            const double c4 = hard ? h.echo_mix * (double)kecho : 0.0;
            const float clip = (float)h.drive_clip;
            // drive without the hash term:
            //   c0 cr rat + c0 cb clip tanh + c0 co root + (c0 ct + c3) t + (c1 - c3) pred' + c4 echo + c2 clip tanh(err' ns)
            ctrl->k_rat = (float)(c0 * cr);
            ctrl->k_ths = (float)(c0 * cb * (double)clip);
            ctrl->k_root = (float)(c0 * co);
            ctrl->k_t = (float)(c0 * ct + c3);
            ctrl->k_pred = (float)(c1 - c3);
            ctrl->k_echo = (float)c4;
            ctrl->k_nov = (float)(c2 * (double)clip);
            ctrl->nscale = 1.0f / (clip * (1.0f + S));
            ctrl->srms = srms;
            s_srms = srms;
        }
    } else {
        // waves 1.. while wave 0 runs the mode lanes: hash refractory / impulse
        // (cresso_v5.py:1140-1184)
        const int t1 = tid - 64, n1 = SP_FN_NT - 64;
        // the closed form's co-occurrence and bin counts (fixed per shape) are
        // loaded before the bin work when they fit CPF values per thread
        constexpr int CPF = 10;
        const int BB = g.B * g.B;
        const bool cpf = c5_closed == 1 && BB <= CPF * n1 && 2 * g.B <= n1;
        unsigned long long cpre[CPF], npre = 0ull;
        if (cpf) {
#pragma unroll
            for (int u = 0; u < CPF; ++u) {
                const int k = t1 + u * n1;
                cpre[u] = cooc[k < BB ? k : 0];
            }
            npre = counts[t1 < 2 * g.B ? t1 : 0];
        }
        if (hash_on) {
            const int TB = g.T * g.B;
            for (int i = t1; i < TB; i += n1) {
                const double cnt = fmax((double)counts[i], 1.0);
                const float cp = (float)((double)(long long)take_hist(hist, TB, i, nc) / ctrl->hs_P / cnt);
                const float ref = st.hash_refractory[i] * (float)h.hash_decay + (float)(1.0 - h.hash_decay) * fabsf(cp);
                const float gate = 1.0f / (1.0f + (float)h.refractory_gain * ref);
                const float im =
                    st.hash_impulse[i] * (float)h.hash_impulse_decay + (float)(1.0 - h.hash_impulse_decay) * (cp * gate);
                st.hash_refractory[i] = ref;
                st.hash_impulse[i] = im;
                imp_tab[i] = im;
                if (c5_closed == 1) s_impv[i] = im;
            }
        }
        if (c5_closed == 1) {
            waves_sync(&s_sync, SP_FN_NT / 64 - 1);   // s_impv complete
            // the hash prediction's sum of squares over the field,
            // sum_i ((imp0[b0] + imp1[b1]) / 2)^2, in closed form from the bin
            // and co-occurrence counts
            const int B = g.B;
            double a = 0.0;
            if (cpf) {
#pragma unroll
                for (int u = 0; u < CPF; ++u) {
                    const int k = t1 + u * n1;
                    if (k < BB) a += (double)cpre[u] * (2.0 * (double)s_impv[k / B] * (double)s_impv[B + k % B]);
                }
                if (t1 < 2 * B) a += (double)npre * ((double)s_impv[t1] * (double)s_impv[t1]);
            } else {
                for (int k = t1; k < B * B; k += n1)
                    a += (double)cooc[k] * (2.0 * (double)s_impv[k / B] * (double)s_impv[B + k % B]);
                for (int k = t1; k < 2 * B; k += n1) a += (double)counts[k] * ((double)s_impv[k] * (double)s_impv[k]);
            }
            const double w = wave_total_d(a);
            if ((tid & 63) == 63) s_hhw[(tid >> 6) - 1] = w;
        }
    }
    if (c5_closed == 2 && tid == 0) ctrl->hard_hash = hard;   // four tables: sweep 4m forms the coefficient
    if (c5_closed == 1) {
        __syncthreads();
        if (tid == 0) {
            double hh = 0.0;
            for (int w = 0; w < SP_FN_NT / 64 - 1; ++w) hh += s_hhw[w];
            hh *= 0.25;
            // the hash term's coefficient as fin4_values forms it, from sum hp^2
            const float khp = s_srms / fmaxf(sqrtf((float)(hh * g.inv_n) + eps), eps);
            ctrl->k_hash = (float)(hard ? h.hash_drive_mix * (double)khp : 0.0);
        }
    }
}



// ---------------------------------------------------------------------------
// F3b, four tables: the hash prediction's sum of squares in closed form over
// the impulse tables fin3 wrote, spread over hh4_blocks(g) blocks: block
// 16-row chunk c of pair p sums cooc_p[b][b'] * 2 imp_t[b] imp_t'[b'] over its
// rows (thread b'), the last block sum_t sum_b cnt_t[b] imp_t[b]^2; each block
// writes its fp64 total to ctrl->hh_part (fixed-order wave and block sums), and
// every block of sweep 4m adds them in block order.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void hh4_kernel(Geom g, const unsigned long long* __restrict__ cooc,
                                                  const unsigned long long* __restrict__ counts,
                                                  const float* __restrict__ imp_tab, Ctrl* __restrict__ ctrl, Lanes L) {
    imp_tab = lane_at(imp_tab, L); ctrl = lane_at(ctrl, L);
    __shared__ double s_w[4];
    const int B = g.B, nc = hh4_chunks(g), j = threadIdx.x;
    const int b = blockIdx.x;
    double a = 0.0;
    if (b < 6 * nc) {
        int t0, t1;
        cooc_pair(b / nc, t0, t1);
        const int r0 = 16 * (b % nc);
        if (j < B) {
            // every load first (rows past B clamped to row r0, not added), then the sums in row order
            const unsigned long long* c = cooc + (size_t)(b / nc) * B * B + j;
            const double w1 = (double)imp_tab[t1 * B + j];
            unsigned long long cv[16];
            float iv[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int rr = r0 + r < B ? r0 + r : r0;
                cv[r] = c[(size_t)rr * B];
                iv[r] = imp_tab[t0 * B + rr];
            }
#pragma unroll
            for (int r = 0; r < 16; ++r)
                if (r0 + r < B) a += (double)cv[r] * (2.0 * (double)iv[r] * w1);
        }
    } else {
        // four rows of loads in flight per thread, added in the order k = j, j + 256, ...
        constexpr int U = 4;
        for (int k0 = j; k0 < 4 * B; k0 += 256 * U) {
            unsigned long long cn[U];
            float im[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int k = k0 + 256 * u < 4 * B ? k0 + 256 * u : k0;
                cn[u] = counts[k];
                im[u] = imp_tab[k];
            }
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (k0 + 256 * u < 4 * B) a += (double)cn[u] * ((double)im[u] * (double)im[u]);
        }
    }
    const double w = wave_total_d(a);
    if ((j & 63) == 63) s_w[j >> 6] = w;
    __syncthreads();
    if (j == 0) ctrl->hh_part[b] = ((s_w[0] + s_w[1]) + s_w[2]) + s_w[3];
}

// ---------------------------------------------------------------------------
// S4: drive without the hash term, written over t; sums for the drive energy
// ---------------------------------------------------------------------------
template <int RM, int KC, int MODE>
__global__ __launch_bounds__(SP_NT, RM >= 16 ? 2 : 4) void sweep4_kernel(
    Geom g, const float* __restrict__ rowtab, const float* __restrict__ coltab, const ModeMeta* __restrict__ meta,
    const unsigned char* __restrict__ bins, const Ctrl* __restrict__ ctrl, const float* __restrict__ imp_tab,
    float* __restrict__ tbuf, double* __restrict__ part, int hash_arg, int echo_on, Lanes L, cresso_hyper h) {
    ctrl = lane_at(ctrl, L); imp_tab = lane_at(imp_tab, L); tbuf = lane_at(tbuf, L); part = lane_at(part, L);
    extern __shared__ __align__(16) unsigned char dyn[];
    __shared__ float red[4 * NV4];
    const SweepFlags F = sweep_flags<MODE>(g, hash_arg, 1, h);
    const Tile t = tile_of(g);
    const int B = g.B;
    const int TB = F.T * B;
    const int nr = (int)(t.r1 - t.r0);
    // LDS: impulse table [T][B] | row coefficients [PR][2][KP] of pred' (set 0)
    // and of k_pred pred' + k_echo echo (set 1), 16-byte aligned | row factors [PR][2 RM]
    constexpr int KP = kcp<KC>();
    float* s_imp = reinterpret_cast<float*>(dyn);
    float* s_al = reinterpret_cast<float*>(dyn + ((sizeof(float) * (size_t)g.T * g.B + 15) & ~(size_t)15));
    float* s_rows = s_al + 2 * KP * g.PR;   // the block's row factors [PR][2 RM]
    stage_rows<RM>(g, rowtab, t.r0, nr, s_rows);
    if (F.hash_on)
        for (int i = threadIdx.x; i < TB; i += SP_NT) s_imp[i] = imp_tab[i];
    const float kp = ctrl->k_pred, ke = ctrl->k_echo;
    float bc[KC];
    load_cols<KC>(g, coltab, t, bc);
    {
        const float (*const r0[2])[2] = {ctrl->rc[2], ctrl->rc[2]};
        const float (*const r1[2])[2] = {nullptr, echo_on ? ctrl->rc[3] : nullptr};
        const float w0[2] = {1.f, kp}, w1[2] = {0.f, ke};
        alpha_rows<RM, KC>(g, meta, s_rows, nr, r0, w0, r1, w1, s_al);
    }
    const float cQ = ctrl->rconst[2];
    const float cX = kp * ctrl->rconst[2] + (echo_on ? ke * ctrl->rconst[3] : 0.f);
    __syncthreads();
    const int64_t base = panel_base(g, t);
    float* __restrict__ tb = tbuf + base;
    const float eps = (float)h.eps;
    const float clip = (float)h.drive_clip, iclip = 1.0f / clip, clip2 = clip * clip;
    const float k_rat = ctrl->k_rat, k_ths = ctrl->k_ths, k_root = ctrl->k_root, k_t = ctrl->k_t, k_nov = ctrl->k_nov;
    const float k2 = -2.8853900817779268f * iclip;            // -2 log2(e) / clip
    const float k2n = -2.8853900817779268f * ctrl->nscale;    // tanh(err' nscale)
    const float invT = 1.0f / (float)F.T;
    float a_dd = 0.f, a_dh = 0.f, a_hh = 0.f;
    PanelBuf tbv, bnv;
    if (MODE == 1) {
        tbv = panel_buf(tb, g, nr);
        bnv = panel_buf(reinterpret_cast<const uint16_t*>(bins) + base, g, nr);
    }
    // one row of the lane's column: t -> drive without the hash term (stored over t)
    auto row = [&](int lr, float tv, uint64_t bval) {
        const float* __restrict__ al = s_al + lr * (2 * KP);
        float pred = cQ, mixed = cX;
#pragma unroll
        for (int k = 0; k < KC; ++k) {
            pred = fmaf(al[k], bc[k], pred);
            mixed = fmaf(al[KP + k], bc[k], mixed);
        }
        const float err = tv - pred;
        const float nov = ftanh_k(err, k2n);
        const float at = fabsf(tv);
        const Shape3A z = shape3a(at, k2, iclip, clip2, eps);
        const float core = xorsign(fmaf(k_t, at, fmaf(k_root, z.root, fmaf(k_ths, z.th, k_rat * z.rat))), tv);
        const float d = fmaf(k_nov, nov, core + mixed);
        if (MODE == 1)
            stb_lane(tbv, lr, d);
        else
            tb[panel_off(g, lr)] = d;
        a_dd = fmaf(d, d, a_dd);
        if (F.hash_on) {
            float hp = 0.f;
#pragma unroll
            for (int tt = 0; tt < SP_MAXT; ++tt) {
                if (tt >= F.T) break;
                hp += s_imp[tt * B + bin_of(bval, tt, F.bpb)];
            }
            hp = hp * invT;
            a_dh = fmaf(d, hp, a_dh);
            a_hh = fmaf(hp, hp, a_hh);
        }
        if (MODE == 1) {
            pin1(a_dd); pin1(a_dh); pin1(a_hh);
        }
        elem_fence();
    };
    if constexpr (MODE == 1) {
        float x0[SP_U];
        uint32_t b0[SP_U];
#pragma unroll
        for (int u = 0; u < SP_U; ++u) {
            x0[u] = ldb_lane<float>(tbv, u);
            b0[u] = ldb_bins16(bnv, u);
        }
        pipelined_rows<SP_U>(
            nr,
            [&](int lr, float& x, uint32_t& b) {
                x = ldb_lane<float>(tbv, lr);
                b = ldb_bins16(bnv, lr);
            },
            [&](int lr, float x, uint32_t b) { row(lr, x, b); }, x0, b0);
    } else if (t.colok) {
        for (int i0 = 0; i0 < nr; i0 += SP_U) {
            float tvs[SP_U];
            uint64_t bv[SP_U];
#pragma unroll
            for (int u = 0; u < SP_U; ++u) {
                tvs[u] = 0.f;
                bv[u] = 0;
                if (i0 + u < nr) {
                    const uint32_t o = panel_off(g, i0 + u);
                    tvs[u] = tb[o];
                    if (F.hash_on) bv[u] = load_bins_at(bins, base, o, F.binbytes);
                }
            }
#pragma unroll
            for (int u = 0; u < SP_U; ++u) {
                if (i0 + u >= nr) break;
                row(i0 + u, tvs[u], bv[u]);
            }
        }
    }
    Partials P{red, 3, NV4};
    P.add(0, a_dd);
    P.add(1, a_dh);
    P.add(2, a_hh);
    P.flush(part);
}



// ---------------------------------------------------------------------------
// S4 on the matrix cores (MODE 1 tiles, TT = 2 or 4 tables of one-byte bins).
// Each wave owns 64 columns of the panel as 4 x 4 tiles of 16 x 16 elements.
// A reconstruction of a tile is KCH MFMAs (v_mfma_f32_16x16x4f32, the K = KC
// carriers in chunks of 4):
//   A[i][k] = alpha_{4kc+k}(row i)   lane l supplies i = l % 16, k = l / 16
//   B[k][j] = b_{4kc+k}(col j)       lane l supplies j = l % 16, k = l / 16
//   D[i][j]                          lane l, register r: i = 4 (l / 16) + r, j = l % 16
// so lane l processes rows 4 (l/16) + r of column l % 16 of each tile, and the
// elementwise drive math is unchanged.  The loads of the next tile are in
// flight while a tile is processed.  The hash term's coefficient c5 is known
// here (from the hash prediction's RMS in closed form over the co-occurrence
// counts: fin3 forms it for two tables; for four, every block adds
// hh4_kernel's partials and block 0 publishes c5 for sweep 5), so the full
// drive is written and sum drive^2 is summed directly (sweep4_kernel instead
// writes the drive without the hash term and sums d^2, d hp and hp^2 for
// sweep 5).
// ---------------------------------------------------------------------------
template <int RM, int KC, int TT, bool Q4>
__global__ __launch_bounds__(SP_NT, (occ4m<RM, KC>())) void sweep4m_kernel(
    Geom g, const float* __restrict__ rowtab, const float* __restrict__ coltab, const ModeMeta* __restrict__ meta,
    const unsigned char* __restrict__ bins, Ctrl* __restrict__ ctrl, const float* __restrict__ imp_tab,
    float* __restrict__ tbuf, double* __restrict__ part, int echo_on, Lanes L, cresso_hyper h, int one_round) {
    ctrl = lane_at(ctrl, L); imp_tab = lane_at(imp_tab, L); tbuf = lane_at(tbuf, L); part = lane_at(part, L);
    static_assert(TT == 2 || TT == 4, "two or four tables of one-byte bins");
    extern __shared__ __align__(16) unsigned char dyn[];
    __shared__ float red[4 * NV4];
    const Tile t = tile_of(g);
    const int B = g.B;
    const int TB = TT * B;
    const int nr = g.PR;
    constexpr int KP = kcp<KC>();
    constexpr int KCH = kch<KC>();
    const int l = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int li = l & 15, lg = l >> 4;
    const int64_t base = panel_base(g, t);
    // the field: 4-row interleaved after sweep 3m (Q4), row-major after the general sweep 3
    float* __restrict__ tb = tbuf + (Q4 ? q4_base(g, t) : base);
    const uint32_t cols = (uint32_t)g.cols;
    const __amdgpu_buffer_rsrc_t rt = make_rsrc(tb, (uint32_t)((int64_t)nr * g.cols * 4));
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(bins + (size_t)TT * base, (uint32_t)((int64_t)nr * g.cols * TT));
    const uint32_t lane_el = 4u * (uint32_t)lg * cols + 64u * (uint32_t)wv + (uint32_t)li;  // element offset
    const uint32_t vt = Q4 ? q4_lane_bytes(cols, lg, wv, li) : lane_el * 4u, vb = lane_el * (uint32_t)TT;
    // tile (tr, tc), lane element r: panel element (16 tr + 4 lg + r, 64 wv + 16 tc + li)
    auto tile_off = [&](int tr, int tc, int r) -> uint32_t { return (uint32_t)(16 * tr + r) * cols + 16u * tc; };
    // A row of tiles (4 tiles x 4 elements) is in flight while the previous row
    // is processed; the first row's loads go out before the block's set-up, so
    // that memory is busy during it.
    float xa[16], xb[16];
    uint32_t ba[16], bb[16];
    auto load_row = [&](int tr, float* x, uint32_t* b) {
#pragma unroll
        for (int tc = 0; tc < 4; ++tc) {
            if constexpr (Q4) {
                const f32x4 v = bload4(rt, vt, q4_tile_bytes(cols, tr, tc));
#pragma unroll
                for (int r = 0; r < 4; ++r) x[4 * tc + r] = v[r];
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t o = tile_off(tr, tc, r);
                if constexpr (!Q4) x[4 * tc + r] = bload1(rt, vt, o * 4u);
                b[4 * tc + r] = ldg_bins<TT>(rb, vb, o * (uint32_t)TT);
            }
        }
    };
    load_row(0, xa, ba);
    float* s_imp = reinterpret_cast<float*>(dyn);
    float* s_al = reinterpret_cast<float*>(dyn + ((sizeof(float) * (size_t)g.T * g.B + 15) & ~(size_t)15));
    float* s_rows = s_al + 2 * KP * g.PR;   // the block's row factors [PR][2 RM]
    // set-up loads, all issued behind the first row's: the coefficient
    // sources, the row factors, the impulse table and the B operands
    // (carriers 4 kc + lg of the lane's column in each column tile)
    const float kp = ctrl->k_pred, ke = ctrl->k_echo;
    const float (*const rcm0[2])[2] = {ctrl->rc[2], ctrl->rc[2]};
    const float (*const rcm1[2])[2] = {nullptr, echo_on ? ctrl->rc[3] : nullptr};
    const float wm0[2] = {1.f, kp}, wm1[2] = {0.f, ke};
    const CmLane<RM> cs = cm_lane<RM>(g, meta, rcm0, wm0, rcm1, wm1);
    constexpr int RW = 2 * RM;
    constexpr int NRW = (64 * RW + SP_NT - 1) / SP_NT;
    Staged<NRW> srw;
    srw.template load_rows<RM>(g, rowtab, t.r0, nr);
    Staged<TT> simp;
    simp.load(imp_tab, TB);
    double hhv = 0.0;   // four tables, closed form: hh4_kernel's partial of this thread
    if constexpr (TT == 4) hhv = (int)threadIdx.x < hh4_blocks(g) ? ctrl->hh_part[threadIdx.x] : 0.0;
    const int64_t colw = (int64_t)t.slab * SP_NT + 64 * wv;
    float bq[4][KCH];
#pragma unroll
    for (int tc = 0; tc < 4; ++tc)
#pragma unroll
        for (int kc = 0; kc < KCH; ++kc) {
            const int k = 4 * kc + lg;
            bq[tc][kc] = coltab[(size_t)(k < KC ? k : 0) * g.cols + colw + 16 * tc + li];
            if (k >= KC) bq[tc][kc] = 0.f;
        }
    srw.store(s_rows, nr * RW);
    stage_rows_rest<RM, NRW>(g, rowtab, t.r0, nr, s_rows);
    simp.store(s_imp, TB);
    stage_rest<TT>(s_imp, imp_tab, TB, [](float x) { return x; });
    alpha_rows_m<RM, KC>(g, cs, s_rows, nr, s_al);
    const float cQ = ctrl->rconst[2];
    const float cX = kp * ctrl->rconst[2] + (echo_on ? ke * ctrl->rconst[3] : 0.f);
    __syncthreads();
    const float eps = (float)h.eps;
    const float clip = (float)h.drive_clip, iclip = 1.0f / clip, clip2 = clip * clip;
    const float k_rat = ctrl->k_rat, k_ths = ctrl->k_ths, k_root = ctrl->k_root, k_t = ctrl->k_t, k_nov = ctrl->k_nov;
    const float k2 = -2.8853900817779268f * iclip;
    const float k2n = -2.8853900817779268f * ctrl->nscale;
    float c5 = 0.f;
    if constexpr (TT == 2) c5 = ctrl->k_hash;   // set by fin3 (closed-form hash-term RMS)
    if constexpr (TT == 4) {
        // sum hp^2 = (hh4_kernel's partials, added in block order) / T^2, and
        // the coefficient as fin3 forms it for two tables
        __shared__ double s_hh[SP_NT / 64];
        const double w = wave_total_d(hhv);
        if (l == 63) s_hh[wv] = w;
        __syncthreads();
        const double hh = (((s_hh[0] + s_hh[1]) + s_hh[2]) + s_hh[3]) * (1.0 / 16.0);
        const float khp = ctrl->srms / fmaxf(sqrtf((float)(hh * g.inv_n) + eps), eps);
        c5 = (float)(ctrl->hard_hash ? h.hash_drive_mix * (double)khp : 0.0);
        if (blockIdx.x == 0 && threadIdx.x == 0) ctrl->k_hash = c5;   // for sweep 5 (fin4_values)
    }
    constexpr float invT = 1.0f / (float)TT;
    float a_dd = 0.f;
    auto tile = [&](int tr, int tc, const float* x, const uint32_t* b, const float* aP, const float* aX) {
        f32x4m pred = {cQ, cQ, cQ, cQ}, mixed = {cX, cX, cX, cX};
        float dv[4];
#pragma unroll
        for (int kc = 0; kc < KCH; ++kc) {
            pred = __builtin_amdgcn_mfma_f32_16x16x4f32(aP[kc], bq[tc][kc], pred, 0, 0, 0);
            mixed = __builtin_amdgcn_mfma_f32_16x16x4f32(aX[kc], bq[tc][kc], mixed, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float tv = x[r];
            const float err = tv - pred[r];
            const float at = fabsf(tv);
            Shape3A z;
            const float nov = shape3a_nov(at, err, k2, k2n, iclip, clip2, eps, z);
            const float core = xorsign(fmaf(k_t, at, fmaf(k_root, z.root, fmaf(k_ths, z.th, k_rat * z.rat))), tv);
            float hp = s_imp[bin_byte<TT>(b[r], 0)];
#pragma unroll
            for (int tt = 1; tt < TT; ++tt) hp += s_imp[tt * B + bin_byte<TT>(b[r], tt)];
            hp = hp * invT;
            const float d = fmaf(c5, hp, fmaf(k_nov, nov, core + mixed[r]));
            if constexpr (Q4)
                dv[r] = d;
            else
                bstore1(rt, vt, tile_off(tr, tc, r) * 4u, d);
            a_dd = fmaf(d, d, a_dd);
        }
        if constexpr (Q4) bstore4(rt, vt, q4_tile_bytes(cols, tr, tc), f32x4{dv[0], dv[1], dv[2], dv[3]});
        pin1(a_dd);
        elem_fence();
    };
    auto row_tiles = [&](int tr, const float* x, const uint32_t* b) {
        if (one_round) progress_prio(64 * tr / nr);   // rows of tiles done of nr / 16
        // A operands of this row of tiles: alpha_{4 kc + lg}(row 16 tr + li)
        const float* __restrict__ alr = s_al + (16 * tr + li) * (2 * KP) + lg;
        float aP[KCH], aX[KCH];
#pragma unroll
        for (int kc = 0; kc < KCH; ++kc) {
            aP[kc] = alr[4 * kc];
            aX[kc] = alr[KP + 4 * kc];
        }
#pragma unroll
        for (int tc = 0; tc < 4; ++tc) tile(tr, tc, x + 4 * tc, b + 4 * tc, aP, aX);
    };
    const int ntr = nr / 16;   // even: PR is a multiple of 32 on this path
    for (int tr = 0; tr < ntr; tr += 2) {
        load_row(tr + 1, xb, bb);
        row_tiles(tr, xa, ba);
        if (tr + 2 < ntr) load_row(tr + 2, xa, ba);
        row_tiles(tr + 1, xb, bb);
    }
    Partials P{red, 1, 1};   // sum drive^2 only: rows of one value (sweep4_kernel's rows hold NV4)
    P.add(0, a_dd);
    P.flush(part);
}



// Sweep 5 after the matrix-core sweeps, whose drive field is 4-row
// interleaved (q4_base): a thread takes four rows by four columns at a time,
// the drive as four float4 (one per column) and the param as four vectors of
// four (one per row), transposed in registers; params not aligned for vector
// access take one column of four rows at a time.  Same grid as sweep 5.
template <typename PT, bool VEC>
__global__ __launch_bounds__(SP_NT) void sweep5q_kernel(Geom g, PT* __restrict__ param, const float* __restrict__ dbuf,
                                                        const Ctrl* __restrict__ ctrl, const double* __restrict__ part,
                                                        float* __restrict__ de_state, int step, int hash_on, int hard,
                                                        int c5_closed, Lanes L, cresso_hyper h);

// F4, in every block of sweep 5: sweep 4's block partials summed in a fixed
// order (so every block gets the same values), then the hash-term
// coefficient, the drive-energy reservoir and the gain.  Block 0 stores the
// new drive energy; the reservoir starts from ctrl->de_prev (stashed by fin3),
// so no block reads a value another block of this launch wrote.
//   sum drive^2 = sum d^2 + 2 c5 sum d hp + c5^2 sum hp^2
__device__ void fin4_values(const Geom& g, const double* __restrict__ part, const Ctrl* __restrict__ ctrl,
                            float* __restrict__ de_state, int step, int hash_on, int hard, int c5_closed,
                            const cresso_hyper& h, float& gain, float& c5f) {
    __shared__ double s_w[SP_NT / 64][NV4];
    double acc[NV4] = {0.0, 0.0, 0.0};
    // blocks threadIdx.x + i SP_NT in groups of NG: a group's loads go out
    // together (indices clamped: no branch between them), then are summed in
    // block order.  With the closed-form hash term sweep 4m writes rows of one
    // value (sum drive^2), sweep4_kernel rows of NV4.
    constexpr int NG = 8;
    const int nv = c5_closed ? 1 : NV4;
    for (int b0 = threadIdx.x; b0 < g.nblk; b0 += NG * SP_NT) {
        double pv[NG][NV4];
#pragma unroll
        for (int i = 0; i < NG; ++i) {
            const int b = b0 + i * SP_NT < g.nblk ? b0 + i * SP_NT : g.nblk - 1;
#pragma unroll
            for (int v = 0; v < NV4; ++v) pv[i][v] = v < nv ? part[(size_t)b * nv + v] : 0.0;
        }
#pragma unroll
        for (int i = 0; i < NG; ++i)
            if (b0 + i * SP_NT < g.nblk)
#pragma unroll
                for (int v = 0; v < NV4; ++v) acc[v] += pv[i][v];
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int v = 0; v < NV4; ++v) {
        const double w = wave_total_d(acc[v]);
        if (lane == 63) s_w[wave][v] = w;
    }
    __syncthreads();
    double m[NV4];
#pragma unroll
    for (int v = 0; v < NV4; ++v) {
        m[v] = 0.0;
        for (int w = 0; w < SP_NT / 64; ++w) m[v] += s_w[w][v];
    }
    const float eps = (float)h.eps;
    double c5, dd;
    if (c5_closed) {
        // sweep 4 summed the full drive (the hash term's coefficient came from fin3)
        c5 = (double)ctrl->k_hash;
        dd = m[0];
    } else {
        float khp = 0.f;
        if (hard && hash_on) khp = ctrl->srms / fmaxf(sqrtf((float)(m[2] * g.inv_n) + eps), eps);
        c5 = hard ? h.hash_drive_mix * (double)khp : 0.0;
        dd = m[0] + 2.0 * c5 * m[1] + c5 * c5 * m[2];
    }
    const float de_now = (float)(fmax(dd, 0.0) * g.inv_n);
    const float de = reservoir_f(ctrl->de_prev, de_now, h.reservoir_decay, step);
    if (blockIdx.x == 0 && threadIdx.x == 0) *de_state = de;
    c5f = (float)c5;
    gain = clampf((float)h.target_update_rms / sqrtf(de + eps), (float)h.min_gain, (float)h.max_gain);
}

// ---------------------------------------------------------------------------
// S5: parameter update, param -= lr * cast(drive * gain) (cresso_v5.py:1353)
// ---------------------------------------------------------------------------
template <typename PT>
__device__ __forceinline__ void apply1(PT* __restrict__ param, int64_t e, float drive, float gain, float nlr) {
    const float u = to_f(from_w<PT>(drive * gain));
    param[e] = from_w<PT>(to_f(param[e]) + nlr * u);
}
// sweep 5's param loads for the fp32 update (fp64 params are read where the
// fp64 update is formed)
template <typename PT> __device__ __forceinline__ void pre4(const PT* __restrict__ p, int64_t e, float* o) {
    if constexpr (!std::is_same<PT, double>::value) Ld4<PT>::go(p, e, o);
}
// fp64 params: the step's drive and gain come from the fp32 sweeps; the
// update p + (-lr) (drive gain) is formed in fp64 as the reference's fp64
// add_ forms it (cresso_v5.py:1353)
__device__ __forceinline__ void apply1d(double* __restrict__ param, int64_t e, float drive, float gain, double nlr) {
    param[e] = param[e] + nlr * (double)(drive * gain);
}

// The packed bins of 4 consecutive elements (e a multiple of 4), one vector
// load for all four (the bins array is 256-byte aligned).
struct Bins4 {
    uint64_t pk[4];
};
__device__ __forceinline__ Bins4 ld_bins4(const unsigned char* __restrict__ bins, int64_t e, int binbytes) {
    Bins4 r;
    switch (binbytes) {
        case 1: {
            const uint32_t v = *reinterpret_cast<const uint32_t*>(bins + e);
#pragma unroll
            for (int c = 0; c < 4; ++c) r.pk[c] = (v >> (8 * c)) & 0xffu;
            break;
        }
        case 2: {
            const uint2 v = *reinterpret_cast<const uint2*>(bins + 2 * e);
            r.pk[0] = v.x & 0xffffu; r.pk[1] = v.x >> 16; r.pk[2] = v.y & 0xffffu; r.pk[3] = v.y >> 16;
            break;
        }
        case 4: {
            const uint4 v = *reinterpret_cast<const uint4*>(bins + 4 * e);
            r.pk[0] = v.x; r.pk[1] = v.y; r.pk[2] = v.z; r.pk[3] = v.w;
            break;
        }
        default: {
            const uint4 a = *reinterpret_cast<const uint4*>(bins + 8 * e);
            const uint4 b = *reinterpret_cast<const uint4*>(bins + 8 * e + 16);
            r.pk[0] = ((uint64_t)a.y << 32) | a.x; r.pk[1] = ((uint64_t)a.w << 32) | a.z;
            r.pk[2] = ((uint64_t)b.y << 32) | b.x; r.pk[3] = ((uint64_t)b.w << 32) | b.z;
            break;
        }
    }
    return r;
}

template <typename PT, bool HASH, bool V4>
__global__ __launch_bounds__(SP_NT) void sweep5_kernel(
    Geom g, PT* __restrict__ param, const float* __restrict__ dbuf, const unsigned char* __restrict__ bins,
    const Ctrl* __restrict__ ctrl, const float* __restrict__ imp_tab, const double* __restrict__ part,
    float* __restrict__ de_state, int step, int hash_on, int hard, int c5_closed, Lanes L, cresso_hyper h) {
    if (L.dv) {
        const cresso_spectral_desc& d = lane_desc(L);
        param = (PT*)d.param; de_state = (float*)d.drive_energy; step = d.step;
    }
    dbuf = lane_at(dbuf, L); ctrl = lane_at(ctrl, L); imp_tab = lane_at(imp_tab, L); part = lane_at(part, L);
    extern __shared__ __align__(16) unsigned char dyn[];
    const int64_t beg = (int64_t)blockIdx.x * g.chunk1;
    const int64_t end = beg + g.chunk1 < g.n ? beg + g.chunk1 : g.n;
    // chunks are multiples of 4 elements: float4 drive loads (param 4-element aligned)
    const int64_t vend = V4 ? beg + ((end - beg) & ~(int64_t)3) : beg;
    const int64_t st = 4 * (int64_t)SP_NT;
    int64_t e = beg + 4 * (int64_t)threadIdx.x;
    const int T = g.T, B = g.B, bpb = g.bpb, binbytes = g.binbytes;
    // the first two float4 of drive and param (and their bins) go out before
    // the gain is known (their loads stay in flight through the finish's reduction)
    const bool pre = e + st < vend;
    float4 d0 = make_float4(0.f, 0.f, 0.f, 0.f), d1 = d0;
    float p0[4] = {0.f, 0.f, 0.f, 0.f}, p1[4] = {0.f, 0.f, 0.f, 0.f};
    Bins4 b0{}, b1{};
    if (pre) {
        d0 = *reinterpret_cast<const float4*>(dbuf + e);
        d1 = *reinterpret_cast<const float4*>(dbuf + e + st);
        pre4<PT>(param, e, p0);
        pre4<PT>(param, e + st, p1);
        if (HASH) {
            b0 = ld_bins4(bins, e, binbytes);
            b1 = ld_bins4(bins, e + st, binbytes);
        }
    }
    // the impulse table's loads go out with the finish's (first 4 values a thread)
    const int TB = T * B;
    float* s_imp = reinterpret_cast<float*>(dyn);
    Staged<4> simp;
    if (HASH) simp.load(imp_tab, TB);
    float gain, c5;
    fin4_values(g, part, ctrl, de_state, step, hash_on, hard, c5_closed, h, gain, c5);
    if (HASH) {
        simp.store(s_imp, TB);
        stage_rest<4>(s_imp, imp_tab, TB, [](float x) { return x; });
        __syncthreads();
    }
    const float kh = c5 * (1.0f / (float)T);
    const float nlr = (float)update_alpha<PT>(-h.lr);
    auto drive_pk = [&](uint64_t pk, float d) -> float {
        if (!HASH) return d;
        float hp = 0.f;
#pragma unroll
        for (int tt = 0; tt < SP_MAXT; ++tt) {
            if (tt >= T) break;
            hp += s_imp[tt * B + bin_of(pk, tt, bpb)];
        }
        return d + kh * hp;
    };
    auto drive_at = [&](int64_t e, float d) -> float { return HASH ? drive_pk(load_bins(bins, e, binbytes), d) : d; };
    auto apply4 = [&](int64_t e, const float4& d4, const float* pv, const Bins4& bk) {
        const float dv[4] = {d4.x, d4.y, d4.z, d4.w};
        if constexpr (std::is_same<PT, double>::value) {
            const double nlrd = -h.lr;
            double2* q = reinterpret_cast<double2*>(param + e);
            double2 a = q[0], b = q[1];
            a.x += nlrd * (double)(drive_pk(bk.pk[0], dv[0]) * gain);
            a.y += nlrd * (double)(drive_pk(bk.pk[1], dv[1]) * gain);
            b.x += nlrd * (double)(drive_pk(bk.pk[2], dv[2]) * gain);
            b.y += nlrd * (double)(drive_pk(bk.pk[3], dv[3]) * gain);
            q[0] = a;
            q[1] = b;
        } else {
            float o[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const float u = to_f(from_w<PT>(drive_pk(bk.pk[c], dv[c]) * gain));
                o[c] = pv[c] + nlr * u;
            }
            St4<PT>::go(param, e, o);
        }
    };
    // two float4 of drive and param (and their bins) per thread in flight per iteration, then the rest
    if (pre) {
        apply4(e, d0, p0, b0);
        apply4(e + st, d1, p1, b1);
        e += 2 * st;
    }
    for (; e + st < vend; e += 2 * st) {
        const float4 da = *reinterpret_cast<const float4*>(dbuf + e);
        const float4 db = *reinterpret_cast<const float4*>(dbuf + e + st);
        float pa[4], pb[4];
        pre4<PT>(param, e, pa);
        pre4<PT>(param, e + st, pb);
        Bins4 ba{}, bb{};
        if (HASH) {
            ba = ld_bins4(bins, e, binbytes);
            bb = ld_bins4(bins, e + st, binbytes);
        }
        apply4(e, da, pa, ba);
        apply4(e + st, db, pb, bb);
    }
    for (; e < vend; e += st) {
        const float4 d4 = *reinterpret_cast<const float4*>(dbuf + e);
        float pv[4];
        pre4<PT>(param, e, pv);
        Bins4 bk{};
        if (HASH) bk = ld_bins4(bins, e, binbytes);
        apply4(e, d4, pv, bk);
    }
    for (int64_t e = vend + threadIdx.x; e < end; e += SP_NT) {
        if constexpr (std::is_same<PT, double>::value)
            apply1d(param, e, drive_at(e, dbuf[e]), gain, -h.lr);
        else
            apply1(param, e, drive_at(e, dbuf[e]), gain, nlr);
    }
}



template <typename PT, bool VEC>
__global__ __launch_bounds__(SP_NT) void sweep5q_kernel(Geom g, PT* __restrict__ param, const float* __restrict__ dbuf,
                                                        const Ctrl* __restrict__ ctrl, const double* __restrict__ part,
                                                        float* __restrict__ de_state, int step, int hash_on, int hard,
                                                        int c5_closed, Lanes L, cresso_hyper h) {
    if (L.dv) {
        const cresso_spectral_desc& d = lane_desc(L);
        param = (PT*)d.param; de_state = (float*)d.drive_energy; step = d.step;
    }
    dbuf = lane_at(dbuf, L); ctrl = lane_at(ctrl, L); part = lane_at(part, L);
    if constexpr (!VEC) {
        // params not aligned for vector access: one column of four rows per
        // item, element loads and stores (coalesced across the wave)
        const int64_t nq = g.n / 4;
        const int64_t per = (nq + gridDim.x - 1) / gridDim.x;
        const int64_t w0 = (int64_t)blockIdx.x * per, w1 = w0 + per < nq ? w0 + per : nq;
        const int32_t cols = (int32_t)g.cols;
        int64_t w = w0 + threadIdx.x;
        int64_t q = w / cols;
        int32_t c = (int32_t)(w - q * cols);
        float gain, c5;
        fin4_values(g, part, ctrl, de_state, step, hash_on, hard, c5_closed, h, gain, c5);
        const float nlr = (float)update_alpha<PT>(-h.lr);
        while (w < w1) {
            const f32x4 d4 = gload4(dbuf + 4 * w);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t e = (4 * q + r) * g.cols + c;
                const float u = to_f(from_w<PT>(d4[r] * gain));
                param[e] = from_w<PT>(to_f(param[e]) + nlr * u);
            }
            w += SP_NT;
            c += SP_NT;
            while (c >= cols) {
                c -= cols;
                ++q;
            }
        }
        return;
    }
    // item w = q (cols / 4) + k: rows 4q .. 4q + 3, columns 4k .. 4k + 3: four
    // float4 of drive (one per column, 64 contiguous bytes) and four of param
    // (one per row); the items of a block are a contiguous range
    const int32_t c4 = (int32_t)(g.cols / 4);   // a multiple of SP_NT / 4 on this path
    const int64_t ni = g.n / 16;
    const int64_t per = (ni + gridDim.x - 1) / gridDim.x;
    const int64_t w0 = (int64_t)blockIdx.x * per, w1 = w0 + per < ni ? w0 + per : ni;
    int64_t w = w0 + threadIdx.x;
    int64_t q = w / c4;
    int32_t k = (int32_t)(w - q * c4);
    auto next = [&]() {
        w += SP_NT;
        k += SP_NT;
        while (k >= c4) {
            k -= c4;
            ++q;
        }
    };
    f32x4 dd[4];
    float pp[4][4];
    auto load = [&]() {
        const float* dq = dbuf + 4 * (q * g.cols + 4 * (int64_t)k);
#pragma unroll
        for (int j = 0; j < 4; ++j) dd[j] = gload4(dq + 4 * j);
#pragma unroll
        for (int r = 0; r < 4; ++r) pre4<PT>(param, (4 * q + r) * g.cols + 4 * (int64_t)k, pp[r]);
    };
    // the first item's loads go out before the gain is known
    const bool pre = w < w1;
    if (pre) load();
    float gain, c5;
    fin4_values(g, part, ctrl, de_state, step, hash_on, hard, c5_closed, h, gain, c5);
    const float nlr = (float)update_alpha<PT>(-h.lr);
    while (w < w1) {
        if (w != w0 + threadIdx.x) load();
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float o[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float u = to_f(from_w<PT>(dd[j][r] * gain));
                o[j] = pp[r][j] + nlr * u;
            }
            St4<PT>::go(param, (4 * q + r) * g.cols + 4 * (int64_t)k, o);
        }
        next();
    }
}

}  // namespace
}  // namespace cresso

struct cresso_spectral_plan {
    cresso::Geom g;
    cresso::Offs o;
    std::vector<cresso::AxisConst> axc;
    std::vector<cresso::ModeMeta> meta;
    std::vector<cresso::CarrierSrc> csrc;
    std::vector<int64_t> freqs;
    int64_t shape[8];
    int32_t rmax;
    int32_t bins_off;   // hash_bins == 0: no bin tables (bins/counts hold a dummy single bin)
    uint64_t serial;    // unique per created plan (never reused): names the tables a workspace holds
    int32_t work;       // CRESSO_F32: the fp32 work dtype (fp32/bf16/fp16 params); CRESSO_F64: fp64 params
    cresso::Offs64 o64; // work == CRESSO_F64: the fp64 regions
    std::vector<cresso::AxisConst64> axc64;
};

namespace cresso {
namespace {

template <typename T> T* at(void* ws, size_t off) { return reinterpret_cast<T*>(reinterpret_cast<char*>(ws) + off); }

size_t lds_sweep2(const Geom& g, int rw) {
    return sizeof(unsigned long long) * SP_NHIST * g.T * g.B + sizeof(float) * (16 + (size_t)rw) * g.PR;
}
size_t lds_sweep3(const Geom& g, int kp, int rw) {
    return lds_al_off(g) + sizeof(float) * (2 * (size_t)kp + rw) * g.PR;
}
// Compute units of the current device (queried once per device).
inline int resident_cus() {
    static int cache[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cache[dev] == 0) {
        int cus = 0;
        cache[dev] = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0 ? cus : 256;
    }
    return cache[dev];
}

template <int KC> size_t lds_sweep3m(const Geom& g, int rw) {
    return lds_sweep3(g, kcp<KC>(), rw) + sizeof(float) * ((bq_in_regs<KC>() ? 0 : (size_t)kcp<KC>() * SP_BQS) + SP_NT);
}
size_t lds_sweep4(const Geom& g, int kp, int rw) {
    return ((sizeof(float) * (size_t)g.T * g.B + 15) & ~(size_t)15) + sizeof(float) * (2 * (size_t)kp + rw) * g.PR;
}
constexpr size_t SP_LDS_MAX = 64 * 1024;
constexpr size_t SP_LDS_MAX_M = 96 * 1024;   // dynamic LDS of a matrix-core sweep (gfx950: 160 KB per workgroup)

// One step of `count` tensors of plan P: hd[0..count) are their descriptors
// on the host; for count > 1, dv is the same array in device memory and each
// tensor's per-step scratch follows the previous one's at a stride of ls
// bytes (a single tensor passes dv = nullptr, ls = 0).  Each tensor's results
// are bit-identical to a single-tensor step of it.
template <int RM, int KC, typename PT, typename GT>
int32_t run_step(const cresso_spectral_plan& P, const cresso_spectral_desc* hd, int count,
                 const cresso_spectral_desc* dv, size_t ls, void* ws, const cresso_hyper& h, hipStream_t s) {
    const Geom& g = P.g;
    const Offs& o = P.o;
    const cresso_spectral_desc& d = hd[0];
    const SpecState st = spec_state(d);
    const Lanes L{dv, ls};
    const unsigned ny = (unsigned)count;
    const int hash_on = d.hash_energy != nullptr && g.B > 0 && P.g.T > 0 ? 1 : 0;
    const int hard = d.hard ? 1 : 0;
    const int echo_on = (hard && h.echo_mix != 0.0) ? 1 : 0;
    const GT* grad = (const GT*)d.grad;
    PT* param = (PT*)d.param;
    const float* rowtab = at<float>(ws, o.rowtab);
    const float* coltab = at<float>(ws, o.coltab);
    const ModeMeta* meta = at<ModeMeta>(ws, o.meta);
    const unsigned char* bins = at<unsigned char>(ws, o.bins);
    const unsigned long long* counts = at<unsigned long long>(ws, o.counts);
    double* part = at<double>(ws, o.part);
    double* sums = at<double>(ws, o.sums);
    unsigned long long* hist = at<unsigned long long>(ws, o.hist);
    unsigned long long* hhi = hist + (size_t)g.hcopies * g.T * g.B;   // the density histogram's high words
    unsigned long long* hpart = at<unsigned long long>(ws, o.hpart);
    const unsigned long long* cooc = at<unsigned long long>(ws, o.cooc);
    float* lt = at<float>(ws, o.lt);
    float* imp = at<float>(ws, o.imp);
    unsigned long long* rowfx = at<unsigned long long>(ws, o.rowfx);
    unsigned long long* colfx = at<unsigned long long>(ws, o.colfx);
    float* colfac = at<float>(ws, o.colfac);
    float* terms = at<float>(ws, o.terms);
    float* tbuf = at<float>(ws, o.tbuf);
    Ctrl* ctrl = at<Ctrl>(ws, o.ctrl);
    const double* stats = at<double>(ws, o.stats);
    const double* bounds = at<double>(ws, o.bounds);
    const double* gram = at<double>(ws, o.gram);
    double* part1 = at<double>(ws, o.part1);
    const int step = d.step;
    const int axes_on = (hard && h.instant_metric_coupling != 0.0 && !g.one_d) ? 1 : 0;
    const size_t l2 = lds_sweep2(g, 2 * RM), l3 = lds_sweep3(g, kcp<KC>(), 2 * RM), l4 = lds_sweep4(g, kcp<KC>(), 2 * RM);
    if (l2 > SP_LDS_MAX || l3 > SP_LDS_MAX || l4 > SP_LDS_MAX)
        return fail(CRESSO_E_UNSUPPORTED, "spectral route: hash_tables x hash_bins = %d needs %zu bytes of LDS per block",
                    g.T * g.B, std::max(l2, std::max(l3, l4)));
    const dim3 grid(g.nblk, ny), grid1(g.nblk1, ny), fin(1, ny), blk(SP_NT);
    // float4 loads and stores when every tensor's grad and param allow them
    bool v4 = true, pv4 = true;
    for (int i = 0; i < count; ++i) {
        pv4 = pv4 && ((uintptr_t)hd[i].param % (4 * sizeof(PT))) == 0;
        v4 = v4 && ((uintptr_t)hd[i].grad % (4 * sizeof(GT))) == 0;
    }
    v4 = v4 && pv4;
    if (v4)
        hipLaunchKernelGGL((sweep1_kernel<PT, GT, true>), grid1, blk, 0, s, g, grad, param, part1, rowfx, colfx, ctrl,
                           st.force_rms, L, h);
    else
        hipLaunchKernelGGL((sweep1_kernel<PT, GT, false>), grid1, blk, 0, s, g, grad, param, part1, rowfx, colfx, ctrl,
                           st.force_rms, L, h);
    const bool fast = fast_mode(g, hash_on, axes_on, h);    // MODE 1 tiles of the general sweeps (two tables)
    // the matrix-core sweeps (two or four tables; ranks up to 16: two 16-row projection tiles)
    constexpr bool MX = RM <= 16;
    const bool mf = MX && mfast_mode(g, hash_on, axes_on, h);
    const bool t4 = g.T == 4;
    // the matrix-core sweeps write per-block histogram partials (hpart),
    // which part_reduce sums into hist; the general sweeps add into hist
    const bool m2 = mf;
    // the matrix-core sweeps' wave priorities pay only when every block is
    // resident at once (one round: the blocks of a CU then start together)
    const int64_t nb = (int64_t)g.nblk * count, cus = resident_cus();
    const int one_round2 = nb <= cus * occ2m<RM, KC>(), one_round3 = nb <= cus * occ3m<RM, KC>();
    const int one_round4 = nb <= cus * occ4m<RM, KC>();
    const bool m3 = mf && lds_sweep3m<KC>(g, 2 * RM) <= SP_LDS_MAX_M;
    // histogram merges: per-block partial rows summed by part_reduce, or, in
    // multi-round launches of plans with histogram copies, atomics of every
    // block straight into the copies (blocks end at different times; one-round
    // launches end together and would contend)
    const int hd2 = (m2 && !one_round2 && g.hcopies == SP_HCOPIES) ? 1 : 0;
    const int hd3 = (m3 && !one_round3 && g.hcopies == SP_HCOPIES) ? 1 : 0;
    // histogram copies the finishes read: all of them after atomic merges
    // (direct, or part_reduce's row groups), else copy 0 only
    const int prh = pr_hist_rows(g.T * g.B, g.nblk) > 0;
    const int nc2 = (hd2 || (m2 && prh)) ? g.hcopies : 1, nc3 = (hd3 || (m3 && prh)) ? g.hcopies : 1;
    if (m2) {
        if constexpr (MX) {
            if (t4)
                hipLaunchKernelGGL((sweep2m_kernel<RM, KC, GT, 4>), grid, blk, l2, s, g, grad, rowtab, coltab, meta, bins,
                                   ctrl, part, hd2 ? hist : hpart, hhi, rowfx, colfx, part1, st.force_rms, step, L, h,
                                   one_round2, hd2);
            else
                hipLaunchKernelGGL((sweep2m_kernel<RM, KC, GT, 2>), grid, blk, l2, s, g, grad, rowtab, coltab, meta, bins,
                                   ctrl, part, hd2 ? hist : hpart, hhi, rowfx, colfx, part1, st.force_rms, step, L, h,
                                   one_round2, hd2);
        }
    } else if (fast) {
        hipLaunchKernelGGL((sweep2_kernel<RM, KC, PT, GT, 1>), grid, blk, l2, s, g, grad, param, rowtab, coltab, meta, bins,
                           ctrl, part, hist, rowfx, colfx, hash_on, axes_on, part1, st.force_rms, step, L, h);
    } else {
        hipLaunchKernelGGL((sweep2_kernel<RM, KC, PT, GT, 0>), grid, blk, l2, s, g, grad, param, rowtab, coltab, meta, bins,
                           ctrl, part, hist, rowfx, colfx, hash_on, axes_on, part1, st.force_rms, step, L, h);
    }
    hipLaunchKernelGGL(part_reduce_kernel, dim3(NV2 + (m2 && !hd2 ? pr_hist_blocks(g.T * g.B, g.nblk) : 0), ny), dim3(256), 0, s,
                       part, g.nblk, NV2, sums, hpart, hist, g.T * g.B, L);
    hipLaunchKernelGGL(fin2_kernel, fin, dim3(SP_FN_NT), 0, s, g, meta, stats, bounds, sums, hist, counts, lt, st, ctrl,
                       step, hash_on, hard, nc2, L, h);
    if (axes_on && g.ntrail > 1) {
        int64_t nterms = 0;
        for (int a = 0; a < g.ntrail; ++a) nterms += g.tdim[a];
        hipLaunchKernelGGL(marg_terms_kernel, dim3((unsigned)nterms, ny), dim3(SP_MARG_NT), 0, s, g, colfx, terms, ctrl,
                           (float)h.eps, L);
        hipLaunchKernelGGL(marg_fac_kernel, dim3((unsigned)((g.cols + SP_MARG_NT - 1) / SP_MARG_NT), ny), dim3(SP_MARG_NT),
                           0, s, g, terms, colfac, L);
    }
    if (m3) {
        if constexpr (MX) {
            const size_t l3m = lds_sweep3m<KC>(g, 2 * RM);
            if (t4)
                hipLaunchKernelGGL((sweep3m_kernel<RM, KC, GT, 4>), grid, blk, l3m, s, g, grad, rowtab, coltab, meta, bins,
                                   ctrl, lt, rowfx, colfx, colfac, tbuf, part, hd3 ? hist : hpart, L, h, one_round3, hd3);
            else
                hipLaunchKernelGGL((sweep3m_kernel<RM, KC, GT, 2>), grid, blk, l3m, s, g, grad, rowtab, coltab, meta, bins,
                                   ctrl, lt, rowfx, colfx, colfac, tbuf, part, hd3 ? hist : hpart, L, h, one_round3, hd3);
        }
    } else if (fast) {
        hipLaunchKernelGGL((sweep3_kernel<RM, KC, PT, GT, 1>), grid, blk, l3, s, g, grad, param, rowtab, coltab, meta, bins,
                           ctrl, lt, rowfx, colfx, colfac, tbuf, part, hist, hash_on, L, h);
    } else {
        hipLaunchKernelGGL((sweep3_kernel<RM, KC, PT, GT, 0>), grid, blk, l3, s, g, grad, param, rowtab, coltab, meta, bins,
                           ctrl, lt, rowfx, colfx, colfac, tbuf, part, hist, hash_on, L, h);
    }
    // the matrix-core sweep 4 writes the full drive: the hash term's RMS comes
    // from the co-occurrence counts (two tables: in fin3, c5c = 1; four: in
    // hh4_kernel's blocks and sweep 4m, c5c = 2), and sweep 5 needs no bins
    const int c5c = (mf && cooc_closed(g)) ? (g.T == 2 ? 1 : 2) : 0;
    hipLaunchKernelGGL(part_reduce_kernel, dim3(NV3 + (m3 && !hd3 ? pr_hist_blocks(g.T * g.B, g.nblk) : 0), ny), dim3(256), 0, s,
                       part, g.nblk, NV3, sums, hpart, hist, g.T * g.B, L);
    hipLaunchKernelGGL(fin3_kernel, fin, dim3(SP_FN_NT), 0, s, g, meta, stats, gram, sums, hist, counts, imp, st, ctrl,
                       cooc, step, hash_on, hard, echo_on, c5c, nc3, L, h);
    if (c5c == 2)
        hipLaunchKernelGGL(hh4_kernel, dim3((unsigned)hh4_blocks(g), ny), dim3(256), 0, s, g, cooc, counts, imp, ctrl, L);
    // the field is 4-row interleaved when sweep 3m wrote it (then sweep 4m
    // runs too, in place, and sweep 5q applies it)
    const bool q4 = m3 && c5c != 0;
    if (!MX || c5c == 0) {
        if (fast)
            hipLaunchKernelGGL((sweep4_kernel<RM, KC, 1>), grid, blk, l4, s, g, rowtab, coltab, meta, bins, ctrl, imp, tbuf,
                               part, hash_on, echo_on, L, h);
        else
            hipLaunchKernelGGL((sweep4_kernel<RM, KC, 0>), grid, blk, l4, s, g, rowtab, coltab, meta, bins, ctrl, imp, tbuf,
                               part, hash_on, echo_on, L, h);
    } else if constexpr (MX) {
        if (c5c == 1 && q4)
            hipLaunchKernelGGL((sweep4m_kernel<RM, KC, 2, true>), grid, blk, l4, s, g, rowtab, coltab, meta, bins, ctrl,
                               imp, tbuf, part, echo_on, L, h, one_round4);
        else if (c5c == 1)
            hipLaunchKernelGGL((sweep4m_kernel<RM, KC, 2, false>), grid, blk, l4, s, g, rowtab, coltab, meta, bins, ctrl,
                               imp, tbuf, part, echo_on, L, h, one_round4);
        else if (q4)
            hipLaunchKernelGGL((sweep4m_kernel<RM, KC, 4, true>), grid, blk, l4, s, g, rowtab, coltab, meta, bins, ctrl,
                               imp, tbuf, part, echo_on, L, h, one_round4);
        else
            hipLaunchKernelGGL((sweep4m_kernel<RM, KC, 4, false>), grid, blk, l4, s, g, rowtab, coltab, meta, bins, ctrl,
                               imp, tbuf, part, echo_on, L, h, one_round4);
    }
    const bool hash5 = hash_on && !c5c;   // sweep 5 adds the hash term itself
    const size_t l5 = hash5 ? sizeof(float) * (size_t)g.T * g.B : 0;
    if (q4 && pv4)
        hipLaunchKernelGGL((sweep5q_kernel<PT, true>), grid1, blk, 0, s, g, param, tbuf, ctrl, part, st.drive_energy, step,
                           hash_on, hard, c5c, L, h);
    else if (q4)
        hipLaunchKernelGGL((sweep5q_kernel<PT, false>), grid1, blk, 0, s, g, param, tbuf, ctrl, part, st.drive_energy,
                           step, hash_on, hard, c5c, L, h);
    else if (hash5 && pv4)
        hipLaunchKernelGGL((sweep5_kernel<PT, true, true>), grid1, blk, l5, s, g, param, tbuf, bins, ctrl, imp, part,
                           st.drive_energy, step, hash_on, hard, c5c, L, h);
    else if (hash5)
        hipLaunchKernelGGL((sweep5_kernel<PT, true, false>), grid1, blk, l5, s, g, param, tbuf, bins, ctrl, imp, part,
                           st.drive_energy, step, hash_on, hard, c5c, L, h);
    else if (pv4)
        hipLaunchKernelGGL((sweep5_kernel<PT, false, true>), grid1, blk, 0, s, g, param, tbuf, bins, ctrl, imp, part,
                           st.drive_energy, step, hash_on, hard, c5c, L, h);
    else
        hipLaunchKernelGGL((sweep5_kernel<PT, false, false>), grid1, blk, 0, s, g, param, tbuf, bins, ctrl, imp, part,
                           st.drive_energy, step, hash_on, hard, c5c, L, h);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? CRESSO_OK : hip_fail(e, "spectral route: launch");
}

// Variant dispatch shared by the instantiation units.
template <typename PT, typename GT>
int32_t spectral_run(const cresso_spectral_plan& P, const cresso_spectral_desc* hd, int count,
                     const cresso_spectral_desc* dv, size_t ls, void* ws, const cresso_hyper& h, hipStream_t s) {
    const int R = P.g.R, K = P.g.K;
    const int var = (R <= 4 && K <= 9) ? 0 : (R <= 8 && K <= 11) ? 1 : (R <= 8) ? 2 : (R <= 16) ? 3 : 4;
    switch (var) {
        case 0: return run_step<4, 9, PT, GT>(P, hd, count, dv, ls, ws, h, s);
        case 1: return run_step<8, 11, PT, GT>(P, hd, count, dv, ls, ws, h, s);
        case 2: return run_step<8, 17, PT, GT>(P, hd, count, dv, ls, ws, h, s);
        case 3: return run_step<16, 33, PT, GT>(P, hd, count, dv, ls, ws, h, s);
        default: return run_step<32, 65, PT, GT>(P, hd, count, dv, ls, ws, h, s);   // general sweeps only
    }
}

}  // namespace

// One spectral step per (param dtype, grad dtype) pair, each instantiated in
// its own translation unit (spectral_step_<pt>_<gt>.hip) so they compile in
// parallel.  The carrier-count variant (rank and distinct column carriers
// fixed at compile time) is chosen inside.
// fp64 work dtype (spectral_f64.hip): the plan's fp64 regions after `off`
// (-> the new end), their set-up, and one step of an fp64 tensor
size_t plan_f64_layout(cresso_spectral_plan& P, size_t off);
int32_t workspace_init_f64(const cresso_spectral_plan& P, void* ws, hipStream_t s);
int32_t spectral_run_f64(const cresso_spectral_plan& P, const cresso_spectral_desc& d, void* ws, const cresso_hyper& h,
                         hipStream_t s);

typedef int32_t (*SpectralRunFn)(const cresso_spectral_plan&, const cresso_spectral_desc*, int,
                                 const cresso_spectral_desc*, size_t, void*, const cresso_hyper&, hipStream_t);
#define CRESSO_SP_DECL(NAME)                                                                                      \
    int32_t NAME(const cresso_spectral_plan&, const cresso_spectral_desc*, int, const cresso_spectral_desc*, size_t, \
                 void*, const cresso_hyper&, hipStream_t);
CRESSO_SP_DECL(spectral_run_f32_f32)
CRESSO_SP_DECL(spectral_run_bf16_bf16)
CRESSO_SP_DECL(spectral_run_f16_f16)
CRESSO_SP_DECL(spectral_run_f32_bf16)
CRESSO_SP_DECL(spectral_run_f32_f16)
#undef CRESSO_SP_DECL

}  // namespace cresso
