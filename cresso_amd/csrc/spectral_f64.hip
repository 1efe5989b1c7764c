// Spectral / coordinate-hash route of CRESSO5 for fp64 params, in the fp64
// work dtype of the reference (cresso_v5.py:119-124, the step at 945-1353):
// every carrier, field, sum and state update is fp64.
//
// Layout and passes (one tensor per call; fp64 params are rare, so the design
// favours exactness and simplicity over the fp32 route's fused sweeps):
//  * per-axis carrier tables AxisTab[mode][axis offset + coordinate] =
//    (cos, sin, window) of the axis' phase part, the fp64 counterpart of the
//    reference's per-axis basis cache (basis_axis_cache_cuda,
//    cresso_cuda_kernel.cu:406-451).  A carrier at an element is the product of
//    its axes' factors: additive kinds as a complex product (cos and sin of
//    the summed phase), product kinds as plain products, kind 3 times the
//    product of the windows (cresso_v5.py:295-348);
//  * normalization stats by two dense passes over the carriers at workspace
//    set-up (mean, then the centred second moment; cresso_v5.py:138-142);
//  * per step: A (sum f^2, max |f|), B (log-density sums and projection,
//    density histograms), axis marginals (one wave per coordinate), C (the
//    tangent field t, stored; prediction error, port histograms and
//    projections), D (drive moments), E (drive, stored over t, sum drive^2),
//    F (update).  Single-block finish kernels between them update the state.
// Reductions are fixed-order fp64 trees (block partials merged in block
// order), so results are bit-identical run to run.  Hash-bin sums use a
// two-word fixed point: each value scaled by 2^F is split into a high word
// (signed, multiples of 2^k) and a low word (unsigned, below 2^k + 1), each
// summed with 64-bit integer atomics; k leaves every bin's low-word sum below
// 2^63 and F keeps the high-word sums below 2^62, which leaves about 2^-70 of
// absolute resolution at typical densities: the bin sums are exact to fp64
// rounding in any arrival order.
#include "spectral_kernels.hpp"

#pragma clang fp contract(off)

namespace cresso {
namespace {

constexpr int D_NT = 256;
constexpr int D_NW = D_NT / 64;
constexpr int D_LDS_TB = 1536;                 // tables x bins kept per block in LDS (two words: 24 KiB)
constexpr int D_NV = 6 * SP_MAXR;              // block partials per block (the stats pass needs 6 R)

struct AxisTab {
    double c, s, w, pad;
};

// shape of the tensor and the table offsets (kernel argument)
struct DGeo {
    int64_t n, sumd;
    int64_t dim[8], aoff[8], inner[8];
    int32_t nd, R, T, B, bpb, binbytes, nblk, pad;
    double shrink;
};

DGeo dgeo(const cresso_spectral_plan& P) {
    DGeo d;
    std::memset(&d, 0, sizeof(d));
    const Geom& g = P.g;
    d.n = g.n;
    d.nd = g.ndim;
    int64_t off = 0;
    for (int a = 0; a < g.ndim; ++a) {
        d.dim[a] = P.shape[a];
        d.aoff[a] = off;
        off += P.shape[a];
    }
    int64_t in = 1;
    for (int a = g.ndim - 1; a >= 0; --a) {
        d.inner[a] = in;
        in *= P.shape[a];
    }
    d.sumd = off;
    d.R = g.R;
    d.T = g.T;
    d.B = g.B;
    d.bpb = g.bpb;
    d.binbytes = g.binbytes;
    d.nblk = P.o64.nblk;
    d.shrink = g.shrink;
    return d;
}

// per-step control block
struct Ctrl64 {
    double s;                  // force scale max(force_rms, eps)
    double fds, fP;            // 2^F of the density and port histograms
    double lo_unit;            // 2^k of the histograms' low words (as a double)
    double kappa;              // instant metric: coupling / (ndim p')
    double gden;               // 1-D instant metric: max(mean density, eps)
    double rc[4][SP_MAXR][2];  // coefficients on the normalized carriers: 0 metric, 1 pred, 2 pred', 3 echo
    // drive: (1-mix) core + mix pred' + nov_mix nov + k_res err' + k_echo echo + k_hash hash_pred, with
    // core = c_rat rat + c_bnd bnd + c_root root_raw + c_t t
    double mix, c_rat, c_bnd, c_root, c_t, nov_mix, nov_div, k_res, k_echo, k_hash;
    double gain;
    int32_t k_lo, inst, ls_on, pad;
};

struct DState {
    double *force_rms, *drive_energy, *surprise, *action;
    const double* omega;
    double *q_cos, *q_sin, *p_cos, *p_sin, *metric_cos, *metric_sin, *metric_p_cos, *metric_p_sin;
    double *calcium_cos, *calcium_sin, *conf;
    double *hash_energy, *hash_impulse, *hash_refractory;
};

DState dstate(const cresso_spectral_desc& d) {
    DState st;
    st.force_rms = (double*)d.force_rms; st.drive_energy = (double*)d.drive_energy;
    st.surprise = (double*)d.surprise; st.action = (double*)d.action; st.omega = (const double*)d.omega;
    st.q_cos = (double*)d.q_cos; st.q_sin = (double*)d.q_sin; st.p_cos = (double*)d.p_cos; st.p_sin = (double*)d.p_sin;
    st.metric_cos = (double*)d.metric_cos; st.metric_sin = (double*)d.metric_sin;
    st.metric_p_cos = (double*)d.metric_p_cos; st.metric_p_sin = (double*)d.metric_p_sin;
    st.calcium_cos = (double*)d.calcium_cos; st.calcium_sin = (double*)d.calcium_sin;
    st.conf = (double*)d.mode_confidence;
    st.hash_energy = (double*)d.hash_energy; st.hash_impulse = (double*)d.hash_impulse;
    st.hash_refractory = (double*)d.hash_refractory;
    return st;
}

// ---------------------------------------------------------------------------
// element helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ void coords_of(const DGeo& g, int64_t i, int64_t (&c)[8]) {
    for (int a = g.nd - 1; a >= 0; --a) {
        const int64_t q = i / g.dim[a];
        c[a] = i - q * g.dim[a];
        i = q;
    }
}

// normalized carriers (Cn_r, Sn_r) of every mode at the element with coordinates c
template <int RM>
__device__ __forceinline__ void carriers(const DGeo& g, const ModeMeta* __restrict__ meta,
                                         const AxisTab* __restrict__ tab, const double* __restrict__ nst,
                                         const int64_t (&c)[8], double (&cn)[RM], double (&sn)[RM]) {
#pragma unroll
    for (int r = 0; r < RM; ++r) {
        cn[r] = 0.0;
        sn[r] = 0.0;
        if (r >= g.R) continue;
        const ModeMeta m = meta[r];
        double C = 1.0, S = 0.0;
        if (m.type == M_PROD) {
            S = 1.0;
            for (int a = 0; a < g.nd; ++a) {
                const AxisTab e = tab[(size_t)r * g.sumd + g.aoff[a] + c[a]];
                C = C * e.c;
                S = S * e.s;
            }
        } else if (m.type == M_ADD) {
            double W = 1.0;
            for (int a = 0; a < g.nd; ++a) {
                const AxisTab e = tab[(size_t)r * g.sumd + g.aoff[a] + c[a]];
                const double cc = C * e.c - S * e.s;
                const double ss = S * e.c + C * e.s;
                C = cc;
                S = ss;
                if (m.kind == 3) W = (a == 0) ? e.w : W * e.w;
            }
            if (m.kind == 3) {
                C = W * C;
                S = W * S;
            }
        }
        const double* q = nst + 8 * r;
        cn[r] = (C - q[0]) * q[1];
        sn[r] = (S - q[2]) * q[3];
    }
}

// shrink * sum_r g_r (cc_r Cn_r + sc_r Sn_r) in mode order (cresso_v5.py:362-376);
// the coefficients hold shrink * g * (cc, sc), zero for a skipped mode
template <int RM>
__device__ __forceinline__ double recon(const double (&rc)[SP_MAXR][2], const double (&cn)[RM], const double (&sn)[RM], int R) {
    double out = 0.0;
#pragma unroll
    for (int r = 0; r < RM; ++r) {
        if (r >= R) break;
        out = out + rc[r][0] * cn[r];
        out = out + rc[r][1] * sn[r];
    }
    return out;
}

__device__ __forceinline__ int bin_of(const DGeo& g, const unsigned char* __restrict__ bins, int64_t i, int t) {
    uint64_t packed;
    switch (g.binbytes) {
        case 1: packed = bins[i]; break;
        case 2: packed = reinterpret_cast<const uint16_t*>(bins)[i]; break;
        case 4: packed = reinterpret_cast<const uint32_t*>(bins)[i]; break;
        default: packed = reinterpret_cast<const uint64_t*>(bins)[i]; break;
    }
    const int sh = 8 * g.bpb * t;
    return (int)((packed >> sh) & (g.bpb == 1 ? 0xFFull : 0xFFFFull));
}

// two-word fixed point of x * fs (fs = 2^F): high word (signed multiple of
// 2^k, as an integer count of 2^k) and low word (0 .. 2^k)
__device__ __forceinline__ void two_word(double x, double fs, double lo_unit, double inv_lo_unit,
                                         unsigned long long& hi, unsigned long long& lo) {
    const double y = x * fs;
    const double h = floor(y * inv_lo_unit);
    const double l = rint(y - h * lo_unit);
    hi = (unsigned long long)(long long)h;
    lo = (unsigned long long)l;
}
__device__ __forceinline__ double from_two_word(unsigned long long hi, unsigned long long lo, double fs, double lo_unit) {
    return ((double)(long long)hi * lo_unit + (double)lo) / fs;
}

// force f = sign * grad (+ weight_decay * param) (cresso_v5.py:835-836, 907-912)
__device__ __forceinline__ double force_at(const double* __restrict__ grad, const double* __restrict__ param, int64_t i,
                                           double sg, double wd) {
    double f = sg * grad[i];
    if (wd != 0.0) f = f + wd * param[i];
    return f;
}

__device__ __forceinline__ double rel_of(double f, double s, double eps) { return fmin(fabs(f) / s + eps, 1.0e4); }

__device__ __forceinline__ double sigmoid_d(double x) { return 1.0 / (1.0 + exp(-x)); }

// block partials: thread values summed in a fixed order, one row per block
template <int V>
__device__ __forceinline__ void put_partials(double (&v)[V], int nv, double* __restrict__ part) {
    __shared__ double red[D_NW * V];
    block_sum<V>(v, red);
    if (threadIdx.x == 0)
        for (int i = 0; i < nv; ++i) part[(size_t)blockIdx.x * D_NV + i] = v[i];
}

// sums[v] = sum over blocks of part[b][v] in block order (max for v >= max_from)
__global__ __launch_bounds__(D_NT) void d_reduce_kernel(const double* __restrict__ part, int nblk, int max_from,
                                                        double* __restrict__ sums) {
    __shared__ double red[D_NW];
    const int v = blockIdx.x;
    const bool mx = v >= max_from;
    double a = 0.0;
    for (int b = threadIdx.x; b < nblk; b += D_NT) {
        const double x = part[(size_t)b * D_NV + v];
        a = mx ? fmax(a, x) : a + x;
    }
    if (mx) {
        for (int o = 32; o > 0; o >>= 1) a = fmax(a, __shfl_xor(a, o));
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = a;
        __syncthreads();
        if (threadIdx.x == 0) {
            double m = red[0];
            for (int w = 1; w < D_NW; ++w) m = fmax(m, red[w]);
            sums[v] = m;
        }
        return;
    }
    double t[1] = {a};
    block_sum<1>(t, red);
    if (threadIdx.x == 0) sums[v] = t[0];
}

__global__ void d_clear_kernel(unsigned long long* __restrict__ p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) p[i] = 0ull;
}

// ---------------------------------------------------------------------------
// workspace set-up: axis tables and normalization stats
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(D_NT) void d_tab_kernel(DGeo g, const AxisConst64* __restrict__ axc,
                                                     AxisTab* __restrict__ tab) {
    const int64_t total = (int64_t)g.R * g.sumd;
    for (int64_t e = (int64_t)blockIdx.x * D_NT + threadIdx.x; e < total; e += (int64_t)gridDim.x * D_NT) {
        const int r = (int)(e / g.sumd);
        const int64_t j = e - (int64_t)r * g.sumd;
        int a = 0;
        while (a + 1 < g.nd && j >= g.aoff[a + 1]) ++a;
        const int64_t k = j - g.aoff[a];
        const AxisConst64 x = axc[(size_t)r * g.nd + a];
        const double u = ((double)k + 0.5) / (double)g.dim[a];   // cresso_v5.py:237-239
        AxisTab t{1.0, 0.0, 1.0, 0.0};
        if (x.kind == 1) {   // product of cos / sin over the axes with f != 0
            if (x.f != 0) {
                const double ph = x.pf * u;
                t.c = cos(ph);
                t.s = sin(ph);
            } else {
                t.s = 1.0;
            }
        } else if (x.kind == 0) {   // additive phase over the axes with f != 0
            if (x.f != 0) {
                const double ph = x.pf * u;
                t.c = cos(ph);
                t.s = sin(ph);
            }
        } else {   // chirped phase on every axis (cresso_v5.py:272-292), window for kind 3
            const double d = u - 0.5;
            const double ph = x.pf * u + x.pcm * (d * d);
            t.c = cos(ph);
            t.s = sin(ph);
            if (x.kind == 3) {
                const double z = (u - x.mu) / x.sig;
                t.w = exp(-0.5 * (z * z));
            }
        }
        tab[e] = t;
    }
}

// pass 1 of the stats: sums of the raw carriers; pass 2: centred second
// moments, centred sums and the largest centred magnitude
template <int RM, int PASS>
__global__ __launch_bounds__(D_NT) void d_stats_kernel(DGeo g, const ModeMeta* __restrict__ meta,
                                                       const AxisTab* __restrict__ tab, const double* __restrict__ mu,
                                                       double* __restrict__ part) {
    // raw carriers: the normalization with (mean 0, scale 1)
    __shared__ double s_id[8 * SP_MAXR];
    for (int i = threadIdx.x; i < 8 * SP_MAXR; i += D_NT) {
        const int r = i / 8, c = i % 8;
        s_id[i] = (c == 1 || c == 3) ? 1.0 : ((PASS == 2 && (c == 0 || c == 2) && r < g.R) ? mu[2 * r + c / 2] : 0.0);
    }
    __syncthreads();
    double v[6 * RM];
#pragma unroll
    for (int i = 0; i < 6 * RM; ++i) v[i] = 0.0;
    for (int64_t i = (int64_t)blockIdx.x * D_NT + threadIdx.x; i < g.n; i += (int64_t)gridDim.x * D_NT) {
        int64_t c[8];
        coords_of(g, i, c);
        double cn[RM], sn[RM];
        carriers<RM>(g, meta, tab, s_id, c, cn, sn);
#pragma unroll
        for (int r = 0; r < RM; ++r) {
            if (PASS == 1) {
                v[2 * r] += cn[r];
                v[2 * r + 1] += sn[r];
            } else {
                v[2 * r] += cn[r] * cn[r];
                v[2 * r + 1] += sn[r] * sn[r];
                v[2 * RM + 2 * r] += cn[r];
                v[2 * RM + 2 * r + 1] += sn[r];
                v[4 * RM + 2 * r] = fmax(v[4 * RM + 2 * r], fabs(cn[r]));
                v[4 * RM + 2 * r + 1] = fmax(v[4 * RM + 2 * r + 1], fabs(sn[r]));
            }
        }
    }
    // maxima: wave and block maxima (order-free), sums: fixed-order block sums
    __shared__ double s_mx[D_NW * 2 * SP_MAXR];
    if (PASS == 2) {
#pragma unroll
        for (int q = 0; q < 2 * RM; ++q) {
            double m = v[4 * RM + q];
            for (int o = 32; o > 0; o >>= 1) m = fmax(m, __shfl_xor(m, o));
            if ((threadIdx.x & 63) == 0) s_mx[(threadIdx.x >> 6) * 2 * SP_MAXR + q] = m;
        }
    }
    constexpr int VS = PASS == 1 ? 2 * RM : 4 * RM;
    double w[VS];
#pragma unroll
    for (int q = 0; q < VS; ++q) w[q] = v[q];
    __shared__ double red[D_NW * VS];
    block_sum<VS>(w, red);
    if (threadIdx.x == 0) {
        double* row = part + (size_t)blockIdx.x * D_NV;
        for (int r = 0; r < g.R; ++r) {
            row[2 * r] = w[2 * r];
            row[2 * r + 1] = w[2 * r + 1];
            if (PASS == 2) {
                row[2 * SP_MAXR + 2 * r] = w[2 * RM + 2 * r];
                row[2 * SP_MAXR + 2 * r + 1] = w[2 * RM + 2 * r + 1];
                for (int c = 0; c < 2; ++c) {
                    double m = 0.0;
                    for (int ww = 0; ww < D_NW; ++ww) m = fmax(m, s_mx[ww * 2 * SP_MAXR + 2 * r + c]);
                    row[4 * SP_MAXR + 2 * r + c] = m;
                }
            }
        }
    }
}

// mu[2r], mu[2r+1] = means of the raw carriers
__global__ void d_stats_mid_kernel(DGeo g, const double* __restrict__ sums, double* __restrict__ mu) {
    for (int q = threadIdx.x; q < 2 * g.R; q += blockDim.x) mu[q] = sums[q] / (double)g.n;
}

// nst[8r..]: mean C, 1/max(rms C, 1e-6), mean S, 1/max(rms S, 1e-6), mean of
// the normalized C and S, max |normalized C|, max |normalized S|; the zero
// mode is unnormalized: C = 1, S = 0 (cresso_v5.py:138-142, 299-300)
__global__ void d_stats_fin_kernel(DGeo g, const ModeMeta* __restrict__ meta, const double* __restrict__ mu,
                                   const double* __restrict__ sums, double* __restrict__ nst) {
    const int r = threadIdx.x;
    if (r >= g.R) return;
    double* q = nst + 8 * r;
    if (meta[r].type == M_ZERO) {
        q[0] = 0.0; q[1] = 1.0; q[2] = 0.0; q[3] = 0.0;
        q[4] = 1.0; q[5] = 0.0; q[6] = 1.0; q[7] = 0.0;
        return;
    }
    const double n = (double)g.n;
    for (int c = 0; c < 2; ++c) {
        const double rms = sqrt(sums[2 * r + c] / n + 1e-12);
        const double inv = 1.0 / fmax(rms, 1e-6);
        q[2 * c] = mu[2 * r + c];
        q[2 * c + 1] = inv;
        q[4 + c] = sums[2 * SP_MAXR + 2 * r + c] / n * inv;
        q[6 + c] = sums[4 * SP_MAXR + 2 * r + c] * inv;
    }
}

// ---------------------------------------------------------------------------
// the step
// ---------------------------------------------------------------------------
struct DArgs {
    const double* grad;
    double* param;
    const unsigned char* bins;
    const unsigned long long* counts;
    const ModeMeta* meta;
    const AxisTab* tab;
    const double* nst;
    double* part;
    double* sums;
    unsigned long long* hist;   // [4][T][B]: density lo, density hi, port lo, port hi
    double* lt;                 // [T][B] log hash metric
    const double* imp;          // [T][B] hash impulse (state, after this step's update)
    double* marg;               // axis marginal sums, then their log terms (in terms)
    double* terms;
    Ctrl64* ctrl;
    double* tbuf;
    double sg, wd, eps;
    int hash_on, step;
};

// A: sum f^2 and max |f|
__global__ __launch_bounds__(D_NT) void d_sweepA_kernel(DGeo g, DArgs A) {
    double v[2] = {0.0, 0.0};
    double m = 0.0;
    for (int64_t i = (int64_t)blockIdx.x * D_NT + threadIdx.x; i < g.n; i += (int64_t)gridDim.x * D_NT) {
        const double f = force_at(A.grad, A.param, i, A.sg, A.wd);
        v[0] += f * f;
        m = fmax(m, fabs(f));
    }
    for (int o = 32; o > 0; o >>= 1) m = fmax(m, __shfl_xor(m, o));
    __shared__ double s_m[D_NW];
    if ((threadIdx.x & 63) == 0) s_m[threadIdx.x >> 6] = m;
    put_partials<2>(v, 1, A.part);
    if (threadIdx.x == 0) {
        for (int w = 1; w < D_NW; ++w) m = fmax(m, s_m[w]);
        A.part[(size_t)blockIdx.x * D_NV + 1] = fmax(m, s_m[0]);
    }
}

// ceil(log2(x)) for x >= 1 (an integer count)
__device__ __forceinline__ int ceil_log2(double x) { return (int)ceil(log2(fmax(x, 1.0))); }

// the force-RMS reservoir, the scale and the density histogram's fixed point
__global__ void d_finA_kernel(DGeo g, DArgs A, DState st, const Ctrl* __restrict__ c32, cresso_hyper h) {
    if (threadIdx.x != 0) return;
    Ctrl64* c = A.ctrl;
    const double n = (double)g.n, eps = h.eps;
    const double sum = A.sums[0], mx = A.sums[1];
    const double now = sqrt(sum / n + eps);
    const double fr = A.step <= 1 ? now : *st.force_rms * h.reservoir_decay + now * (1.0 - h.reservoir_decay);
    *st.force_rms = fr;
    const double s = fmax(fr, eps);
    c->s = s;
    const double cmax = c32->cmax;
    const int k = 63 - ceil_log2(cmax);
    c->k_lo = k;
    c->lo_unit = ldexp(1.0, k);
    // a bin's density sum is at most the smaller of cmax rmax^p and the whole
    // histogram's sum of rel^p (power means over sum rel^2 <= sum f^2/s^2 +
    // 2 eps sqrt(n sum f^2)/s + n eps^2); its high words stay below 2^62
    const double p = h.energy_power;
    const double rmax = fmin(mx / s + eps, 1.0e4);
    const double lr = log2(rmax);
    const double s2 = (sum / (s * s) + 2.0 * eps * sqrt(n * sum) / s + n * eps * eps) * (1.0 + 1e-9);
    const double l2s = log2(s2 + 1e-300);
    const double ltot = p >= 2.0 ? (p - 2.0) * lr + l2s : (1.0 - 0.5 * p) * log2(n) + 0.5 * p * l2s;
    const double lbin = p * lr + log2(cmax);
    const int F = (int)floor(62.0 + k - fmin(lbin, ltot) - 1e-6);
    c->fds = ldexp(1.0, F < 900 ? F : 900);
}

// B: log-density sum and projection, density histograms, 1-D density sum
template <int RM>
__global__ __launch_bounds__(D_NT) void d_sweepB_kernel(DGeo g, DArgs A, cresso_hyper h) {
    const Ctrl64* c = A.ctrl;
    const double s = c->s, eps = A.eps, p = h.energy_power, ip = fmax(h.instant_metric_power, 0.25);
    const bool lds = g.T * g.B <= D_LDS_TB;
    __shared__ unsigned long long s_h[2 * D_LDS_TB];
    const int TB = g.T * g.B;
    if (A.hash_on && lds) {
        for (int i = threadIdx.x; i < 2 * TB; i += D_NT) s_h[i] = 0ull;
        __syncthreads();
    }
    const double fs = c->fds, lu = c->lo_unit, ilu = 1.0 / lu;
    double v[2 + 2 * RM];
#pragma unroll
    for (int i = 0; i < 2 + 2 * RM; ++i) v[i] = 0.0;
    for (int64_t i = (int64_t)blockIdx.x * D_NT + threadIdx.x; i < g.n; i += (int64_t)gridDim.x * D_NT) {
        const double f = force_at(A.grad, A.param, i, A.sg, A.wd);
        const double rel = rel_of(f, s, eps);
        const double ds = pow(rel, p);
        const double d = log1p(ds);
        v[0] += d;
        if (g.nd == 1) v[1] += fmin(pow(fmax(rel, eps), ip), 1.0e6);
        int64_t cc[8];
        coords_of(g, i, cc);
        double cn[RM], sn[RM];
        carriers<RM>(g, A.meta, A.tab, A.nst, cc, cn, sn);
#pragma unroll
        for (int r = 0; r < RM; ++r) {
            v[2 + 2 * r] += d * cn[r];
            v[3 + 2 * r] += d * sn[r];
        }
        if (A.hash_on) {
            unsigned long long hi, lo;
            two_word(ds, fs, lu, ilu, hi, lo);
            for (int t = 0; t < g.T; ++t) {
                const int b = t * g.B + bin_of(g, A.bins, i, t);
                if (lds) {
                    atomicAdd(&s_h[b], lo);
                    if (hi) atomicAdd(&s_h[TB + b], hi);
                } else {
                    atomicAdd(&A.hist[b], lo);
                    if (hi) atomicAdd(&A.hist[TB + b], hi);
                }
            }
        }
    }
    if (A.hash_on && lds) {
        __syncthreads();
        for (int i = threadIdx.x; i < 2 * TB; i += D_NT)
            if (s_h[i]) atomicAdd(&A.hist[i], s_h[i]);
    }
    put_partials<2 + 2 * RM>(v, 2 + 2 * g.R, A.part);
}

// axis a's marginal density sums: one wave per coordinate, elements in a fixed order
__global__ __launch_bounds__(D_NT) void d_marg_kernel(DGeo g, DArgs A, cresso_hyper h, int a) {
    const int64_t k = (int64_t)blockIdx.x * D_NW + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (k >= g.dim[a]) return;
    const double s = A.ctrl->s, eps = A.eps, ip = fmax(h.instant_metric_power, 0.25);
    const int64_t inner = g.inner[a], cnt = g.n / g.dim[a];
    double acc = 0.0;
    for (int64_t j = lane; j < cnt; j += 64) {
        const int64_t outer = j / inner, in = j - outer * inner;
        const int64_t i = outer * g.dim[a] * inner + k * inner + in;
        const double f = force_at(A.grad, A.param, i, A.sg, A.wd);
        acc += fmin(pow(fmax(rel_of(f, s, eps), eps), ip), 1.0e6);
    }
    acc = wave_total_d(acc);   // the total lands in lane 63
    if (lane == 63) A.marg[g.aoff[a] + k] = acc;
}

// B's finish: metric oscillator, metric and prediction coefficients, hash
// metric tables, instant metric terms, the port histogram's fixed point
__global__ __launch_bounds__(D_NT) void d_finB_kernel(DGeo g, DArgs A, DState st, const Ctrl* __restrict__ c32,
                                                      cresso_hyper h, int hard) {
    __shared__ double red[D_NW];
    Ctrl64* c = A.ctrl;
    const double n = (double)g.n, eps = h.eps;
    const int R = g.R;
    if (threadIdx.x == 0) {
        // log-density projection (cresso_v5.py:1058-1062): mean((d/m - 1) Cn) = mean(d Cn)/m - mean(Cn)
        const double m = fmax(A.sums[0] / n, eps);
        const double damp = fmax(0.0, 1.0 - h.metric_dt * h.metric_friction);
        for (int r = 0; r < R; ++r) {
            const double* q = A.nst + 8 * r;
            const double port[2] = {(A.sums[2 + 2 * r] / n) / m - q[4], (A.sums[3 + 2 * r] / n) / m - q[5]};
            double* mq[2] = {st.metric_cos, st.metric_sin};
            double* mp[2] = {st.metric_p_cos, st.metric_p_sin};
            const double w2 = st.omega[r] * st.omega[r];
            for (int b = 0; b < 2; ++b) {   // cresso_v5.py:1064-1088
                const double pv = mp[b][r] * damp + h.metric_dt * (port[b] - w2 * mq[b][r]);
                mp[b][r] = pv;
                mq[b][r] = fmin(fmax(mq[b][r] + h.metric_dt * pv, -3.0), 3.0);
            }
            c->rc[0][r][0] = st.metric_cos[r] * g.shrink;
            c->rc[0][r][1] = st.metric_sin[r] * g.shrink;
            // prediction with the pre-contact state (cresso_v5.py:1204-1206)
            const double gt = sigmoid_d(h.confidence_gain * st.conf[r]);
            c->rc[1][r][0] = st.q_cos[r] * g.shrink * gt;
            c->rc[1][r][1] = st.q_sin[r] * g.shrink * gt;
        }
        // port histogram fixed point: |P| <= (1 + transport_mix) 1e4 + max |pred|
        double pm = 0.0;
        for (int r = 0; r < R; ++r) {
            const double* q = A.nst + 8 * r;
            pm += fabs(c->rc[1][r][0]) * q[6] + fabs(c->rc[1][r][1]) * q[7];
        }
        const double vmax = (1.0 + h.transport_mix) * 1.0e4 + pm * (1.0 + 1e-9) + 1.0;
        const int F = (int)floor(62.0 + c->k_lo - log2(vmax * c32->cmax) - 1e-6);
        c->fP = ldexp(1.0, F < 900 ? F : 900);
        const double icoup = hard ? h.instant_metric_coupling : 0.0;
        const double ip = fmax(h.instant_metric_power, 0.25);
        c->inst = (icoup != 0.0 && g.n > 1) ? 1 : 0;
        c->kappa = icoup / ((double)g.nd * ip);
        c->gden = fmax(A.sums[1] / n, eps);
        c->ls_on = h.local_sharpness != 0.0 ? 1 : 0;
    }
    // hash metric per table (cresso_v5.py:1014-1026)
    if (A.hash_on) {
        const int TB = g.T * g.B;
        const double ex = h.hash_metric_coupling / fmax(0.25, h.energy_power);
        for (int t = 0; t < g.T; ++t) {
            double acc[1] = {0.0};
            for (int b = threadIdx.x; b < g.B; b += D_NT) {
                const int i = t * g.B + b;
                const double cell = from_two_word(A.hist[TB + i], A.hist[i], c->fds, c->lo_unit) /
                                    fmax((double)A.counts[i], 1.0);
                const double e = A.step <= 1 ? cell : st.hash_energy[i] * h.hash_decay + cell * (1.0 - h.hash_decay);
                st.hash_energy[i] = e;
                acc[0] += e;
            }
            block_sum<1>(acc, red);
            const double mean = fmax(acc[0] / (double)g.B, eps);
            for (int b = threadIdx.x; b < g.B; b += D_NT) {
                const int i = t * g.B + b;
                const double hm = fmax(st.hash_energy[i] / mean, eps);
                const double hp = pow(hm, ex);
                A.lt[i] = log(fmax(fmin(fmax(hp, 0.08), 12.0), eps));
            }
        }
    }
    // instant metric: per axis, log(max(mean_k / max(mean of the means, eps), eps)) (cresso_v5.py:243-262)
    const double icoup = hard ? h.instant_metric_coupling : 0.0;
    if (icoup != 0.0 && g.nd >= 2 && g.n > 1) {
        for (int a = 0; a < g.nd; ++a) {
            const double cnt = (double)(g.n / g.dim[a]);
            double acc[1] = {0.0};
            for (int64_t k = threadIdx.x; k < g.dim[a]; k += D_NT) acc[0] += A.marg[g.aoff[a] + k] / cnt;
            block_sum<1>(acc, red);
            const double mm = fmax(acc[0] / (double)g.dim[a], eps);
            for (int64_t k = threadIdx.x; k < g.dim[a]; k += D_NT)
                A.terms[g.aoff[a] + k] = log(fmax((A.marg[g.aoff[a] + k] / cnt) / mm, eps));
        }
    }
}

// the tangent field of one element (cresso_v5.py:1090-1128)
template <int RM>
__device__ __forceinline__ double tangent_at(const DGeo& g, const DArgs& A, const Ctrl64* c, const cresso_hyper& h,
                                             int64_t i, const int64_t (&cc)[8], const double (&cn)[RM],
                                             const double (&sn)[RM], double f) {
    const double eps = A.eps, s = c->s;
    const double rel = rel_of(f, s, eps);
    double hm = 1.0;
    if (A.hash_on) {
        double ls = 0.0;
        for (int t = 0; t < g.T; ++t) ls = ls + A.lt[t * g.B + bin_of(g, A.bins, i, t)];
        hm = fmin(fmax(exp(ls / (double)g.T), 0.08), 12.0);
    }
    const double logm = fmin(fmax(recon<RM>(c->rc[0], cn, sn, g.R), -3.0), 3.0);
    const double metric = fmin(fmax(exp(h.metric_coupling * logm), 0.06), 16.0);
    double local = 1.0;
    if (c->ls_on) local = fmin(fmax(1.0 + h.local_sharpness * sqrt(fmin(rel, 100.0)), 1.0), 8.0);
    double inst = 1.0;
    if (c->inst) {
        double lg;
        if (g.nd == 1) {
            const double dens = fmin(pow(fmax(rel, eps), fmax(h.instant_metric_power, 0.25)), 1.0e6);
            lg = log(fmax(dens / c->gden, eps));
        } else {
            lg = A.terms[g.aoff[0] + cc[0]];
            for (int a = 1; a < g.nd; ++a) lg = lg + A.terms[g.aoff[a] + cc[a]];
        }
        inst = fmin(fmax(exp(c->kappa * lg), 0.08), 12.0);
    }
    const double den = s * metric * local * inst * hm + eps;
    return fmin(fmax(f / den, -1.0e4), 1.0e4);
}

// C: t (stored), e = t - pred, port P = e + transport_mix t: sum e^2, port
// histograms, projections of P and (echo) of t
template <int RM>
__global__ __launch_bounds__(D_NT) void d_sweepC_kernel(DGeo g, DArgs A, cresso_hyper h, int echo_on) {
    const Ctrl64* c = A.ctrl;
    const bool lds = g.T * g.B <= D_LDS_TB;
    __shared__ unsigned long long s_h[2 * D_LDS_TB];
    const int TB = g.T * g.B;
    if (A.hash_on && lds) {
        for (int i = threadIdx.x; i < 2 * TB; i += D_NT) s_h[i] = 0ull;
        __syncthreads();
    }
    const double fs = c->fP, lu = c->lo_unit, ilu = 1.0 / lu, tm = h.transport_mix;
    double v[1 + 4 * RM];
#pragma unroll
    for (int i = 0; i < 1 + 4 * RM; ++i) v[i] = 0.0;
    for (int64_t i = (int64_t)blockIdx.x * D_NT + threadIdx.x; i < g.n; i += (int64_t)gridDim.x * D_NT) {
        const double f = force_at(A.grad, A.param, i, A.sg, A.wd);
        int64_t cc[8];
        coords_of(g, i, cc);
        double cn[RM], sn[RM];
        carriers<RM>(g, A.meta, A.tab, A.nst, cc, cn, sn);
        const double t = tangent_at<RM>(g, A, c, h, i, cc, cn, sn, f);
        A.tbuf[i] = t;
        const double e = t - recon<RM>(c->rc[1], cn, sn, g.R);
        v[0] += e * e;
        const double P = e + tm * t;
#pragma unroll
        for (int r = 0; r < RM; ++r) {
            v[1 + 2 * r] += P * cn[r];
            v[2 + 2 * r] += P * sn[r];
            if (echo_on) {
                v[1 + 2 * RM + 2 * r] += t * cn[r];
                v[2 + 2 * RM + 2 * r] += t * sn[r];
            }
        }
        if (A.hash_on) {
            unsigned long long hi, lo;
            two_word(P, fs, lu, ilu, hi, lo);
            for (int tt = 0; tt < g.T; ++tt) {
                const int b = tt * g.B + bin_of(g, A.bins, i, tt);
                if (lds) {
                    atomicAdd(&s_h[b], lo);
                    if (hi) atomicAdd(&s_h[TB + b], hi);
                } else {
                    atomicAdd(&A.hist[2 * TB + b], lo);
                    if (hi) atomicAdd(&A.hist[3 * TB + b], hi);
                }
            }
        }
    }
    if (A.hash_on && lds) {
        __syncthreads();
        for (int i = threadIdx.x; i < 2 * TB; i += D_NT)
            if (s_h[i]) atomicAdd(&A.hist[2 * TB + i], s_h[i]);
    }
    // partial layout: 0 sum e^2, 1.. P projections (C, S per mode), then t projections
    double w[1 + 4 * RM];
#pragma unroll
    for (int q = 0; q < 1 + 4 * RM; ++q) w[q] = v[q];
    __shared__ double red[D_NW * (1 + 4 * RM)];
    block_sum<1 + 4 * RM>(w, red);
    if (threadIdx.x == 0) {
        double* row = A.part + (size_t)blockIdx.x * D_NV;
        row[0] = w[0];
        for (int q = 0; q < 2 * g.R; ++q) {
            row[1 + q] = w[1 + q];
            row[1 + 2 * g.R + q] = w[1 + 2 * RM + q];
        }
    }
}

// one bank of the contact oscillator (cresso_v5.py:914-943), one thread
__device__ void contact_bank(double* q, double* pm, const double* port, const double* omega, double* calcium,
                             double* action, double sur, int R, const cresso_hyper& h) {
    const double dt = h.dt, rd = h.refractory_decay;
    double gp[SP_MAXR];
    const double plast = 1.0 + h.surprise_gain * sur / (1.0 + sur);
    const double brake = 1.0 / (1.0 + h.surprise_brake * sur);
    double p2 = 0.0, wq2 = 0.0, pw = 0.0;
    for (int r = 0; r < R; ++r) {
        calcium[r] = calcium[r] * rd + fabs(port[r]) * (1.0 - rd);
        const double gate = 1.0 / (1.0 + h.refractory_gain * calcium[r]);
        gp[r] = port[r] * gate * plast * brake;
        const double wq = omega[r] * q[r];
        p2 += pm[r] * pm[r];
        wq2 += wq * wq;
        pw += gp[r] * pm[r];
    }
    const double energy = 0.5 * (p2 / (double)R + wq2 / (double)R);
    const double power = pw / (double)R;
    *action = *action * 0.985 + dt * (power - energy);
    const double fr = h.impulse_friction + h.contact_gain * tanh(fabs(*action));
    const double damp = fmax(1.0 - dt * fr, 0.0);
    for (int r = 0; r < R; ++r) {
        const double qv = q[r];
        const double drive = gp[r] - h.restoring * (omega[r] * omega[r]) * qv - h.cubic * (qv * qv * qv);
        pm[r] = pm[r] * damp + dt * drive;
        q[r] = fmin(fmax(q[r] + dt * pm[r], -8.0), 8.0);
    }
}

// C's finish: surprise, hash impulse, confidence, contact oscillator,
// post-contact prediction and echo coefficients
__global__ __launch_bounds__(D_NT) void d_finC_kernel(DGeo g, DArgs A, DState st, cresso_hyper h, int echo_on) {
    Ctrl64* c = A.ctrl;
    const double n = (double)g.n, eps = h.eps;
    const int R = g.R;
    if (A.hash_on) {   // cresso_v5.py:1140-1184
        const int TB = g.T * g.B;
        for (int i = threadIdx.x; i < TB; i += D_NT) {
            const double cp = from_two_word(A.hist[3 * TB + i], A.hist[2 * TB + i], c->fP, c->lo_unit) /
                              fmax((double)A.counts[i], 1.0);
            const double ref = st.hash_refractory[i] * h.hash_decay + fabs(cp) * (1.0 - h.hash_decay);
            st.hash_refractory[i] = ref;
            const double gate = 1.0 / (1.0 + h.refractory_gain * ref);
            st.hash_impulse[i] = st.hash_impulse[i] * h.hash_impulse_decay + (cp * gate) * (1.0 - h.hash_impulse_decay);
        }
    }
    if (threadIdx.x != 0) return;
    const double sur_now = sqrt(A.sums[0] / n + eps);
    const double sur = A.step <= 1 ? sur_now : *st.surprise * h.surprise_decay + sur_now * (1.0 - h.surprise_decay);
    *st.surprise = sur;
    double pcp[SP_MAXR], psp[SP_MAXR];
    for (int r = 0; r < R; ++r) {
        pcp[r] = A.sums[1 + 2 * r] / n;
        psp[r] = A.sums[2 + 2 * r] / n;
        // confidence with the pre-contact q (cresso_v5.py:1199-1202)
        const double qc = st.q_cos[r], qs = st.q_sin[r];
        const double pe = sqrt(pcp[r] * pcp[r] + psp[r] * psp[r] + eps);
        const double support = (pcp[r] * qc + psp[r] * qs) / (pe * sqrt(qc * qc + qs * qs + eps) + eps);
        const double cf = st.conf[r] * h.confidence_decay + fmin(fmax(support, -1.0), 1.0) * (1.0 - h.confidence_decay);
        st.conf[r] = fmin(fmax(cf, -4.0), 4.0);
    }
    contact_bank(st.q_cos, st.p_cos, pcp, st.omega, st.calcium_cos, st.action, sur, R, h);
    contact_bank(st.q_sin, st.p_sin, psp, st.omega, st.calcium_sin, st.action, sur, R, h);
    for (int r = 0; r < R; ++r) {
        const double gt = sigmoid_d(h.confidence_gain * st.conf[r]);
        c->rc[2][r][0] = st.q_cos[r] * g.shrink * gt;
        c->rc[2][r][1] = st.q_sin[r] * g.shrink * gt;
        c->rc[3][r][0] = echo_on ? (A.sums[1 + 2 * R + 2 * r] / n) * g.shrink : 0.0;
        c->rc[3][r][1] = echo_on ? (A.sums[2 + 2 * R + 2 * r] / n) * g.shrink : 0.0;
    }
}

// fields of the drive at one element: pred', err', echo, hash prediction
template <int RM>
__device__ __forceinline__ void drive_fields(const DGeo& g, const DArgs& A, const Ctrl64* c, int64_t i, int echo_on,
                                             double t, double& pred, double& err, double& echo, double& hp) {
    int64_t cc[8];
    coords_of(g, i, cc);
    double cn[RM], sn[RM];
    carriers<RM>(g, A.meta, A.tab, A.nst, cc, cn, sn);
    pred = recon<RM>(c->rc[2], cn, sn, g.R);
    err = t - pred;
    echo = echo_on ? recon<RM>(c->rc[3], cn, sn, g.R) : 0.0;
    hp = 0.0;
    if (A.hash_on) {
        double acc = 0.0;
        for (int t2 = 0; t2 < g.T; ++t2) acc = acc + A.imp[t2 * g.B + bin_of(g, A.bins, i, t2)];
        hp = acc / (double)g.T;
    }
}

// rat, bnd = clip tanh(t/clip), root_raw = sign(t) sqrt(min(|t|, clip^2) + eps) (cresso_v5.py:1318-1324)
__device__ __forceinline__ void shapes(double t, double clip, double eps, double& rat, double& bnd, double& root) {
    bnd = tanh(t / clip) * clip;
    rat = t / (1.0 + fabs(t) / clip);
    const double sgn = t > 0.0 ? 1.0 : (t < 0.0 ? -1.0 : 0.0);
    root = sgn * sqrt(fmin(fabs(t), clip * clip) + eps);
}

// D: the drive's 15 moments: tt pp tp rr bb oo rb ro bo tr tb to ee echo^2 hp^2
template <int RM>
__global__ __launch_bounds__(D_NT) void d_sweepD_kernel(DGeo g, DArgs A, cresso_hyper h, int echo_on) {
    const Ctrl64* c = A.ctrl;
    const double clip = h.drive_clip, eps = h.eps;
    double v[15];
#pragma unroll
    for (int q = 0; q < 15; ++q) v[q] = 0.0;
    for (int64_t i = (int64_t)blockIdx.x * D_NT + threadIdx.x; i < g.n; i += (int64_t)gridDim.x * D_NT) {
        const double t = A.tbuf[i];
        double pr, e, ec, hp, rat, bnd, root;
        drive_fields<RM>(g, A, c, i, echo_on, t, pr, e, ec, hp);
        shapes(t, clip, eps, rat, bnd, root);
        v[0] += t * t; v[1] += pr * pr; v[2] += t * pr;
        v[3] += rat * rat; v[4] += bnd * bnd; v[5] += root * root;
        v[6] += rat * bnd; v[7] += rat * root; v[8] += bnd * root;
        v[9] += t * rat; v[10] += t * bnd; v[11] += t * root;
        v[12] += e * e; v[13] += ec * ec; v[14] += hp * hp;
    }
    put_partials<15>(v, 15, A.part);
}

// D's finish: the drive coefficients (cresso_v5.py:1303-1345), one thread
__global__ void d_finD_kernel(DGeo g, DArgs A, DState st, cresso_hyper h, int hard, int echo_on) {
    if (threadIdx.x != 0) return;
    Ctrl64* c = A.ctrl;
    const double* m = A.sums;
    const double n = (double)g.n, eps = h.eps;
    const double sur = *st.surprise;
    const double frms = sqrt(m[0] / n + eps);
    const double prms = sqrt(m[1] / n + eps);
    const double align = fmin(fmax((m[2] / n) / (frms * prms + eps), -1.0), 1.0);
    const double agate = prms > sqrt(eps) ? fmin(fmax((align + 1.0) * 0.5, 0.0), 1.0) : 0.0;
    const double warm = h.warmup_steps == 0 ? 1.0 : 1.0 - exp(-(double)A.step / (double)(h.warmup_steps > 1 ? h.warmup_steps : 1));
    const double mix = h.prediction_mix * warm * agate * (1.0 / (1.0 + sur));
    const double rrat = sqrt(m[3] / n + eps);
    const double kroot = rrat / fmax(sqrt(m[5] / n + eps), eps);
    const double spike = h.spike_mix / (1.0 + sur);
    const double rmix = (hard ? h.root_channel_mix : 0.0) / (1.0 + 0.5 * sur);
    // shaped = ar rat + ab bnd + ao root_raw
    const double ar = (1.0 - rmix) * (1.0 - spike), ab = (1.0 - rmix) * spike, ao = rmix * kroot;
    const double sh2 = ar * ar * m[3] + ab * ab * m[4] + ao * ao * m[5] + 2.0 * (ar * ab * m[6] + ar * ao * m[7] + ab * ao * m[8]);
    const double srms = sqrt(sh2 / n + eps);
    const double dmix = h.direct_force_mix / (1.0 + 0.35 * sur);
    const double kdir = srms / fmax(frms, eps);
    const double cr = (1.0 - dmix) * ar, cb = (1.0 - dmix) * ab, co = (1.0 - dmix) * ao, ct = dmix * kdir;
    const double core2 = cr * cr * m[3] + cb * cb * m[4] + co * co * m[5] + ct * ct * m[0] +
                         2.0 * (cr * cb * m[6] + cr * co * m[7] + cb * co * m[8] + ct * cr * m[9] + ct * cb * m[10] + ct * co * m[11]);
    const double crms = sqrt(core2 / n + eps);
    const double erms = sqrt(m[12] / n + eps);
    const double resmix = h.residual_feedback_mix / (1.0 + sur);
    c->mix = mix;
    c->c_rat = cr; c->c_bnd = cb; c->c_root = co; c->c_t = ct;
    c->nov_mix = h.novelty_mix;
    c->nov_div = h.drive_clip * (1.0 + sur);
    c->k_res = resmix * (crms / fmax(erms, eps));
    const bool echo = hard && h.echo_mix != 0.0 && echo_on;
    c->k_echo = echo ? h.echo_mix * (srms / fmax(sqrt(m[13] / n + eps), eps)) : 0.0;
    c->k_hash = (hard && A.hash_on) ? h.hash_drive_mix * (srms / fmax(sqrt(m[14] / n + eps), eps)) : 0.0;
}

template <int RM>
__device__ __forceinline__ double drive_at(const DGeo& g, const DArgs& A, const Ctrl64* c, const cresso_hyper& h,
                                           int64_t i, int echo_on, double t) {
    double pr, e, ec, hp, rat, bnd, root;
    drive_fields<RM>(g, A, c, i, echo_on, t, pr, e, ec, hp);
    shapes(t, h.drive_clip, h.eps, rat, bnd, root);
    const double core = c->c_rat * rat + c->c_bnd * bnd + c->c_root * root + c->c_t * t;
    const double nov = tanh(e / c->nov_div) * h.drive_clip;
    return (1.0 - c->mix) * core + c->mix * pr + c->nov_mix * nov + c->k_res * e + c->k_echo * ec + c->k_hash * hp;
}

// E: the drive (stored over t) and sum drive^2
template <int RM>
__global__ __launch_bounds__(D_NT) void d_sweepE_kernel(DGeo g, DArgs A, cresso_hyper h, int echo_on) {
    const Ctrl64* c = A.ctrl;
    double v[1] = {0.0};
    for (int64_t i = (int64_t)blockIdx.x * D_NT + threadIdx.x; i < g.n; i += (int64_t)gridDim.x * D_NT) {
        const double d = drive_at<RM>(g, A, c, h, i, echo_on, A.tbuf[i]);
        A.tbuf[i] = d;
        v[0] += d * d;
    }
    put_partials<1>(v, 1, A.part);
}

// E's finish: drive-energy reservoir and gain (cresso_v5.py:1346-1352)
__global__ void d_finE_kernel(DGeo g, DArgs A, DState st, cresso_hyper h) {
    if (threadIdx.x != 0) return;
    const double now = A.sums[0] / (double)g.n;
    const double de = A.step <= 1 ? now : *st.drive_energy * h.reservoir_decay + now * (1.0 - h.reservoir_decay);
    *st.drive_energy = de;
    A.ctrl->gain = fmin(fmax(h.target_update_rms / sqrt(de + h.eps), h.min_gain), h.max_gain);
}

// F: param -= lr * drive * gain (cresso_v5.py:1353)
__global__ __launch_bounds__(D_NT) void d_sweepF_kernel(DGeo g, DArgs A, double lr) {
    const double gain = A.ctrl->gain;
    for (int64_t i = (int64_t)blockIdx.x * D_NT + threadIdx.x; i < g.n; i += (int64_t)gridDim.x * D_NT)
        A.param[i] = A.param[i] + (-lr) * (A.tbuf[i] * gain);
}

template <typename T> T* wat(void* ws, size_t off) { return reinterpret_cast<T*>(reinterpret_cast<char*>(ws) + off); }

template <int RM>
int32_t run_f64(const cresso_spectral_plan& P, const cresso_spectral_desc& d, void* ws, const cresso_hyper& h,
                hipStream_t s) {
    const Offs64& o = P.o64;
    const DGeo g = dgeo(P);
    const DState st = dstate(d);
    const int hash_on = (d.hash_energy != nullptr && !P.bins_off) ? 1 : 0;
    const int hard = d.hard ? 1 : 0;
    const int echo_on = (hard && h.echo_mix != 0.0) ? 1 : 0;
    DArgs A;
    A.grad = (const double*)d.grad;
    A.param = (double*)d.param;
    A.bins = wat<unsigned char>(ws, P.o.bins);
    A.counts = wat<unsigned long long>(ws, P.o.counts);
    A.meta = wat<ModeMeta>(ws, P.o.meta);
    A.tab = wat<AxisTab>(ws, o.tab);
    A.nst = wat<double>(ws, o.nst);
    A.part = wat<double>(ws, o.part);
    A.sums = wat<double>(ws, o.sums);
    A.hist = wat<unsigned long long>(ws, o.hist);
    A.lt = wat<double>(ws, o.lt);
    A.imp = st.hash_impulse;
    A.marg = wat<double>(ws, o.marg);
    A.terms = wat<double>(ws, o.terms);
    A.ctrl = wat<Ctrl64>(ws, o.ctrl);
    A.tbuf = wat<double>(ws, o.tbuf);
    A.sg = h.maximize ? -1.0 : 1.0;
    A.wd = h.weight_decay;
    A.eps = h.eps;
    A.hash_on = hash_on;
    A.step = d.step;
    const Ctrl* c32 = wat<Ctrl>(ws, P.o.ctrl);
    const dim3 grid(g.nblk), blk(D_NT);
    const int64_t TB = (int64_t)g.T * g.B;
    if (hash_on)
        hipLaunchKernelGGL(d_clear_kernel, dim3((unsigned)std::min<int64_t>(1024, (4 * TB + 255) / 256)), dim3(256), 0, s,
                           A.hist, 4 * TB);
    hipLaunchKernelGGL(d_sweepA_kernel, grid, blk, 0, s, g, A);
    hipLaunchKernelGGL(d_reduce_kernel, dim3(2), blk, 0, s, A.part, g.nblk, 1, A.sums);
    hipLaunchKernelGGL(d_finA_kernel, dim3(1), dim3(64), 0, s, g, A, st, c32, h);
    hipLaunchKernelGGL((d_sweepB_kernel<RM>), grid, blk, 0, s, g, A, h);
    const bool axes = hard && h.instant_metric_coupling != 0.0 && g.nd >= 2 && g.n > 1;
    if (axes)
        for (int a = 0; a < g.nd; ++a)
            hipLaunchKernelGGL(d_marg_kernel, dim3((unsigned)((g.dim[a] + D_NW - 1) / D_NW)), blk, 0, s, g, A, h, a);
    hipLaunchKernelGGL(d_reduce_kernel, dim3(2 + 2 * g.R), blk, 0, s, A.part, g.nblk, 1 << 30, A.sums);
    hipLaunchKernelGGL(d_finB_kernel, dim3(1), blk, 0, s, g, A, st, c32, h, hard);
    hipLaunchKernelGGL((d_sweepC_kernel<RM>), grid, blk, 0, s, g, A, h, echo_on);
    hipLaunchKernelGGL(d_reduce_kernel, dim3(1 + 4 * g.R), blk, 0, s, A.part, g.nblk, 1 << 30, A.sums);
    hipLaunchKernelGGL(d_finC_kernel, dim3(1), blk, 0, s, g, A, st, h, echo_on);
    hipLaunchKernelGGL((d_sweepD_kernel<RM>), grid, blk, 0, s, g, A, h, echo_on);
    hipLaunchKernelGGL(d_reduce_kernel, dim3(15), blk, 0, s, A.part, g.nblk, 1 << 30, A.sums);
    hipLaunchKernelGGL(d_finD_kernel, dim3(1), dim3(64), 0, s, g, A, st, h, hard, echo_on);
    hipLaunchKernelGGL((d_sweepE_kernel<RM>), grid, blk, 0, s, g, A, h, echo_on);
    hipLaunchKernelGGL(d_reduce_kernel, dim3(1), blk, 0, s, A.part, g.nblk, 1 << 30, A.sums);
    hipLaunchKernelGGL(d_finE_kernel, dim3(1), dim3(64), 0, s, g, A, st, h);
    hipLaunchKernelGGL(d_sweepF_kernel, grid, blk, 0, s, g, A, h.lr);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? CRESSO_OK : hip_fail(e, "spectral route (fp64): launch");
}

template <int RM>
void init_f64_tables(const cresso_spectral_plan& P, void* ws, hipStream_t s) {
    const Offs64& o = P.o64;
    const DGeo g = dgeo(P);
    const ModeMeta* meta = wat<ModeMeta>(ws, P.o.meta);
    AxisTab* tab = wat<AxisTab>(ws, o.tab);
    double* part = wat<double>(ws, o.part);
    double* sums = wat<double>(ws, o.sums);
    double* nst = wat<double>(ws, o.nst);
    double* mu = wat<double>(ws, o.lt);   // scratch for the raw means (2 R doubles)
    const int64_t total = (int64_t)g.R * g.sumd;
    hipLaunchKernelGGL(d_tab_kernel, dim3((unsigned)std::min<int64_t>(4096, (total + D_NT - 1) / D_NT)), dim3(D_NT), 0, s,
                       g, wat<AxisConst64>(ws, o.axc), tab);
    hipLaunchKernelGGL((d_stats_kernel<RM, 1>), dim3(g.nblk), dim3(D_NT), 0, s, g, meta, tab, mu, part);
    hipLaunchKernelGGL(d_reduce_kernel, dim3(2 * g.R), dim3(D_NT), 0, s, part, g.nblk, 1 << 30, sums);
    hipLaunchKernelGGL(d_stats_mid_kernel, dim3(1), dim3(64), 0, s, g, sums, mu);
    hipLaunchKernelGGL((d_stats_kernel<RM, 2>), dim3(g.nblk), dim3(D_NT), 0, s, g, meta, tab, mu, part);
    // centred second moments and sums (values 0 .. 4 SP_MAXR), maxima after
    hipLaunchKernelGGL(d_reduce_kernel, dim3(6 * SP_MAXR), dim3(D_NT), 0, s, part, g.nblk, 4 * SP_MAXR, sums);
    hipLaunchKernelGGL(d_stats_fin_kernel, dim3(1), dim3(64), 0, s, g, meta, mu, sums, nst);
}

}  // namespace

// fp64 regions of a plan (called by the planner for work == CRESSO_F64)
size_t plan_f64_layout(cresso_spectral_plan& P, size_t off) {
    Offs64& o = P.o64;
    const Geom& g = P.g;
    auto take = [&](size_t bytes) { size_t at = off; off = (off + bytes + 255) & ~(size_t)255; return at; };
    int64_t sumd = 0;
    for (int a = 0; a < g.ndim; ++a) sumd += P.shape[a];
    o.sumd = sumd;
    o.nblk = (int32_t)std::max<int64_t>(1, std::min<int64_t>(1024, (g.n + D_NT - 1) / D_NT));
    const size_t TB = (size_t)g.T * g.B;
    o.axc = take(sizeof(AxisConst64) * (size_t)g.R * g.ndim);
    o.tab = take(sizeof(AxisTab) * (size_t)g.R * (size_t)sumd);
    o.nst = take(sizeof(double) * 8 * (size_t)g.R);
    o.sums = take(sizeof(double) * D_NV);
    o.part = take(sizeof(double) * D_NV * (size_t)o.nblk);
    o.hist = take(sizeof(unsigned long long) * 4 * TB);
    o.lt = take(sizeof(double) * std::max<size_t>(TB, 2 * SP_MAXR));
    o.marg = take(sizeof(double) * (size_t)sumd);
    o.terms = take(sizeof(double) * (size_t)sumd);
    o.ctrl = take(sizeof(Ctrl64));
    o.tbuf = take(sizeof(double) * (size_t)g.n);
    return off;
}

int32_t workspace_init_f64(const cresso_spectral_plan& P, void* ws, hipStream_t s) {
    hipError_t e = hipMemcpyAsync(wat<AxisConst64>(ws, P.o64.axc), P.axc64.data(), sizeof(AxisConst64) * P.axc64.size(),
                                  hipMemcpyHostToDevice, s);
    if (e != hipSuccess) return hip_fail(e, "spectral route (fp64): workspace upload");
    if (P.g.R <= 8)
        init_f64_tables<8>(P, ws, s);
    else if (P.g.R <= 16)
        init_f64_tables<16>(P, ws, s);
    else
        init_f64_tables<32>(P, ws, s);
    e = hipGetLastError();
    return e == hipSuccess ? CRESSO_OK : hip_fail(e, "spectral route (fp64): workspace init");
}

int32_t spectral_run_f64(const cresso_spectral_plan& P, const cresso_spectral_desc& d, void* ws, const cresso_hyper& h,
                         hipStream_t s) {
    // ranks 17-32: correct, not tuned (the per-thread carrier arrays spill to scratch)
    if (P.g.R <= 8) return run_f64<8>(P, d, ws, h, s);
    if (P.g.R <= 16) return run_f64<16>(P, d, ws, h, s);
    return run_f64<32>(P, d, ws, h, s);
}

}  // namespace cresso
