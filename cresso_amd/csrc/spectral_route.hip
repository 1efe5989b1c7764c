// Spectral / coordinate-hash route of CRESSO5 on gfx950 (large tensors).
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
//   panel in LDS from the mode coefficients.
// * Step = 5 sweeps over the field, each followed by a one-block finalize
//   (deterministic fixed-order fp64 reductions of per-block partials) that
//   runs the rank-level recurrences and writes the next sweep's coefficients:
//     S1 sum f^2 -> F1 force RMS, scale
//     S2 density: hash histograms (64-bit fixed point, integer atomics),
//        log-density projection, axis density sums -> F2 hash metric tables,
//        metric oscillator, recon coefficients; M1 instant-metric factors
//     S3 tangent t (stored), surprise, port projection, port histograms,
//        echo projection, 13 moments of t -> F3 surprise, hash impulse,
//        confidence, contact oscillator, core coefficients
//     S4 the 22 cross moments of {core, pred, nov, err, echo, hash} that give
//        every remaining RMS and the drive energy in closed form -> F4 gain
//     S5 param -= lr * cast(drive * gain)
#include "common.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <tuple>
#include <vector>

namespace cresso {
namespace {

constexpr int SP_NT = 256;
constexpr int SP_MAXR = 16;
constexpr int SP_MAXT = 8;
constexpr int SP_FIN_NT = 1024;

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
    int32_t binbytes, bpb, one_d, pad;
};

struct Offs {
    size_t axc, meta, csrc, rowtab, coltab, stats, bounds, counts, bins, tbuf, part, hist, lt, imp, alpha, rowfx, colfx,
        rowfac, colfac, terms, ctrl, total;
};

// per-step device scalars (written by finalize kernels)
struct Ctrl {
    float scale, inv_s;
    float gden, kappa;
    float rc[4][SP_MAXR][2];  // recon coefficients: 0 metric, 1 pred, 2 pred', 3 echo
    float rconst[4];
    double hs_ds, hs_P;       // fixed-point scales of the histograms
    float nscale, cr, cb, co, ct;
    float dcore, dpred, dnov, derr, decho, dhp, gain;
    float pad[3];
};

// state pointers of one tensor (kernel argument)
struct SpecState {
    float *force_rms, *drive_energy, *surprise, *action;
    const float* omega;
    float *q_cos, *q_sin, *p_cos, *p_sin, *metric_cos, *metric_sin, *metric_p_cos, *metric_p_sin;
    float *calcium_cos, *calcium_sin, *conf;
    float *hash_energy, *hash_impulse, *hash_refractory;
};

constexpr int NV1 = 1;
constexpr int NV2 = 2 + 2 * SP_MAXR;            // sum L, sum dens, proj L (C,S)
constexpr int NV3 = 15 + 4 * SP_MAXR;           // see sweep3
constexpr int NV4 = 22;
constexpr int NVMAX = NV3;

__device__ __forceinline__ float uniform(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
}

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
// bound of max|C_n|, max|S_n| used to size fixed-point histograms.
__global__ __launch_bounds__(SP_FIN_NT) void ws_stats_kernel(Geom g, const ModeMeta* __restrict__ meta,
                                                             const float* __restrict__ rowtab,
                                                             const float* __restrict__ coltab, double* __restrict__ stats,
                                                             double* __restrict__ bounds) {
    __shared__ double red[16 * 8];
    const int tid = threadIdx.x;
    for (int r = 0; r < g.R; ++r) {
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
        __syncthreads();
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

// Block partials, one value at a time: DPP wave totals into LDS [wave][V],
// then a fixed-order sum over the block's waves, written value-major
// part[v][block].
struct Partials {
    float* lds;
    int V;
    __device__ __forceinline__ void add(int idx, float x) {
        const float w = wave_total(x);
        if ((threadIdx.x & 63) == 63) lds[(threadIdx.x >> 6) * V + idx] = w;
    }
    __device__ __forceinline__ void flush(double* part, int nblk) {
        __syncthreads();
        for (int v = threadIdx.x; v < V; v += SP_NT) {
            double s = 0.0;
            for (int w = 0; w < SP_NT / 64; ++w) s += (double)lds[w * V + v];
            part[(size_t)v * nblk + blockIdx.x] = s;
        }
    }
};

// Non-negative float (already scaled by a power of two, < 2^62) to a 64-bit
// fixed-point integer, truncating: two exact 32-bit conversions.
__device__ __forceinline__ unsigned long long to_fixed_u(float x) {
    const float hf = floorf(x * 2.3283064365386963e-10f);  // x / 2^32 (exact scaling)
    const float lf = fmaf(-hf, 4294967296.0f, x);           // x - hi*2^32: exact, in [0, 2^32)
    return ((unsigned long long)(unsigned)hf << 32) | (unsigned long long)(unsigned)lf;
}
__device__ __forceinline__ unsigned long long to_fixed_s(float x) {
    const unsigned long long u = to_fixed_u(fabsf(x));
    return x < 0.f ? (0ull - u) : u;
}

template <int KM>
__device__ __forceinline__ void load_cols(const Geom& g, const float* __restrict__ coltab, const Tile& t, float (&b)[KM]) {
#pragma unroll
    for (int k = 0; k < KM; ++k) b[k] = (k < g.K && t.colok) ? coltab[(size_t)k * g.cols + t.col] : 0.f;
}

// reconstruction at (row, lane column): alpha row (wave-uniform) against the
// lane's column carriers
// (alpha rows are zero beyond the K live carriers and the lane's b is zero
// there too, so the loop has no guards and the row loads vectorize)
template <int KM>
__device__ __forceinline__ float recon(const float* __restrict__ al, const float (&b)[KM]) {
    float v = al[KM];
#pragma unroll
    for (int k = 0; k < KM; ++k) v += al[k] * b[k];
    return v;
}

// lane contribution of a projection (Z1/Z2 accumulated over the lane's rows)
// reduced mode by mode into partial slots base + 2r (C) and base + 2r + 1 (S)
template <int RM, int KM>
__device__ __forceinline__ void proj_finish(const Geom& g, const ModeMeta* __restrict__ meta, const float (&Z1)[RM],
                                            const float (&Z2)[RM], const float (&b)[KM], Partials& P, int base) {
#pragma unroll
    for (int r = 0; r < RM; ++r) {
        if (r < g.R) {
            const ModeMeta m = meta[r];
            float b1 = 0.f, b2 = 0.f;
#pragma unroll
            for (int k = 0; k < KM; ++k) {
                if (k == m.k1) b1 = b[k];
                if (k == m.k2) b2 = b[k];
            }
            float c, sn;
            if (m.type == M_ADD) {
                c = b1 * Z1[r] - b2 * Z2[r];
                sn = b1 * Z2[r] + b2 * Z1[r];
            } else {
                c = b1 * Z1[r];
                sn = b2 * Z2[r];
            }
            P.add(base + 2 * r, c);
            P.add(base + 2 * r + 1, sn);
        }
    }
}

// rat = t/(1+|t|/clip), bnd = clip*tanh(t/clip), root = sign(t)*sqrt(min(|t|,clip^2)+eps)
// (cresso_v5.py:1321-1324); rat and bnd share one reciprocal.
__device__ __forceinline__ void shape3f(float t, float iclip, float clip, float clip2, float eps, float& rat, float& bnd,
                                        float& root) {
    const float at = fabsf(t);
    const float ex = fexp2(-2.8853900817779268f * at * iclip);
    const float d1 = 1.0f + ex;
    const float d2 = 1.0f + at * iclip;
    const float inv = frcp(d1 * d2);
    const float th = (1.0f - ex) * d2 * inv;
    bnd = copysignf(th, t) * clip;
    rat = t * d1 * inv;
    root = fsign(t) * fsqrt(fminf(at, clip2) + eps);
}

__device__ __forceinline__ float reservoir_f(float old, float cur, double decay, int step) {
    if (step <= 1) return cur;
    return old * (float)decay + (float)(1.0 - decay) * cur;
}

// All partial values of a sweep reduced over blocks in a fixed order; result
// in out[v] (LDS), visible after return.  Each value owns TPV consecutive
// threads (TPV = largest power of two with V*TPV <= block size, at most 64):
// thread j of value v sums blocks j, j+TPV, ... (the group's loads coalesce),
// eight independent accumulators deep, and one thread per value adds the TPV
// sums in order.  No cross-lane traffic; the loads of a thread are all in
// flight together.
__device__ void reduce_all(const double* __restrict__ part, int nblk, int V, double* out) {
    __shared__ double s_seg[SP_FIN_NT];
    const int tid = threadIdx.x;
    int tpv = 64;
    while (tpv > 1 && tpv * V > SP_FIN_NT) tpv >>= 1;
    const int v = tid / tpv, j = tid % tpv;
    if (v < V) {
        const double* __restrict__ p = part + (size_t)v * nblk;
        double a0 = 0.0, a1 = 0.0, a2 = 0.0, a3 = 0.0, a4 = 0.0, a5 = 0.0, a6 = 0.0, a7 = 0.0;
        int b = j;
        const int step = tpv;
        for (; b + 7 * step < nblk; b += 8 * step) {
            a0 += p[b];
            a1 += p[b + step];
            a2 += p[b + 2 * step];
            a3 += p[b + 3 * step];
            a4 += p[b + 4 * step];
            a5 += p[b + 5 * step];
            a6 += p[b + 6 * step];
            a7 += p[b + 7 * step];
        }
        for (; b < nblk; b += step) a0 += p[b];
        s_seg[tid] = ((a0 + a1) + (a2 + a3)) + ((a4 + a5) + (a6 + a7));
    }
    __syncthreads();
    if (tid < V) {
        double sum = 0.0;
        for (int k = 0; k < tpv; ++k) sum += s_seg[tid * tpv + k];
        out[tid] = sum;
    }
    __syncthreads();
}

// ---------------------------------------------------------------------------
// S1: sum f^2 over contiguous chunks (float4 loads when aligned)
// ---------------------------------------------------------------------------
template <typename PT, typename GT, bool V4>
__global__ __launch_bounds__(SP_NT) void sweep1_kernel(Geom g, const GT* __restrict__ grad, const PT* __restrict__ param,
                                                       double* __restrict__ part, cresso_hyper h) {
    __shared__ float red[4];
    const float wd = (float)h.weight_decay;
    const bool wd_on = h.weight_decay != 0.0;
    const int64_t beg = (int64_t)blockIdx.x * g.chunk1;
    const int64_t end = beg + g.chunk1 < g.n ? beg + g.chunk1 : g.n;
    const float sg = h.maximize ? -1.f : 1.f;
    float a = 0.f;
    const int64_t vend = beg + ((end - beg) & ~(int64_t)3);
    if (V4) {
        for (int64_t e = beg + 4 * (int64_t)threadIdx.x; e < vend; e += 4 * SP_NT) {
            float f[4];
            Ld4<GT>::go(grad, e, f);
            if (wd_on) {
                float pv[4];
                Ld4<PT>::go(param, e, pv);
#pragma unroll
                for (int c = 0; c < 4; ++c) f[c] = sg * f[c] + wd * pv[c];
            }
#pragma unroll
            for (int c = 0; c < 4; ++c) a += f[c] * f[c];
        }
    }
    // scalar elements: the < 4 tail of a vectorized chunk, or the whole chunk
    for (int64_t i = (V4 ? vend : beg) + threadIdx.x; i < end; i += SP_NT) {
        float f = sg * ld(grad, i);
        if (wd_on) f = f + wd * ld(param, i);
        a += f * f;
    }
    Partials P{red, 1};
    P.add(0, a);
    P.flush(part, g.nblk1);
}

__global__ __launch_bounds__(SP_FIN_NT) void fin1_kernel(Geom g, const double* __restrict__ part, SpecState st,
                                                         Ctrl* __restrict__ ctrl, unsigned long long* __restrict__ rowfx,
                                                         unsigned long long* __restrict__ colfx, int step, cresso_hyper h) {
    __shared__ double red[1];
    reduce_all(part, g.nblk1, 1, red);
    // clear the axis density sums for this step's sweep 2
    for (int64_t i = threadIdx.x; i < g.rows; i += SP_FIN_NT) rowfx[i] = 0ull;
    for (int64_t i = threadIdx.x; i < g.cols; i += SP_FIN_NT) colfx[i] = 0ull;
    if (threadIdx.x == 0) {
        const float eps = (float)h.eps;
        const float now = sqrtf((float)(red[0] / (double)g.n) + eps);
        const float fr = reservoir_f(*st.force_rms, now, h.reservoir_decay, step);
        *st.force_rms = fr;
        const float s = fmaxf(fr, eps);
        ctrl->scale = s;
        ctrl->inv_s = 1.0f / s;
        // density histogram scale: ds = rel^p <= (1e4)^p, at most n elements per bin
        const double dsmax = pow(1.0e4, h.energy_power) + 1.0;
        ctrl->hs_ds = ldexp(1.0, (int)floor(62.0 - log2(dsmax * (double)g.n)));
    }
}

// ---------------------------------------------------------------------------
// S2: density field
// ---------------------------------------------------------------------------
template <int RM, int KM, typename PT, typename GT>
__global__ __launch_bounds__(SP_NT) void sweep2_kernel(Geom g, const GT* __restrict__ grad, const PT* __restrict__ param,
                                                       const float* __restrict__ rowtab, const float* __restrict__ coltab,
                                                       const ModeMeta* __restrict__ meta,
                                                       const unsigned char* __restrict__ bins, const Ctrl* __restrict__ ctrl,
                                                       double* __restrict__ part, unsigned long long* __restrict__ hist,
                                                       unsigned long long* __restrict__ rowfx,
                                                       unsigned long long* __restrict__ colfx, int hash_on, int axes_on,
                                                       cresso_hyper h) {
    extern __shared__ __align__(16) unsigned char dyn[];
    __shared__ float red[4 * NV2];
    const Tile t = tile_of(g);
    // LDS: histogram [T][B] u64, wave row sums [4][PR]
    unsigned long long* s_hist = reinterpret_cast<unsigned long long*>(dyn);
    float* s_wrow = reinterpret_cast<float*>(dyn + sizeof(unsigned long long) * (size_t)g.T * g.B);
    const int TB = g.T * g.B;
    if (hash_on)
        for (int i = threadIdx.x; i < TB; i += SP_NT) s_hist[i] = 0ull;
    __syncthreads();
    float b[KM];
    load_cols<KM>(g, coltab, t, b);
    const float inv_s = ctrl->inv_s;
    const float eps = (float)h.eps;
    const float pw = (float)h.energy_power;
    const float ipw = (float)fmax(h.instant_metric_power, 0.25);
    const bool ip_one = ipw == 1.0f;
    const float wd = (float)h.weight_decay;
    const bool wd_on = h.weight_decay != 0.0;
    const float sg = h.maximize ? -1.f : 1.f;
    const float hs = (float)ctrl->hs_ds;
    float Z1[RM], Z2[RM];
#pragma unroll
    for (int r = 0; r < RM; ++r) Z1[r] = Z2[r] = 0.f;
    float aL = 0.f, aD = 0.f, colsum = 0.f;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int64_t i = t.r0; i < t.r1; ++i) {
        const int lr = (int)(i - t.r0);
        const float* __restrict__ ar = rowtab + i * g.RW;
        float dens = 0.f;
        if (t.colok) {
            const int64_t e = i * g.cols + t.col;
            float f = sg * ld(grad, e);
            if (wd_on) f = f + wd * ld(param, e);
            const float rel = fminf(fabsf(f) * inv_s + eps, 1.0e4f);
            const float ds = fpow(rel, pw);
            const float L = flog1p(ds);
            const float rl = fmaxf(rel, eps);
            dens = fminf(ip_one ? rl : fpow(rl, ipw), 1.0e6f);
            aL += L;
            aD += dens;
            colsum += dens;
#pragma unroll
            for (int q = 0; q < RM; ++q) {
                Z1[q] += ar[2 * q] * L;
                Z2[q] += ar[2 * q + 1] * L;
            }
            if (hash_on) {
                const uint64_t pk = load_bins(bins, e, g.binbytes);
                const unsigned long long v = to_fixed_u(ds * hs);
                for (int tt = 0; tt < g.T; ++tt) atomicAdd(&s_hist[tt * g.B + bin_of(pk, tt, g.bpb)], v);
            }
        }
        if (axes_on) {
            const float ws = wave_total(dens);
            if (lane == 63) s_wrow[wave * g.PR + lr] = ws;
        }
    }
    __syncthreads();
    if (axes_on) {
        // axis density sums: one fixed-point atomic per row of this slab and per column of this panel
        for (int lr = threadIdx.x; lr < (int)(t.r1 - t.r0); lr += SP_NT) {
            float s = 0.f;
            for (int w = 0; w < SP_NT / 64; ++w) s += s_wrow[w * g.PR + lr];
            atomicAdd(&rowfx[t.r0 + lr], to_fixed_u(s * (float)g.hs_row));
        }
        if (t.colok) atomicAdd(&colfx[t.col], to_fixed_u(colsum * (float)g.hs_col));
    }
    if (hash_on)
        for (int i = threadIdx.x; i < TB; i += SP_NT)
            if (s_hist[i]) atomicAdd(&hist[i], s_hist[i]);
    Partials P{red, 2 + 2 * g.R};
    P.add(0, aL);
    P.add(1, aD);
    proj_finish<RM, KM>(g, meta, Z1, Z2, b, P, 2);
    P.flush(part, g.nblk);
}

// ---------------------------------------------------------------------------
// F2: hash metric, metric oscillator, recon coefficients
// ---------------------------------------------------------------------------
// Coefficients (wc, ws) per mode and the constant of
//   shrink * sum_r g_r (cc_r Cn_r + sc_r Sn_r)  (cresso_v5.py:362-376)
// with Cn = (Craw - mu_c) ic; a gate of exactly 0 drops the mode.
__device__ void set_recon(const Geom& g, const double* stats, float (*rc)[2], float& rconst, const float* cc,
                          const float* sc, const float* gates) {
    const double shrink = 1.0 / sqrt(fmax(1.0, 0.7 * log2((double)g.R + 1.0)));
    float cst = 0.f;
    for (int r = 0; r < g.R; ++r) {
        const float gate = gates ? gates[r] : 1.0f;
        float wc = 0.f, ws = 0.f;
        if (gate != 0.0f) {
            const float kc = (float)((double)cc[r] * shrink) * gate;
            const float ks = (float)((double)sc[r] * shrink) * gate;
            wc = (float)((double)kc * stats[4 * r + 1]);
            ws = (float)((double)ks * stats[4 * r + 3]);
            cst -= (float)((double)wc * stats[4 * r + 0] + (double)ws * stats[4 * r + 2]);
        }
        rc[r][0] = wc;
        rc[r][1] = ws;
    }
    rconst = cst;
}

// alpha[row][k] = sum of the coefficients of reconstruction `w` that multiply
// column carrier k at this row (zero for k >= K), alpha[row][KM] = constant.
// One thread per row; reconstructions w0 .. w0+count-1.
template <int RM>
__global__ void alpha_kernel(Geom g, const ModeMeta* __restrict__ meta, const float* __restrict__ rowtab,
                             const Ctrl* __restrict__ ctrl, int w0, int count, float* __restrict__ alpha) {
    constexpr int KM = 2 * RM + 1;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= g.rows) return;
    for (int w = w0; w < w0 + count; ++w) {
        float al[KM + 1];
#pragma unroll
        for (int k = 0; k < KM; ++k) al[k] = 0.f;
        al[KM] = ctrl->rconst[w];
        for (int r = 0; r < g.R; ++r) {
            const ModeMeta m = meta[r];
            const float wc = ctrl->rc[w][r][0], ws = ctrl->rc[w][r][1];
            const float a1 = rowtab[i * g.RW + 2 * r], a2 = rowtab[i * g.RW + 2 * r + 1];
            // additive: C = a1 b1 - a2 b2, S = a2 b1 + a1 b2; product/constant: C = a1 b1, S = a2 b2
            const float c1 = m.type == M_ADD ? wc * a1 + ws * a2 : wc * a1;
            const float c2 = m.type == M_ADD ? ws * a1 - wc * a2 : ws * a2;
#pragma unroll
            for (int k = 0; k < KM; ++k) al[k] += (k == m.k1 ? c1 : 0.f) + (k == m.k2 ? c2 : 0.f);
        }
        float* dst = alpha + ((size_t)w * g.rows + i) * g.KA;
#pragma unroll
        for (int k = 0; k <= KM; ++k) dst[k] = al[k];
    }
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

__global__ __launch_bounds__(SP_FIN_NT) void fin2_kernel(Geom g, const ModeMeta* __restrict__ meta,
                                                         const double* __restrict__ stats, const double* __restrict__ bounds,
                                                         const float* __restrict__ rowtab, const double* __restrict__ part,
                                                         unsigned long long* __restrict__ hist,
                                                         const unsigned long long* __restrict__ counts,
                                                         float* __restrict__ lt, float* __restrict__ alpha, SpecState st,
                                                         Ctrl* __restrict__ ctrl, int step, int hash_on, int hard,
                                                         cresso_hyper h) {
    __shared__ double s_v[NV2];
    __shared__ double red[16];
    __shared__ float s_emean[SP_MAXT];
    const int tid = threadIdx.x;
    const float eps = (float)h.eps;
    const double n = (double)g.n;
    reduce_all(part, g.nblk, 2 + 2 * g.R, s_v);
    // hash energy per table (cresso_v5.py:1012-1056)
    if (hash_on) {
        const int TB = g.T * g.B;
        for (int i = tid; i < TB; i += SP_FIN_NT) {
            const double cnt = (double)counts[i];
            const float cell = (float)((double)(long long)hist[i] / ctrl->hs_ds / fmax(cnt, 1.0));
            hist[i] = 0ull;
            float e = st.hash_energy[i];
            e = step <= 1 ? cell : e * (float)h.hash_decay + (float)(1.0 - h.hash_decay) * cell;
            st.hash_energy[i] = e;
        }
        __syncthreads();
        for (int tt = 0; tt < g.T; ++tt) {
            double s[1] = {0.0};
            for (int b = tid; b < g.B; b += SP_FIN_NT) s[0] += (double)st.hash_energy[tt * g.B + b];
            block_sum<1>(s, red);
            if (tid == 0) s_emean[tt] = (float)(s[0] / (double)g.B);
        }
        __syncthreads();
        const float ex = (float)(h.hash_metric_coupling / fmax(0.25, h.energy_power));
        for (int i = tid; i < TB; i += SP_FIN_NT) {
            const int tt = i / g.B;
            const float hm = fmaxf(st.hash_energy[i] / fmaxf(s_emean[tt], eps), eps);
            lt[i] = logf(fmaxf(clampf(powf(hm, ex), 0.08f, 12.0f), eps));
        }
    }
    // per-mode state staged in LDS by parallel threads; the recurrences run
    // on one thread over LDS, results written back in parallel
    __shared__ double s_st[SP_MAXR][6];
    __shared__ float s_f[SP_MAXR][8];
    __shared__ int s_type[SP_MAXR];
    if (tid < g.R) {
        const int r = tid;
        for (int j = 0; j < 4; ++j) s_st[r][j] = stats[4 * r + j];
        s_st[r][4] = bounds[2 * r];
        s_st[r][5] = bounds[2 * r + 1];
        s_f[r][0] = st.omega[r];
        s_f[r][1] = st.metric_cos[r];
        s_f[r][2] = st.metric_p_cos[r];
        s_f[r][3] = st.metric_sin[r];
        s_f[r][4] = st.metric_p_sin[r];
        s_f[r][5] = st.q_cos[r];
        s_f[r][6] = st.q_sin[r];
        s_f[r][7] = st.conf[r];
        s_type[r] = meta[r].type;
    }
    __syncthreads();
    if (tid == 0) {
        // log-density projections: d = L/max(mean L, eps) - 1, mean(d Cn) = mean(L Cn)/m - mean(Cn)
        const double sumL = s_v[0], sumD = s_v[1];
        const double m = fmax((double)(float)(sumL / n), (double)eps);
        double stt[4 * SP_MAXR];
        for (int r = 0; r < g.R; ++r)
            for (int j = 0; j < 4; ++j) stt[4 * r + j] = s_st[r][j];
        float port[2 * SP_MAXR];
        for (int v = 0; v < 2 * g.R; ++v) {
            const int r = v / 2;
            const double mu = s_st[r][2 * (v & 1)], inv = s_st[r][2 * (v & 1) + 1];
            double pr = (s_v[2 + v] - mu * sumL) * inv / n / m;
            if (s_type[r] == M_ZERO && (v & 1) == 0) pr -= 1.0;  // mean(Cn) = 1 for the constant mode
            port[v] = (float)pr;
        }
        // metric oscillator (cresso_v5.py:1064-1088)
        const float mdt = (float)h.metric_dt;
        const float damp = (float)fmax(0.0, 1.0 - h.metric_dt * h.metric_friction);
        float mcs[SP_MAXR], mss[SP_MAXR];
        for (int r = 0; r < g.R; ++r) {
            const float om = s_f[r][0];
            const float o2 = om * om;
            float mq = s_f[r][1], mp = s_f[r][2];
            mp = mp * damp;
            mp = mp + mdt * (port[2 * r] - o2 * mq);
            mq = clampf(mq + mdt * mp, -3.0f, 3.0f);
            s_f[r][1] = mq; s_f[r][2] = mp; mcs[r] = mq;
            mq = s_f[r][3]; mp = s_f[r][4];
            mp = mp * damp;
            mp = mp + mdt * (port[2 * r + 1] - o2 * mq);
            mq = clampf(mq + mdt * mp, -3.0f, 3.0f);
            s_f[r][3] = mq; s_f[r][4] = mp; mss[r] = mq;
        }
        set_recon(g, stt, ctrl->rc[0], ctrl->rconst[0], mcs, mss, nullptr);
        // prediction with the pre-contact state and gates
        float qc[SP_MAXR], qs[SP_MAXR], gt[SP_MAXR];
        double pmax = 0.0;
        const double shrink = 1.0 / sqrt(fmax(1.0, 0.7 * log2((double)g.R + 1.0)));
        for (int r = 0; r < g.R; ++r) {
            qc[r] = s_f[r][5];
            qs[r] = s_f[r][6];
            gt[r] = sigmoidf_((float)h.confidence_gain * s_f[r][7]);
            pmax += shrink * gt[r] * (fabs((double)qc[r]) * s_st[r][4] + fabs((double)qs[r]) * s_st[r][5]);
        }
        set_recon(g, stt, ctrl->rc[1], ctrl->rconst[1], qc, qs, gt);
        // instant metric: mean density and coupling (cresso_v5.py:243-262)
        ctrl->gden = (float)fmax(sumD / n, (double)eps);
        const float icoup = hard ? (float)h.instant_metric_coupling : 0.0f;
        ctrl->kappa = (float)((double)icoup / ((double)g.ndim * fmax(h.instant_metric_power, 0.25)));
        // fixed-point scale of the port histogram: |P| <= (1+tm)*1e4 + max|pred|, <= n elements per bin
        const double vmax = (1.0 + h.transport_mix) * 1.0e4 + pmax * 1.01 + 1.0;
        ctrl->hs_P = ldexp(1.0, (int)floor(62.0 - log2(vmax * (double)g.n)));
    }
    __syncthreads();
    if (tid < g.R) {
        const int r = tid;
        st.metric_cos[r] = s_f[r][1];
        st.metric_p_cos[r] = s_f[r][2];
        st.metric_sin[r] = s_f[r][3];
        st.metric_p_sin[r] = s_f[r][4];
    }
}

// M1: instant-metric factors (cresso_v5.py:243-262) from the fixed-point axis
// density sums: rows always; columns directly for 2-D tensors.
__global__ void marg_kernel(Geom g, const unsigned long long* __restrict__ rowfx,
                            const unsigned long long* __restrict__ colfx, float* __restrict__ rowfac,
                            float* __restrict__ colfac, const Ctrl* __restrict__ ctrl, float eps) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const float gden = ctrl->gden, kappa = ctrl->kappa;
    if (i < g.rows) {
        const float mean = (float)((double)rowfx[i] / g.hs_row / (double)g.cols);
        rowfac[i] = expf(kappa * logf(fmaxf(mean / gden, eps)));
    } else if (g.ntrail == 1 && i < g.rows + g.cols) {
        const int64_t c = i - g.rows;
        const float mean = (float)((double)colfx[c] / g.hs_col / (double)g.rows);
        colfac[c] = expf(kappa * logf(fmaxf(mean / gden, eps)));
    }
}

// ndim >= 3: axis terms of the column group by summing the column sums that
// share a coordinate (fixed order), then the per-column factor.
__global__ __launch_bounds__(SP_FIN_NT) void marg_axes_kernel(Geom g, const unsigned long long* __restrict__ colfx,
                                                              float* __restrict__ terms, float* __restrict__ colfac,
                                                              const Ctrl* __restrict__ ctrl, float eps) {
    const float gden = ctrl->gden, kappa = ctrl->kappa;
    const double n = (double)g.n;
    int64_t off = 0;
    for (int a = 0; a < g.ntrail; ++a) {
        int64_t inner = 1;
        for (int b = a + 1; b < g.ntrail; ++b) inner *= g.tdim[b];
        const int64_t dim = g.tdim[a];
        const int64_t outer = g.cols / (dim * inner);
        for (int64_t k = threadIdx.x; k < dim; k += SP_FIN_NT) {
            double s = 0.0;
            for (int64_t o = 0; o < outer; ++o)
                for (int64_t in = 0; in < inner; ++in) s += (double)colfx[(o * dim + k) * inner + in];
            const float mean = (float)(s / g.hs_col / (n / (double)dim));
            terms[off + k] = kappa * logf(fmaxf(mean / gden, eps));
        }
        off += dim;
    }
    __syncthreads();
    for (int64_t c = threadIdx.x; c < g.cols; c += SP_FIN_NT) {
        float ls = 0.f;
        int64_t rem = c, o2 = 0;
        int64_t coord[8];
        for (int a = g.ntrail - 1; a >= 0; --a) {
            coord[a] = rem % g.tdim[a];
            rem /= g.tdim[a];
        }
        for (int a = 0; a < g.ntrail; ++a) {
            ls += terms[o2 + coord[a]];
            o2 += g.tdim[a];
        }
        colfac[c] = expf(ls);
    }
}

// ---------------------------------------------------------------------------
// S3: tangent force, prediction error, port projection / histograms, echo
// ---------------------------------------------------------------------------
template <int RM, int KM, typename PT, typename GT>
__global__ __launch_bounds__(SP_NT) void sweep3_kernel(Geom g, const GT* __restrict__ grad, const PT* __restrict__ param,
                                                       const float* __restrict__ rowtab, const float* __restrict__ coltab,
                                                       const ModeMeta* __restrict__ meta,
                                                       const unsigned char* __restrict__ bins, const Ctrl* __restrict__ ctrl,
                                                       const float* __restrict__ lt, const float* __restrict__ alpha,
                                                       const float* __restrict__ rowfac, const float* __restrict__ colfac,
                                                       float* __restrict__ tbuf, double* __restrict__ part,
                                                       unsigned long long* __restrict__ hist, int hash_on, int echo_on,
                                                       cresso_hyper h) {
    extern __shared__ __align__(16) unsigned char dyn[];
    __shared__ float red[4 * NV3];
    const Tile t = tile_of(g);
    const int TB = g.T * g.B;
    unsigned long long* s_hist = reinterpret_cast<unsigned long long*>(dyn);
    float* s_lt = reinterpret_cast<float*>(dyn + sizeof(unsigned long long) * (size_t)TB);
    if (hash_on)
        for (int i = threadIdx.x; i < TB; i += SP_NT) {
            s_hist[i] = 0ull;
            s_lt[i] = lt[i];
        }
    __syncthreads();
    float b[KM];
    load_cols<KM>(g, coltab, t, b);
    const float eps = (float)h.eps;
    const float inv_s = ctrl->inv_s, scale = ctrl->scale;
    const float mcoup = (float)h.metric_coupling;
    const float wd = (float)h.weight_decay;
    const bool wd_on = h.weight_decay != 0.0;
    const float sg = h.maximize ? -1.f : 1.f;
    const bool ls_on = h.local_sharpness != 0.0;
    const float ls = (float)h.local_sharpness;
    const float kappa = ctrl->kappa, gden = ctrl->gden;
    const bool inst_on = kappa != 0.0f;
    const float ipw = (float)fmax(h.instant_metric_power, 0.25);
    const float ec = inst_on && !g.one_d && t.colok ? colfac[t.col] : 1.0f;
    const float invT = 1.0f / (float)g.T;
    const float tm = (float)h.transport_mix;
    const float hs = (float)ctrl->hs_P;
    const float clip = (float)h.drive_clip, iclip = 1.0f / clip, clip2 = clip * clip;
    const float* __restrict__ alM = alpha;
    const float* __restrict__ alP = alpha + (size_t)g.rows * g.KA;
    float ZP1[RM], ZP2[RM], ZT1[RM], ZT2[RM];
#pragma unroll
    for (int r = 0; r < RM; ++r) ZP1[r] = ZP2[r] = ZT1[r] = ZT2[r] = 0.f;
    float m_ee = 0.f, m_P = 0.f, m_t = 0.f, m_tt = 0.f, m_rr = 0.f, m_bb = 0.f, m_oo = 0.f, m_rb = 0.f, m_ro = 0.f,
          m_bo = 0.f, m_tr = 0.f, m_tb = 0.f, m_to = 0.f;
    if (t.colok) {
        for (int64_t i = t.r0; i < t.r1; ++i) {
            const int64_t e = i * g.cols + t.col;
            float f = sg * ld(grad, e);
            if (wd_on) f = f + wd * ld(param, e);
            // metric field exp(c * clamp(recon(metric), +-3)) clamped (cresso_v5.py:1090-1093)
            const float lm = clampf(recon<KM>(alM + i * g.KA, b), -3.0f, 3.0f);
            const float M = clampf(fexp(mcoup * lm), 0.06f, 16.0f);
            float den = scale * M;
            if (ls_on) {
                const float rel = fminf(fabsf(f) * inv_s + eps, 1.0e4f);
                den = den * clampf(1.0f + ls * fsqrt(fminf(rel, 100.0f)), 1.0f, 8.0f);
            }
            if (inst_on) {
                float I;
                if (g.one_d) {
                    const float rel = fmaxf(fminf(fabsf(f) * inv_s + eps, 1.0e4f), eps);
                    const float dens = fminf(ipw == 1.0f ? rel : fpow(rel, ipw), 1.0e6f);
                    I = fexp(kappa * flog(fmaxf(dens / gden, eps)));
                } else {
                    I = rowfac[i] * ec;
                }
                den = den * clampf(I, 0.08f, 12.0f);
            }
            uint64_t pk = 0;
            if (hash_on) {
                pk = load_bins(bins, e, g.binbytes);
                float ls_ = 0.f;
                for (int tt = 0; tt < g.T; ++tt) ls_ += s_lt[tt * g.B + bin_of(pk, tt, g.bpb)];
                den = den * clampf(fexp(ls_ * invT), 0.08f, 12.0f);
            }
            const float tv = clampf(f * frcp(den + eps), -1.0e4f, 1.0e4f);
            tbuf[e] = tv;
            const float pred = recon<KM>(alP + i * g.KA, b);
            const float err = tv - pred;
            const float P = err + tm * tv;
            m_ee += err * err;
            m_P += P;
            m_t += tv;
            m_tt += tv * tv;
            float rat, bnd, root;
            shape3f(tv, iclip, clip, clip2, eps, rat, bnd, root);
            m_rr += rat * rat; m_bb += bnd * bnd; m_oo += root * root;
            m_rb += rat * bnd; m_ro += rat * root; m_bo += bnd * root;
            m_tr += tv * rat; m_tb += tv * bnd; m_to += tv * root;
            const float* __restrict__ ar = rowtab + i * g.RW;
#pragma unroll
            for (int q = 0; q < RM; ++q) {
                ZP1[q] += ar[2 * q] * P;
                ZP2[q] += ar[2 * q + 1] * P;
            }
            if (echo_on) {
#pragma unroll
                for (int q = 0; q < RM; ++q) {
                    ZT1[q] += ar[2 * q] * tv;
                    ZT2[q] += ar[2 * q + 1] * tv;
                }
            }
            if (hash_on) {
                const unsigned long long v = to_fixed_s(P * hs);
                for (int tt = 0; tt < g.T; ++tt) atomicAdd(&s_hist[tt * g.B + bin_of(pk, tt, g.bpb)], v);
            }
        }
    }
    __syncthreads();
    if (hash_on)
        for (int i = threadIdx.x; i < TB; i += SP_NT)
            if (s_hist[i]) atomicAdd(&hist[i], s_hist[i]);
    Partials P{red, 15 + 4 * g.R};
    const float mm[13] = {m_ee, m_P, m_t, m_tt, m_rr, m_bb, m_oo, m_rb, m_ro, m_bo, m_tr, m_tb, m_to};
#pragma unroll
    for (int k = 0; k < 13; ++k) P.add(k, mm[k]);
    P.add(13, 0.f);
    P.add(14, 0.f);
    proj_finish<RM, KM>(g, meta, ZP1, ZP2, b, P, 15);
    proj_finish<RM, KM>(g, meta, ZT1, ZT2, b, P, 15 + 2 * g.R);
    P.flush(part, g.nblk);
}

// ---------------------------------------------------------------------------
// F3: surprise, hash impulse, confidence, contact, core coefficients
// ---------------------------------------------------------------------------
__device__ void contact_bank(float* q, float* p, const float* port, const float* omega, float* calcium, float& action,
                             float S, int R, const cresso_hyper& h) {
    // cresso_v5.py:914-943
    const float dt = (float)h.dt;
    const float rd = (float)h.refractory_decay;
    const float plast = 1.0f + (float)h.surprise_gain * S / (1.0f + S);
    const float brake = 1.0f / (1.0f + (float)h.surprise_brake * S);
    float gp[SP_MAXR];
    double e1 = 0.0, e2 = 0.0, pw = 0.0;
    for (int r = 0; r < R; ++r) {
        calcium[r] = calcium[r] * rd + (float)(1.0 - h.refractory_decay) * fabsf(port[r]);
        const float gate = 1.0f / (1.0f + (float)h.refractory_gain * calcium[r]);
        gp[r] = port[r] * gate * plast * brake;
        e1 += (double)(p[r] * p[r]);
        const float oq = omega[r] * q[r];
        e2 += (double)(oq * oq);
        pw += (double)(gp[r] * p[r]);
    }
    if (R > 0) {
        const float energy = 0.5f * ((float)(e1 / R) + (float)(e2 / R));
        const float power = (float)(pw / R);
        action = action * 0.985f + dt * (power - energy);
    }
    const float fric = (float)h.impulse_friction + (float)h.contact_gain * tanhf(fabsf(action));
    const float damp = fmaxf(1.0f - dt * fric, 0.0f);
    for (int r = 0; r < R; ++r) {
        float pr = p[r] * damp;
        const float qq = q[r];
        pr = pr + dt * (gp[r] - (float)h.restoring * (omega[r] * omega[r]) * qq - (float)h.cubic * (qq * qq * qq));
        p[r] = pr;
        q[r] = clampf(qq + dt * pr, -8.0f, 8.0f);
    }
}

__global__ __launch_bounds__(SP_FIN_NT) void fin3_kernel(Geom g, const ModeMeta* __restrict__ meta,
                                                         const double* __restrict__ stats, const float* __restrict__ rowtab,
                                                         const double* __restrict__ part,
                                                         unsigned long long* __restrict__ hist,
                                                         const unsigned long long* __restrict__ counts,
                                                         float* __restrict__ imp_tab, float* __restrict__ alpha,
                                                         SpecState st, Ctrl* __restrict__ ctrl, int step, int hash_on,
                                                         int hard, int echo_on, cresso_hyper h,
                                                         double* __restrict__ moments) {
    __shared__ double s_m[NV3];
    const int tid = threadIdx.x;
    const double n = (double)g.n;
    reduce_all(part, g.nblk, 15 + 4 * g.R, s_m);
    const float eps = (float)h.eps;
    // hash refractory / impulse (cresso_v5.py:1140-1184)
    if (hash_on) {
        const int TB = g.T * g.B;
        for (int i = tid; i < TB; i += SP_FIN_NT) {
            const double cnt = fmax((double)counts[i], 1.0);
            const float cp = (float)((double)(long long)hist[i] / ctrl->hs_P / cnt);
            hist[i] = 0ull;
            const float ref = st.hash_refractory[i] * (float)h.hash_decay + (float)(1.0 - h.hash_decay) * fabsf(cp);
            const float gate = 1.0f / (1.0f + (float)h.refractory_gain * ref);
            const float im = st.hash_impulse[i] * (float)h.hash_impulse_decay + (float)(1.0 - h.hash_impulse_decay) * (cp * gate);
            st.hash_refractory[i] = ref;
            st.hash_impulse[i] = im;
            imp_tab[i] = im;
        }
    }
    __shared__ double s_st[SP_MAXR][4];
    __shared__ float s_f[SP_MAXR][9];
    __shared__ float s_sc[2];
    if (tid < g.R) {
        const int r = tid;
        for (int j = 0; j < 4; ++j) s_st[r][j] = stats[4 * r + j];
        s_f[r][0] = st.omega[r];
        s_f[r][1] = st.q_cos[r];
        s_f[r][2] = st.q_sin[r];
        s_f[r][3] = st.p_cos[r];
        s_f[r][4] = st.p_sin[r];
        s_f[r][5] = st.calcium_cos[r];
        s_f[r][6] = st.calcium_sin[r];
        s_f[r][7] = st.conf[r];
    }
    if (tid == 0) {
        s_sc[0] = *st.surprise;
        s_sc[1] = *st.action;
    }
    __syncthreads();
    if (tid == 0) {
        const double sP = s_m[1], sT = s_m[2];
        // surprise reservoir (cresso_v5.py:1127-1129)
        const float sur = reservoir_f(s_sc[0], sqrtf((float)(s_m[0] / n) + eps), h.surprise_decay, step);
        s_sc[0] = sur;
        double stt[4 * SP_MAXR];
        for (int r = 0; r < g.R; ++r)
            for (int j = 0; j < 4; ++j) stt[4 * r + j] = s_st[r][j];
        // port and echo projections -> mean(x Cn)
        float pc[SP_MAXR], ps[SP_MAXR], ecs[SP_MAXR], ess[SP_MAXR];
        for (int r = 0; r < g.R; ++r) {
            const double mc = s_st[r][0], ic = s_st[r][1], ms = s_st[r][2], is = s_st[r][3];
            pc[r] = (float)((s_m[15 + 2 * r] - mc * sP) * ic / n);
            ps[r] = (float)((s_m[16 + 2 * r] - ms * sP) * is / n);
            ecs[r] = (float)((s_m[15 + 2 * g.R + 2 * r] - mc * sT) * ic / n);
            ess[r] = (float)((s_m[16 + 2 * g.R + 2 * r] - ms * sT) * is / n);
        }
        float om[SP_MAXR], qc[SP_MAXR], qs[SP_MAXR], pcv[SP_MAXR], psv[SP_MAXR], cac[SP_MAXR], cas[SP_MAXR];
        for (int r = 0; r < g.R; ++r) {
            om[r] = s_f[r][0]; qc[r] = s_f[r][1]; qs[r] = s_f[r][2]; pcv[r] = s_f[r][3]; psv[r] = s_f[r][4];
            cac[r] = s_f[r][5]; cas[r] = s_f[r][6];
        }
        // confidence (cresso_v5.py:1199-1202) with the pre-contact q
        const float cd = (float)h.confidence_decay;
        float gt[SP_MAXR];
        for (int r = 0; r < g.R; ++r) {
            const float pe = sqrtf(pc[r] * pc[r] + ps[r] * ps[r] + eps);
            const float sup = (pc[r] * qc[r] + ps[r] * qs[r]) / (pe * sqrtf(qc[r] * qc[r] + qs[r] * qs[r] + eps) + eps);
            const float c = s_f[r][7] * cd + (float)(1.0 - h.confidence_decay) * clampf(sup, -1.0f, 1.0f);
            s_f[r][7] = clampf(c, -4.0f, 4.0f);
            gt[r] = sigmoidf_((float)h.confidence_gain * s_f[r][7]);
        }
        // contact on the cos bank then the sin bank with the shared action
        float action = s_sc[1];
        contact_bank(qc, pcv, pc, om, cac, action, sur, g.R, h);
        contact_bank(qs, psv, ps, om, cas, action, sur, g.R, h);
        s_sc[1] = action;
        for (int r = 0; r < g.R; ++r) {
            s_f[r][1] = qc[r]; s_f[r][2] = qs[r]; s_f[r][3] = pcv[r]; s_f[r][4] = psv[r];
            s_f[r][5] = cac[r]; s_f[r][6] = cas[r];
        }
        set_recon(g, stt, ctrl->rc[2], ctrl->rconst[2], qc, qs, gt);
        if (echo_on) set_recon(g, stt, ctrl->rc[3], ctrl->rconst[3], ecs, ess, nullptr);
        // drive shaping coefficients that depend only on moments of t
        // (cresso_v5.py:1303-1337): shaped = ar rat + ab bnd + ao root,
        // core = (1-dmix) shaped + dmix t srms/max(frms,eps)
        const double Stt = s_m[3], Srr = s_m[4], Sbb = s_m[5], Soo = s_m[6], Srb = s_m[7], Sro = s_m[8], Sbo = s_m[9];
        const float S = sur;
        const float frms = sqrtf((float)(Stt / n) + eps);
        const float rms_rat = sqrtf((float)(Srr / n) + eps);
        const float rms_root = sqrtf((float)(Soo / n) + eps);
        const float kroot = rms_rat / fmaxf(rms_root, eps);
        const float spike = (float)h.spike_mix / (1.0f + S);
        const float rmix = (hard ? (float)h.root_channel_mix : 0.0f) / (1.0f + 0.5f * S);
        const double ar = (double)((1.0f - rmix) * (1.0f - spike));
        const double ab = (double)((1.0f - rmix) * spike);
        const double ao = (double)(rmix * kroot);
        const double sh2 = ar * ar * Srr + ab * ab * Sbb + ao * ao * Soo + 2.0 * (ar * ab * Srb + ar * ao * Sro + ab * ao * Sbo);
        const float srms = sqrtf((float)(sh2 / n) + eps);
        const float dmix = (float)h.direct_force_mix / (1.0f + 0.35f * S);
        const float kdir = srms / fmaxf(frms, eps);
        ctrl->cr = (float)((1.0 - (double)dmix) * ar);
        ctrl->cb = (float)((1.0 - (double)dmix) * ab);
        ctrl->co = (float)((1.0 - (double)dmix) * ao);
        ctrl->ct = dmix * kdir;
        ctrl->nscale = 1.0f / ((float)h.drive_clip * (1.0f + S));
        moments[0] = Stt;
        moments[1] = (double)srms;
        moments[2] = (double)frms;
    }
    __syncthreads();
    if (tid < g.R) {
        const int r = tid;
        st.q_cos[r] = s_f[r][1];
        st.q_sin[r] = s_f[r][2];
        st.p_cos[r] = s_f[r][3];
        st.p_sin[r] = s_f[r][4];
        st.calcium_cos[r] = s_f[r][5];
        st.calcium_sin[r] = s_f[r][6];
        st.conf[r] = s_f[r][7];
    }
    if (tid == 0) {
        *st.surprise = s_sc[0];
        *st.action = s_sc[1];
    }
}

// ---------------------------------------------------------------------------
// S4: cross moments for the drive energy
// ---------------------------------------------------------------------------
// Y = {core, pred', nov, err', echo, hash}; sums of Y_a Y_b (a <= b) and t*pred'
__device__ __forceinline__ int pair_index(int a, int b) {  // a <= b < 6
    return a * 6 - (a * (a - 1)) / 2 + (b - a);
}

template <int RM, int KM>
__global__ __launch_bounds__(SP_NT) void sweep4_kernel(Geom g, const float* __restrict__ coltab,
                                                       const unsigned char* __restrict__ bins, const Ctrl* __restrict__ ctrl,
                                                       const float* __restrict__ imp_tab, const float* __restrict__ alpha,
                                                       const float* __restrict__ tbuf, double* __restrict__ part,
                                                       int hash_on, int echo_on, cresso_hyper h) {
    extern __shared__ __align__(16) unsigned char dyn[];
    __shared__ float red[4 * NV4];
    const Tile t = tile_of(g);
    const int TB = g.T * g.B;
    float* s_imp = reinterpret_cast<float*>(dyn);
    if (hash_on)
        for (int i = threadIdx.x; i < TB; i += SP_NT) s_imp[i] = imp_tab[i];
    __syncthreads();
    float b[KM];
    load_cols<KM>(g, coltab, t, b);
    const float eps = (float)h.eps;
    const float clip = (float)h.drive_clip, iclip = 1.0f / clip, clip2 = clip * clip;
    const float cr = ctrl->cr, cb = ctrl->cb, co = ctrl->co, ct = ctrl->ct, ns = ctrl->nscale;
    const float invT = 1.0f / (float)g.T;
    const float* __restrict__ alQ = alpha + 2 * (size_t)g.rows * g.KA;
    const float* __restrict__ alE = alQ + (size_t)g.rows * g.KA;
    float m[NV4];
#pragma unroll
    for (int k = 0; k < NV4; ++k) m[k] = 0.f;
    if (t.colok) {
        for (int64_t i = t.r0; i < t.r1; ++i) {
            const int64_t e = i * g.cols + t.col;
            const float tv = tbuf[e];
            const float pred = recon<KM>(alQ + i * g.KA, b);
            const float err = tv - pred;
            const float nov = ftanh(err * ns) * clip;
            const float echo = echo_on ? recon<KM>(alE + i * g.KA, b) : 0.f;
            float hp = 0.f;
            if (hash_on) {
                const uint64_t pk = load_bins(bins, e, g.binbytes);
                for (int tt = 0; tt < g.T; ++tt) hp += s_imp[tt * g.B + bin_of(pk, tt, g.bpb)];
                hp = hp * invT;
            }
            float rat, bnd, root;
            shape3f(tv, iclip, clip, clip2, eps, rat, bnd, root);
            const float core = cr * rat + cb * bnd + co * root + ct * tv;
            const float Y[6] = {core, pred, nov, err, echo, hp};
#pragma unroll
            for (int a = 0; a < 6; ++a)
#pragma unroll
                for (int c = a; c < 6; ++c) m[pair_index(a, c)] += Y[a] * Y[c];
            m[21] += tv * pred;
        }
    }
    Partials P{red, NV4};
#pragma unroll
    for (int k = 0; k < NV4; ++k) P.add(k, m[k]);
    P.flush(part, g.nblk);
}

__global__ __launch_bounds__(SP_FIN_NT) void fin4_kernel(Geom g, const double* __restrict__ part, SpecState st,
                                                         Ctrl* __restrict__ ctrl, int step, int hash_on, int hard,
                                                         int echo_on, cresso_hyper h, const double* __restrict__ moments) {
    __shared__ double s_m[NV4];
    reduce_all(part, g.nblk, NV4, s_m);
    if (threadIdx.x != 0) return;
    const double n = (double)g.n;
    const float eps = (float)h.eps;
    auto G = [&](int a, int b) { return a <= b ? s_m[pair_index(a, b)] : s_m[pair_index(b, a)]; };
    const float S = *st.surprise;
    const float frms = (float)moments[2];
    const float srms = (float)moments[1];
    // alignment gate and prediction mix (cresso_v5.py:1303-1313)
    const float prms = sqrtf((float)(G(1, 1) / n) + eps);
    const float align = clampf((float)(s_m[21] / n) / (frms * prms + eps), -1.0f, 1.0f);
    float agate = clampf((align + 1.0f) * 0.5f, 0.0f, 1.0f);
    if (!(prms > (float)sqrt(h.eps))) agate = 0.0f;
    const double warm = h.warmup_steps == 0 ? 1.0 : 1.0 - exp(-(double)step / (double)(h.warmup_steps > 1 ? h.warmup_steps : 1));
    const float mix = (float)(h.prediction_mix * warm) * agate * (1.0f / (1.0f + S));
    const float crms = sqrtf((float)(G(0, 0) / n) + eps);
    const float erms = sqrtf((float)(G(3, 3) / n) + eps);
    const float kres = crms / fmaxf(erms, eps);
    const float resmix = (float)h.residual_feedback_mix / (1.0f + S);
    float kecho = 0.f, khp = 0.f;
    if (hard && echo_on) kecho = srms / fmaxf(sqrtf((float)(G(4, 4) / n) + eps), eps);
    if (hard && hash_on) khp = srms / fmaxf(sqrtf((float)(G(5, 5) / n) + eps), eps);
    double c[6];
    c[0] = 1.0 - (double)mix;
    c[1] = mix;
    c[2] = h.novelty_mix;
    c[3] = (double)(resmix * kres);
    c[4] = hard ? h.echo_mix * (double)kecho : 0.0;
    c[5] = hard ? h.hash_drive_mix * (double)khp : 0.0;
    double dd = 0.0;
    for (int a = 0; a < 6; ++a)
        for (int b = 0; b < 6; ++b) dd += c[a] * c[b] * G(a, b);
    const float de_now = (float)(fmax(dd, 0.0) / n);
    const float de = reservoir_f(*st.drive_energy, de_now, h.reservoir_decay, step);
    *st.drive_energy = de;
    const float gain = clampf((float)h.target_update_rms / sqrtf(de + eps), (float)h.min_gain, (float)h.max_gain);
    ctrl->dcore = (float)c[0];
    ctrl->dpred = (float)c[1];
    ctrl->dnov = (float)c[2];
    ctrl->derr = (float)c[3];
    ctrl->decho = (float)c[4];
    ctrl->dhp = (float)c[5];
    ctrl->gain = gain;
}

// ---------------------------------------------------------------------------
// S5: parameter update
// ---------------------------------------------------------------------------
template <int RM, int KM, typename PT>
__global__ __launch_bounds__(SP_NT) void sweep5_kernel(Geom g, PT* __restrict__ param, const float* __restrict__ coltab,
                                                       const unsigned char* __restrict__ bins, const Ctrl* __restrict__ ctrl,
                                                       const float* __restrict__ imp_tab, const float* __restrict__ alpha,
                                                       const float* __restrict__ tbuf, int hash_on, int echo_on,
                                                       cresso_hyper h) {
    extern __shared__ __align__(16) unsigned char dyn[];
    const Tile t = tile_of(g);
    const int TB = g.T * g.B;
    float* s_imp = reinterpret_cast<float*>(dyn);
    if (hash_on)
        for (int i = threadIdx.x; i < TB; i += SP_NT) s_imp[i] = imp_tab[i];
    __syncthreads();
    if (!t.colok) return;
    float b[KM];
    load_cols<KM>(g, coltab, t, b);
    const float eps = (float)h.eps;
    const float clip = (float)h.drive_clip, iclip = 1.0f / clip, clip2 = clip * clip;
    const float cr = ctrl->cr, cb = ctrl->cb, co = ctrl->co, ct = ctrl->ct, ns = ctrl->nscale;
    const float d0 = ctrl->dcore, d1 = ctrl->dpred, d2 = ctrl->dnov, d3 = ctrl->derr, d4 = ctrl->decho, d5 = ctrl->dhp;
    const float gain = ctrl->gain;
    const float nlr = (float)(-h.lr);
    const float invT = 1.0f / (float)g.T;
    const float* __restrict__ alQ = alpha + 2 * (size_t)g.rows * g.KA;
    const float* __restrict__ alE = alQ + (size_t)g.rows * g.KA;
    for (int64_t i = t.r0; i < t.r1; ++i) {
        const int64_t e = i * g.cols + t.col;
        const float tv = tbuf[e];
        const float pred = recon<KM>(alQ + i * g.KA, b);
        const float err = tv - pred;
        const float nov = ftanh(err * ns) * clip;
        float drive = d1 * pred + d2 * nov + d3 * err;
        if (echo_on) drive += d4 * recon<KM>(alE + i * g.KA, b);
        if (hash_on) {
            const uint64_t pk = load_bins(bins, e, g.binbytes);
            float hp = 0.f;
            for (int tt = 0; tt < g.T; ++tt) hp += s_imp[tt * g.B + bin_of(pk, tt, g.bpb)];
            drive += d5 * (hp * invT);
        }
        float rat, bnd, root;
        shape3f(tv, iclip, clip, clip2, eps, rat, bnd, root);
        const float core = cr * rat + cb * bnd + co * root + ct * tv;
        drive += d0 * core;
        const float u = to_f(from_w<PT>(drive * gain));
        param[e] = from_w<PT>(to_f(param[e]) + nlr * u);
    }
}

// ---------------------------------------------------------------------------
// host-side planning
// ---------------------------------------------------------------------------
double hash_unit_host(int64_t n, int64_t salt) {
    // cresso_v5.py:127-135 on unbounded integers (first product unmasked)
    unsigned __int128 x = (unsigned __int128)(n + 1) * 0x9E3779B1ull + (unsigned __int128)(salt + 11) * 0x85EBCA77ull;
    x ^= (x >> 16);
    uint64_t y = (uint64_t)((x * 0x7FEB352Dull) & 0xFFFFFFFFull);
    y ^= (y >> 15);
    y = (y * 0x846CA68Bull) & 0xFFFFFFFFull;
    y ^= (y >> 16);
    return (double)(y & 0xFFFFFF) / (double)(1 << 24);
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
};

namespace cresso {
namespace {

size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

int32_t plan_spectral(const int64_t* shape, int32_t ndim, const int64_t* freqs, int32_t rank, int32_t bins,
                      int32_t tables, cresso_spectral_plan& P) {
    if (ndim < 1 || ndim > 8) return fail(CRESSO_E_INVALID, "spectral route: ndim %d outside 1..8", ndim);
    if (rank < 1 || rank > SP_MAXR)
        return fail(CRESSO_E_UNSUPPORTED, "spectral route: rank %d outside 1..%d supported by this build", rank, SP_MAXR);
    if (bins < 0 || tables < 1 || tables > SP_MAXT)
        return fail(CRESSO_E_UNSUPPORTED, "spectral route: hash_tables %d outside 1..%d", tables, SP_MAXT);
    if (bins > 65535) return fail(CRESSO_E_UNSUPPORTED, "spectral route: hash_bins %d above 65535", bins);
    Geom& g = P.g;
    std::memset(&g, 0, sizeof(g));
    int64_t n = 1;
    for (int a = 0; a < ndim; ++a) {
        if (shape[a] <= 0) return fail(CRESSO_E_INVALID, "spectral route: shape[%d] must be positive", a);
        n *= shape[a];
        P.shape[a] = shape[a];
    }
    g.n = n;
    g.ndim = ndim;
    g.one_d = ndim == 1;
    g.rows = g.one_d ? 1 : shape[0];
    g.cols = n / g.rows;
    g.ntrail = g.one_d ? 1 : ndim - 1;
    for (int a = 0; a < g.ntrail; ++a) g.tdim[a] = shape[a + (g.one_d ? 0 : 1)];
    g.R = rank;
    g.T = bins > 0 ? tables : 1;
    g.B = bins > 0 ? bins : 1;
    P.bins_off = bins > 0 ? 0 : 1;
    g.bpb = g.B <= 256 ? 1 : 2;
    int bb = g.T * g.bpb;
    g.binbytes = bb <= 1 ? 1 : (bb <= 2 ? 2 : (bb <= 4 ? 4 : 8));
    if (bb > 8) return fail(CRESSO_E_UNSUPPORTED, "spectral route: %d tables x %d-byte bins exceed 8 bytes", g.T, g.bpb);
    P.freqs.assign(freqs, freqs + (size_t)rank * ndim);
    // per (mode, axis) fp32 constants, cast from double as torch casts Python scalars
    P.axc.assign((size_t)rank * ndim, AxisConst{});
    P.meta.assign((size_t)rank, ModeMeta{});
    for (int r = 0; r < rank; ++r) {
        int64_t fs = 0;
        for (int a = 0; a < ndim; ++a) fs += std::llabs(freqs[(size_t)r * ndim + a]);
        const int kind = r % 4;
        P.meta[r].kind = kind;
        P.meta[r].type = fs == 0 ? M_ZERO : (kind == 1 ? M_PROD : M_ADD);
        for (int a = 0; a < ndim; ++a) {
            AxisConst& c = P.axc[(size_t)r * ndim + a];
            const int64_t f = freqs[(size_t)r * ndim + a];
            c.f = (int32_t)f;
            c.pf = (float)(M_PI * (double)f);
            const double ch = 0.25 + 1.75 * hash_unit_host(r, 17 + a);
            c.pc = (float)(M_PI * ch * (double)std::max<int64_t>(1, f));
            c.mu = (float)(0.15 + 0.70 * hash_unit_host(r, 101 + a));
            c.sig = (float)(0.18 + 0.20 * hash_unit_host(r, 151 + a));
        }
    }
    // distinct column carriers: k = 0 is the constant 1; a mode's column pair
    // is identified symbolically by its column-group parameters
    P.csrc.clear();
    P.csrc.push_back(CarrierSrc{-1, 0});
    std::map<std::vector<int64_t>, int> seen;
    const int fa = g.one_d ? 0 : 1;
    for (int r = 0; r < rank; ++r) {
        ModeMeta& m = P.meta[r];
        if (m.type == M_ZERO) {
            m.k1 = 0;
            m.k2 = -1;
            continue;
        }
        bool active = false;
        std::vector<int64_t> key = {(int64_t)m.kind};
        for (int a = fa; a < ndim; ++a) {
            const AxisConst& c = P.axc[(size_t)r * ndim + a];
            key.push_back(c.f);
            if (c.f != 0) active = true;
            if (m.kind >= 2) {
                int32_t bits;
                std::memcpy(&bits, &c.pc, 4); key.push_back(bits);
                if (m.kind == 3) {
                    std::memcpy(&bits, &c.mu, 4); key.push_back(bits);
                    std::memcpy(&bits, &c.sig, 4); key.push_back(bits);
                }
            }
        }
        if (m.kind == 0 && !active) {  // phase 0 on the column group: b1 = 1, b2 = 0
            m.k1 = 0;
            m.k2 = -1;
            continue;
        }
        if (m.kind == 1 && !active) {  // empty products: b1 = b2 = 1
            m.k1 = 0;
            m.k2 = 0;
            continue;
        }
        auto it = seen.find(key);
        if (it != seen.end()) {
            m.k1 = it->second;
            m.k2 = it->second + 1;
            continue;
        }
        const int k = (int)P.csrc.size();
        P.csrc.push_back(CarrierSrc{r, 0});
        P.csrc.push_back(CarrierSrc{r, 1});
        seen[key] = k;
        m.k1 = k;
        m.k2 = k + 1;
    }
    g.K = (int32_t)P.csrc.size();
    P.rmax = rank <= 8 ? 8 : 16;
    const int KM = 2 * P.rmax + 1;
    if (g.K > KM) return fail(CRESSO_E_INVALID, "spectral route: %d column carriers exceed %d", g.K, KM);
    if ((double)g.K * (double)g.cols * 4.0 > 2.0e9)
        return fail(CRESSO_E_UNSUPPORTED, "spectral route: column carrier table too large (%d x %lld)", g.K, (long long)g.cols);
    g.KA = 2 * P.rmax + 2;
    g.RW = 2 * P.rmax;
    // tiling: 256 columns per block, PR rows per block, ~1024 blocks
    g.slabs = (int32_t)((g.cols + SP_NT - 1) / SP_NT);
    int64_t pr = std::max<int64_t>(16, (g.rows * g.slabs) / 1024);
    pr = std::min<int64_t>(std::min<int64_t>(pr, 64), g.rows);
    g.PR = (int32_t)std::max<int64_t>(1, pr);
    g.panels = (int32_t)((g.rows + g.PR - 1) / g.PR);
    g.nblk = g.slabs * g.panels;
    // flat force-RMS sweep: contiguous chunks (multiple of 4 elements) per block
    g.nblk1 = (int32_t)std::max<int64_t>(1, std::min<int64_t>(1024, (g.n + 16383) / 16384));
    g.chunk1 = (((g.n + g.nblk1 - 1) / g.nblk1) + 3) & ~(int64_t)3;
    g.nblk1 = (int32_t)((g.n + g.chunk1 - 1) / g.chunk1);
    // axis density sums: density <= 1e6 per element, sums below 2^62
    g.hs_row = ldexp(1.0, (int)std::floor(62.0 - std::log2(1.0e6 * (double)g.cols)));
    g.hs_col = ldexp(1.0, (int)std::floor(62.0 - std::log2(1.0e6 * (double)g.rows)));
    // workspace layout
    Offs& o = P.o;
    size_t off = 0;
    auto take = [&](size_t bytes) { size_t at = off; off = al256(off + bytes); return at; };
    o.axc = take(sizeof(AxisConst) * P.axc.size());
    o.meta = take(sizeof(ModeMeta) * P.meta.size());
    o.csrc = take(sizeof(CarrierSrc) * P.csrc.size());
    o.rowtab = take(sizeof(float) * (size_t)g.rows * g.RW);
    o.coltab = take(sizeof(float) * (size_t)g.K * g.cols);
    o.stats = take(sizeof(double) * 4 * g.R);
    o.bounds = take(sizeof(double) * 2 * g.R);
    o.counts = take(sizeof(unsigned long long) * (size_t)g.T * g.B);
    o.bins = take((size_t)g.binbytes * (size_t)g.n);
    o.tbuf = take(sizeof(float) * (size_t)g.n);
    o.part = take(sizeof(double) * (size_t)NVMAX * std::max(g.nblk, g.nblk1));
    o.hist = take(sizeof(unsigned long long) * (size_t)g.T * g.B);
    o.lt = take(sizeof(float) * (size_t)g.T * g.B);
    o.imp = take(sizeof(float) * (size_t)g.T * g.B);
    o.alpha = take(sizeof(float) * 4 * (size_t)g.rows * g.KA);
    o.rowfx = take(sizeof(unsigned long long) * (size_t)g.rows);
    o.colfx = take(sizeof(unsigned long long) * (size_t)g.cols);
    o.rowfac = take(sizeof(float) * (size_t)g.rows);
    o.colfac = take(sizeof(float) * (size_t)g.cols);
    int64_t sum_trail = 0;
    for (int a = 0; a < g.ntrail; ++a) sum_trail += g.tdim[a];
    o.terms = take(sizeof(float) * (size_t)std::max<int64_t>(1, sum_trail));
    o.ctrl = take(sizeof(Ctrl) + 3 * sizeof(double));
    o.total = off;
    return CRESSO_OK;
}

template <typename T> T* at(void* ws, size_t off) { return reinterpret_cast<T*>(reinterpret_cast<char*>(ws) + off); }

size_t lds_sweep2(const Geom& g) { return sizeof(unsigned long long) * g.T * g.B + sizeof(float) * 4 * (size_t)g.PR; }
size_t lds_sweep3(const Geom& g) { return (sizeof(unsigned long long) + sizeof(float)) * g.T * g.B; }
size_t lds_sweep45(const Geom& g) { return sizeof(float) * (size_t)g.T * g.B; }

template <int RM, typename PT, typename GT>
int32_t run_step(const cresso_spectral_plan& P, const cresso_spectral_desc& d, void* ws, const cresso_hyper& h,
                 hipStream_t s) {
    constexpr int KM = 2 * RM + 1;
    const Geom& g = P.g;
    const Offs& o = P.o;
    SpecState st;
    st.force_rms = (float*)d.force_rms; st.drive_energy = (float*)d.drive_energy;
    st.surprise = (float*)d.surprise; st.action = (float*)d.action; st.omega = (const float*)d.omega;
    st.q_cos = (float*)d.q_cos; st.q_sin = (float*)d.q_sin; st.p_cos = (float*)d.p_cos; st.p_sin = (float*)d.p_sin;
    st.metric_cos = (float*)d.metric_cos; st.metric_sin = (float*)d.metric_sin;
    st.metric_p_cos = (float*)d.metric_p_cos; st.metric_p_sin = (float*)d.metric_p_sin;
    st.calcium_cos = (float*)d.calcium_cos; st.calcium_sin = (float*)d.calcium_sin; st.conf = (float*)d.mode_confidence;
    st.hash_energy = (float*)d.hash_energy; st.hash_impulse = (float*)d.hash_impulse;
    st.hash_refractory = (float*)d.hash_refractory;
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
    unsigned long long* hist = at<unsigned long long>(ws, o.hist);
    float* lt = at<float>(ws, o.lt);
    float* imp = at<float>(ws, o.imp);
    float* alpha = at<float>(ws, o.alpha);
    unsigned long long* rowfx = at<unsigned long long>(ws, o.rowfx);
    unsigned long long* colfx = at<unsigned long long>(ws, o.colfx);
    float* rowfac = at<float>(ws, o.rowfac);
    float* colfac = at<float>(ws, o.colfac);
    float* terms = at<float>(ws, o.terms);
    float* tbuf = at<float>(ws, o.tbuf);
    Ctrl* ctrl = at<Ctrl>(ws, o.ctrl);
    double* moments = reinterpret_cast<double*>(ctrl + 1);
    const double* stats = at<double>(ws, o.stats);
    const double* bounds = at<double>(ws, o.bounds);
    const int step = d.step;
    const int axes_on = (hard && h.instant_metric_coupling != 0.0 && !g.one_d) ? 1 : 0;
    const dim3 grid(g.nblk), blk(SP_NT);
    const bool v4 = ((uintptr_t)grad % (4 * sizeof(GT))) == 0 && ((uintptr_t)param % (4 * sizeof(PT))) == 0;
    if (v4)
        hipLaunchKernelGGL((sweep1_kernel<PT, GT, true>), dim3(g.nblk1), blk, 0, s, g, grad, param, part, h);
    else
        hipLaunchKernelGGL((sweep1_kernel<PT, GT, false>), dim3(g.nblk1), blk, 0, s, g, grad, param, part, h);
    hipLaunchKernelGGL(fin1_kernel, dim3(1), dim3(SP_FIN_NT), 0, s, g, part, st, ctrl, rowfx, colfx, step, h);
    hipLaunchKernelGGL((sweep2_kernel<RM, KM, PT, GT>), grid, blk, lds_sweep2(g), s, g, grad, param, rowtab, coltab, meta,
                       bins, ctrl, part, hist, rowfx, colfx, hash_on, axes_on, h);
    hipLaunchKernelGGL(fin2_kernel, dim3(1), dim3(SP_FIN_NT), 0, s, g, meta, stats, bounds, rowtab, part, hist, counts, lt,
                       alpha, st, ctrl, step, hash_on, hard, h);
    const dim3 rgrid((unsigned)((g.rows + 255) / 256)), rblk(256);
    hipLaunchKernelGGL((alpha_kernel<RM>), rgrid, rblk, 0, s, g, meta, rowtab, (const Ctrl*)ctrl, 0, 2, alpha);
    if (axes_on) {
        const int64_t cnt = g.rows + (g.ntrail == 1 ? g.cols : 0);
        hipLaunchKernelGGL(marg_kernel, dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, s, g, rowfx, colfx, rowfac,
                           colfac, ctrl, (float)h.eps);
        if (g.ntrail > 1)
            hipLaunchKernelGGL(marg_axes_kernel, dim3(1), dim3(SP_FIN_NT), 0, s, g, colfx, terms, colfac, ctrl, (float)h.eps);
    }
    hipLaunchKernelGGL((sweep3_kernel<RM, KM, PT, GT>), grid, blk, lds_sweep3(g), s, g, grad, param, rowtab, coltab, meta,
                       bins, ctrl, lt, alpha, rowfac, colfac, tbuf, part, hist, hash_on, echo_on, h);
    hipLaunchKernelGGL(fin3_kernel, dim3(1), dim3(SP_FIN_NT), 0, s, g, meta, stats, rowtab, part, hist, counts, imp, alpha,
                       st, ctrl, step, hash_on, hard, echo_on, h, moments);
    hipLaunchKernelGGL((alpha_kernel<RM>), rgrid, rblk, 0, s, g, meta, rowtab, (const Ctrl*)ctrl, 2, echo_on ? 2 : 1, alpha);
    hipLaunchKernelGGL((sweep4_kernel<RM, KM>), grid, blk, lds_sweep45(g), s, g, coltab, bins, ctrl, imp, alpha, tbuf, part,
                       hash_on, echo_on, h);
    hipLaunchKernelGGL(fin4_kernel, dim3(1), dim3(SP_FIN_NT), 0, s, g, part, st, ctrl, step, hash_on, hard, echo_on, h,
                       (const double*)moments);
    hipLaunchKernelGGL((sweep5_kernel<RM, KM, PT>), grid, blk, lds_sweep45(g), s, g, param, coltab, bins, ctrl, imp, alpha,
                       tbuf, hash_on, echo_on, h);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? CRESSO_OK : hip_fail(e, "spectral route: launch");
}

__global__ void zero_u64_kernel(unsigned long long* p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0ull;
}

}  // namespace
}  // namespace cresso

using namespace cresso;

extern "C" cresso_spectral_plan* cresso_spectral_plan_create(const int64_t* shape, int32_t ndim, const int64_t* freqs,
                                                             int32_t rank, int32_t hash_bins, int32_t hash_tables) {
    if (!shape || !freqs) {
        fail(CRESSO_E_INVALID, "spectral route: null shape or freqs");
        return nullptr;
    }
    cresso_spectral_plan* P = new cresso_spectral_plan();
    if (plan_spectral(shape, ndim, freqs, rank, hash_bins, hash_tables, *P) != CRESSO_OK) {
        delete P;
        return nullptr;
    }
    return P;
}

extern "C" void cresso_spectral_plan_destroy(cresso_spectral_plan* P) { delete P; }

extern "C" size_t cresso_spectral_workspace_bytes(const cresso_spectral_plan* P) { return P ? P->o.total : 0; }

extern "C" int32_t cresso_spectral_workspace_init(const cresso_spectral_plan* P, void* ws, size_t ws_bytes,
                                                  const cresso_hyper* hyper, void* stream) {
    if (!P || !ws || !hyper) return fail(CRESSO_E_INVALID, "spectral route: null argument");
    if (ws_bytes < P->o.total)
        return fail(CRESSO_E_INVALID, "spectral route: workspace of %zu bytes is smaller than %zu", ws_bytes, P->o.total);
    const Geom& g = P->g;
    const Offs& o = P->o;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    hipError_t e = hipMemcpyAsync(at<AxisConst>(ws, o.axc), P->axc.data(), sizeof(AxisConst) * P->axc.size(),
                                  hipMemcpyHostToDevice, s);
    if (e == hipSuccess)
        e = hipMemcpyAsync(at<ModeMeta>(ws, o.meta), P->meta.data(), sizeof(ModeMeta) * P->meta.size(), hipMemcpyHostToDevice, s);
    if (e == hipSuccess)
        e = hipMemcpyAsync(at<CarrierSrc>(ws, o.csrc), P->csrc.data(), sizeof(CarrierSrc) * P->csrc.size(),
                           hipMemcpyHostToDevice, s);
    if (e != hipSuccess) return hip_fail(e, "spectral route: workspace upload");
    const AxisConst* axc = at<AxisConst>(ws, o.axc);
    const ModeMeta* meta = at<ModeMeta>(ws, o.meta);
    hipLaunchKernelGGL(ws_rowtab_kernel, dim3((unsigned)((g.rows + 255) / 256)), dim3(256), 0, s, g, axc, meta,
                       at<float>(ws, o.rowtab));
    hipLaunchKernelGGL(ws_coltab_kernel, dim3((unsigned)((g.cols + 255) / 256)), dim3(256), 0, s, g, axc, meta,
                       at<CarrierSrc>(ws, o.csrc), at<float>(ws, o.coltab));
    hipLaunchKernelGGL(ws_stats_kernel, dim3(1), dim3(SP_FIN_NT), 0, s, g, meta, at<float>(ws, o.rowtab),
                       at<float>(ws, o.coltab), at<double>(ws, o.stats), at<double>(ws, o.bounds));
    const int64_t TB = (int64_t)g.T * g.B;
    hipLaunchKernelGGL(zero_u64_kernel, dim3((unsigned)((TB + 255) / 256)), dim3(256), 0, s, at<unsigned long long>(ws, o.counts), TB);
    hipLaunchKernelGGL(zero_u64_kernel, dim3((unsigned)((TB + 255) / 256)), dim3(256), 0, s, at<unsigned long long>(ws, o.hist), TB);
    const int64_t bins_blocks = std::max<int64_t>(1, std::min<int64_t>(2048, (g.n + 255) / 256));
    hipLaunchKernelGGL(ws_bins_kernel, dim3((unsigned)bins_blocks), dim3(256), 0, s, g, at<unsigned char>(ws, o.bins),
                       at<unsigned long long>(ws, o.counts));
    e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    return e == hipSuccess ? CRESSO_OK : hip_fail(e, "spectral route: workspace init");
}

extern "C" int32_t cresso_spectral_step(const cresso_spectral_plan* P, const cresso_spectral_desc* d, void* ws,
                                        size_t ws_bytes, const cresso_hyper* hyper, void* stream) {
    if (!P || !d || !ws || !hyper) return fail(CRESSO_E_INVALID, "spectral route: null argument");
    if (ws_bytes < P->o.total) return fail(CRESSO_E_INVALID, "spectral route: workspace too small");
    const Geom& g = P->g;
    if (d->numel != g.n) return fail(CRESSO_E_INVALID, "spectral route: numel %lld does not match the plan", (long long)d->numel);
    if (!d->param || !d->grad) return fail(CRESSO_E_INVALID, "spectral route: null param or grad");
    const void* req[] = {d->force_rms, d->drive_energy, d->surprise, d->action, d->omega, d->q_cos, d->q_sin, d->p_cos,
                         d->p_sin, d->metric_cos, d->metric_sin, d->metric_p_cos, d->metric_p_sin, d->calcium_cos,
                         d->calcium_sin, d->mode_confidence};
    for (const void* p : req)
        if (!p) return fail(CRESSO_E_INVALID, "spectral route: null state pointer");
    if (d->hash_energy && (!d->hash_impulse || !d->hash_refractory))
        return fail(CRESSO_E_INVALID, "spectral route: partial hash state");
    if (d->step < 1) return fail(CRESSO_E_INVALID, "spectral route: step must be >= 1 (after the increment)");
    if (!(hyper->drive_clip > 0.0)) return fail(CRESSO_E_INVALID, "spectral route: drive_clip must be positive");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int pt = d->param_dtype, gt = d->grad_dtype;
    const bool r8 = P->rmax == 8;
#define CRESSO_SP_CASE(PC, GC, PTy, GTy)                                                          \
    if (pt == PC && gt == GC)                                                                      \
        return r8 ? run_step<8, PTy, GTy>(*P, *d, ws, *hyper, s) : run_step<16, PTy, GTy>(*P, *d, ws, *hyper, s);
    CRESSO_SP_CASE(CRESSO_F32, CRESSO_F32, float, float)
    CRESSO_SP_CASE(CRESSO_BF16, CRESSO_BF16, __hip_bfloat16, __hip_bfloat16)
    CRESSO_SP_CASE(CRESSO_F16, CRESSO_F16, __half, __half)
#undef CRESSO_SP_CASE
    return fail(CRESSO_E_UNSUPPORTED, "spectral route: param/grad dtype pair (%d,%d) not supported by this build", pt, gt);
}

extern "C" int32_t cresso_spectral_workspace_bins(const cresso_spectral_plan* P, const void* ws, size_t ws_bytes,
                                                  int32_t* bins_out, int64_t* counts_out, void* stream) {
    if (!P || !ws || !bins_out || !counts_out) return fail(CRESSO_E_INVALID, "spectral route: null argument");
    if (ws_bytes < P->o.total) return fail(CRESSO_E_INVALID, "spectral route: workspace too small");
    const Geom& g = P->g;
    if (P->bins_off) return fail(CRESSO_E_INVALID, "spectral route: plan has hash_bins = 0 (no bins)");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(4096, (g.n + 255) / 256));
    hipLaunchKernelGGL(ws_unpack_bins_kernel, dim3((unsigned)blocks), dim3(256), 0, s, g,
                       at<unsigned char>(const_cast<void*>(ws), P->o.bins), bins_out);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess)
        e = hipMemcpyAsync(counts_out, at<unsigned long long>(const_cast<void*>(ws), P->o.counts),
                           sizeof(int64_t) * (size_t)g.T * g.B, hipMemcpyDeviceToDevice, s);
    return e == hipSuccess ? CRESSO_OK : hip_fail(e, "spectral route: workspace bins");
}

extern "C" int32_t cresso_spectral_workspace_basis(const cresso_spectral_plan* P, const void* ws, size_t ws_bytes,
                                                   int32_t mode, float* cos_out, float* sin_out, void* stream) {
    if (!P || !ws || !cos_out || !sin_out) return fail(CRESSO_E_INVALID, "spectral route: null argument");
    if (ws_bytes < P->o.total) return fail(CRESSO_E_INVALID, "spectral route: workspace too small");
    const Geom& g = P->g;
    if (mode < 0 || mode >= g.R) return fail(CRESSO_E_INVALID, "spectral route: mode %d outside 0..%d", mode, g.R - 1);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    void* w = const_cast<void*>(ws);
    const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(4096, (g.n + 255) / 256));
    hipLaunchKernelGGL(ws_basis_kernel, dim3((unsigned)blocks), dim3(256), 0, s, g, at<ModeMeta>(w, P->o.meta),
                       at<float>(w, P->o.rowtab), at<float>(w, P->o.coltab), at<double>(w, P->o.stats), mode, cos_out,
                       sin_out);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? CRESSO_OK : hip_fail(e, "spectral route: workspace basis");
}
