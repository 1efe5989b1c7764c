// Unit operations of the spectral route, one entry point each: the pieces that
// the reference's fused CUDA path exposes as separate ops
// (cresso_cuda/cresso_cuda.cpp:44-125, kernels in cresso_cuda_kernel.cu):
//   hash bin mean                     hash_reduce_mean_cuda (cu:1222-1253)
//   hash gather                       hash_gather_cuda (cu:1255-1276)
//   2-D instant axis metric           instant_axis_metric_2d_cuda (cu:1766-1827)
//   hash metric update + log gather   hash_metric_update_log_cuda (cu:1515-1591)
//   hash impulse update + gather      hash_impulse_update_gather_cuda (cu:1593-1661)
//   metric oscillator                 metric_update_cuda (cu:1829-1867)
//   mode confidence                   confidence_update_cuda (cu:1869-1901)
//   contact oscillator, one bank      contact_update_pair_cuda (cu:1903-1965)
//   drive shaping + parameter update  drive_update_cuda (cu:2995-3223)
// The spectral step (spectral_route.hip) fuses all of them into its sweeps;
// these entry points compute the same quantities from explicit fields, for
// callers that compose a step themselves and for per-piece parity checks.
//
// Hash bin sums are 64-bit fixed-point integer atomics (rounded to nearest;
// the scale comes from this call's max |x|), merged per block in LDS and then
// in global memory: integer addition is associative, so results do not depend
// on arrival order.  Every other reduction is a fixed-order fp64 tree.
#include "common.hpp"

#include <algorithm>
#include <cmath>

namespace cresso {
namespace {

constexpr int UN_NT = 256;
constexpr int UN_MAXB = 4096;    // bins per table (the reference's hash ops, cresso_v5.py:1002)
constexpr int UN_MAXR = 4096;    // rank of the rank-level ops (the reference's contact kernel)
constexpr int UN_DRIVE_V = 16;   // moments of the drive statistics
constexpr int UN_NBLK = 1024;    // blocks of the streaming passes

// Workspace of one unit call (caller memory; cresso_unit_workspace_bytes).
struct UnitHead {
    unsigned int maxbits;    // max |x| as float bits (non-negative floats order as integers)
    unsigned int pad;
    double dstat[UN_DRIVE_V];   // drive statistics, merged
    float coef[24];          // drive coefficients
};
struct UnitOffs {
    size_t head, hist, cnt, tab, part, total;
};
inline size_t al256u(size_t v) { return (v + 255) & ~(size_t)255; }
inline UnitOffs unit_offs(int32_t bins) {
    UnitOffs o;
    size_t off = 0;
    auto take = [&](size_t b) { size_t at = off; off = al256u(off + b); return at; };
    const size_t B = (size_t)std::max(bins, 1);
    o.head = take(sizeof(UnitHead));
    o.hist = take(sizeof(unsigned long long) * B);
    o.cnt = take(sizeof(unsigned long long) * B);
    o.tab = take(sizeof(float) * B);
    o.part = take(sizeof(double) * UN_DRIVE_V * UN_NBLK);
    o.total = off;
    return o;
}
template <typename T> T* wat(void* ws, size_t off) { return reinterpret_cast<T*>(reinterpret_cast<char*>(ws) + off); }

int nblocks(int64_t n) { return (int)std::max<int64_t>(1, std::min<int64_t>(UN_NBLK, (n + UN_NT - 1) / UN_NT)); }

__device__ __forceinline__ int64_t bin_mask(int bins) { return (bins & (bins - 1)) == 0 ? (int64_t)bins - 1 : -1; }

// ---------------------------------------------------------------------------
// hash tables
// ---------------------------------------------------------------------------
__global__ void un_clear_kernel(UnitHead* head, unsigned long long* hist, unsigned long long* cnt, int bins) {
    for (int i = threadIdx.x; i < bins; i += blockDim.x) {
        hist[i] = 0ull;
        cnt[i] = 0ull;
    }
    if (threadIdx.x == 0) head->maxbits = 0u;
}

__global__ __launch_bounds__(UN_NT) void un_absmax_kernel(const float* __restrict__ x, int64_t n, UnitHead* head) {
    __shared__ float s[UN_NT / 64];
    float m = 0.f;
    for (int64_t i = (int64_t)blockIdx.x * UN_NT + threadIdx.x; i < n; i += (int64_t)gridDim.x * UN_NT)
        m = fmaxf(m, fabsf(x[i]));
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < UN_NT / 64; ++w) m = fmaxf(m, s[w]);
        atomicMax(&head->maxbits, __float_as_uint(m));
    }
}

// fixed-point scale: every |x| * scale * n stays below 2^62
__device__ __forceinline__ double un_scale(const UnitHead* head, int64_t n) {
    const double amax = (double)__uint_as_float(head->maxbits);
    // at most 2^100: x * scale stays finite in fp32 (and zero for exact zeros)
    // when every input is zero or tiny
    const int e = (int)floor(62.0 - log2((amax * 1.000001 + 1e-30) * (double)n));
    return ldexp(1.0, e < 100 ? e : 100);
}

// bin sums (fixed point) and counts: LDS per block, then global atomics
__global__ __launch_bounds__(UN_NT) void un_hist_kernel(const float* __restrict__ x, int64_t n, int bins, int salt,
                                                        const UnitHead* head, unsigned long long* __restrict__ hist,
                                                        unsigned long long* __restrict__ cnt) {
    __shared__ unsigned long long s_sum[UN_MAXB];
    __shared__ unsigned int s_cnt[UN_MAXB];
    for (int i = threadIdx.x; i < bins; i += UN_NT) {
        s_sum[i] = 0ull;
        s_cnt[i] = 0u;
    }
    __syncthreads();
    const float sc = (float)un_scale(head, n);
    const HashSalt hs = hash_salt(salt);
    const int64_t mask = bin_mask(bins);
    for (int64_t i = (int64_t)blockIdx.x * UN_NT + threadIdx.x; i < n; i += (int64_t)gridDim.x * UN_NT) {
        const int b = hash_bin((uint64_t)i, hs, bins, mask);
        atomicAdd(&s_sum[b], to_fixed_s(x[i] * sc));
        atomicAdd(&s_cnt[b], 1u);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < bins; i += UN_NT) {
        if (s_sum[i]) atomicAdd(&hist[i], s_sum[i]);
        if (s_cnt[i]) atomicAdd(&cnt[i], (unsigned long long)s_cnt[i]);
    }
}

__device__ __forceinline__ float un_cell(const unsigned long long* hist, const unsigned long long* cnt, int b,
                                         double scale) {
    // bin mean: sum / max(count, 1) (cresso_v5.py:519-526)
    return (float)((double)(long long)hist[b] / scale / fmax((double)cnt[b], 1.0));
}

// hash metric of one table: EMA of the bin means, normalized, powered,
// clamped, logged (cresso_v5.py:1016-1026)
__global__ __launch_bounds__(UN_NT) void un_metric_fin_kernel(const UnitHead* head, int64_t n, int bins,
                                                              const unsigned long long* __restrict__ hist,
                                                              const unsigned long long* __restrict__ cnt,
                                                              float* __restrict__ energy, float* __restrict__ tab,
                                                              int step, double decay, double coupling, double power,
                                                              double epsd) {
    __shared__ double red[UN_NT / 64];
    const double scale = un_scale(head, n);
    const float eps = (float)epsd;
    double acc = 0.0;
    for (int b = threadIdx.x; b < bins; b += UN_NT) {
        const float cell = un_cell(hist, cnt, b, scale);
        const float e = step <= 1 ? cell : fmaf(cell, (float)(1.0 - decay), energy[b] * (float)decay);
        energy[b] = e;
        acc += (double)e;
    }
    double v[1] = {acc};
    block_sum<1>(v, red);
    const float mean = fmaxf((float)(v[0] / (double)bins), eps);
    const float ex = (float)(coupling / fmax(0.25, power));
    for (int b = threadIdx.x; b < bins; b += UN_NT) {
        const float hm = fmaxf(energy[b] / mean, eps);
        const float hp = powf(hm, ex);
        tab[b] = logf(fmaxf(fminf(fmaxf(hp, 0.08f), 12.0f), eps));
    }
}

// hash impulse of one table: refractory EMA of |mean|, gate, impulse EMA
// (cresso_v5.py:1153-1160)
__global__ __launch_bounds__(UN_NT) void un_impulse_fin_kernel(const UnitHead* head, int64_t n, int bins,
                                                               const unsigned long long* __restrict__ hist,
                                                               const unsigned long long* __restrict__ cnt,
                                                               float* __restrict__ refr, float* __restrict__ imp,
                                                               float* __restrict__ tab, double decay, double idecay,
                                                               double gain) {
    const double scale = un_scale(head, n);
    for (int b = threadIdx.x; b < bins; b += UN_NT) {
        const float cp = un_cell(hist, cnt, b, scale);
        const float r = fmaf(fabsf(cp), (float)(1.0 - decay), refr[b] * (float)decay);
        refr[b] = r;
        const float g = 1.0f / (1.0f + (float)gain * r);
        const float m = fmaf(cp * g, (float)(1.0 - idecay), imp[b] * (float)idecay);
        imp[b] = m;
        tab[b] = m;
    }
}

// out[i] = tab[bin(i)]
__global__ __launch_bounds__(UN_NT) void un_gather_kernel(const float* __restrict__ tab, int bins, int salt, int64_t n,
                                                          float* __restrict__ out) {
    __shared__ float s_tab[UN_MAXB];
    for (int i = threadIdx.x; i < bins; i += UN_NT) s_tab[i] = tab[i];
    __syncthreads();
    const HashSalt hs = hash_salt(salt);
    const int64_t mask = bin_mask(bins);
    for (int64_t i = (int64_t)blockIdx.x * UN_NT + threadIdx.x; i < n; i += (int64_t)gridDim.x * UN_NT)
        out[i] = s_tab[hash_bin((uint64_t)i, hs, bins, mask)];
}

// bin means of one table (cresso_v5.py:519-526)
__global__ __launch_bounds__(UN_NT) void un_mean_fin_kernel(const UnitHead* head, int64_t n, int bins,
                                                            const unsigned long long* __restrict__ hist,
                                                            const unsigned long long* __restrict__ cnt,
                                                            float* __restrict__ out) {
    const double scale = un_scale(head, n);
    for (int b = blockIdx.x * UN_NT + threadIdx.x; b < bins; b += gridDim.x * UN_NT) out[b] = un_cell(hist, cnt, b, scale);
}

// out[i] = values[bin(i)] for tables too large for LDS
__global__ __launch_bounds__(UN_NT) void un_gather_global_kernel(const float* __restrict__ tab, int bins, int salt,
                                                                 int64_t n, float* __restrict__ out) {
    const HashSalt hs = hash_salt(salt);
    const int64_t mask = bin_mask(bins);
    for (int64_t i = (int64_t)blockIdx.x * UN_NT + threadIdx.x; i < n; i += (int64_t)gridDim.x * UN_NT)
        out[i] = tab[hash_bin((uint64_t)i, hs, bins, mask)];
}

// ---------------------------------------------------------------------------
// 2-D instant axis metric (cresso_v5.py:243-262 for ndim = 2): density
// min(max(rel, eps)^p, 1e6), its row and column means, each normalized by the
// mean of its marginal, exp(coupling / (2 p) * (log row term + log col term))
// clamped to [0.08, 12].  Sums are fp64 in a fixed order (no atomics).
// ---------------------------------------------------------------------------
struct AxisOffs {
    size_t rows, cols, part, glob, total;
    int chunks;
};
inline AxisOffs axis_offs(int64_t rows, int64_t cols) {
    AxisOffs o;
    // row chunks of the column pass: about 256 Ki threads in all, at most one per row
    o.chunks = (int)std::max<int64_t>(1, std::min<int64_t>({rows, 1024, (262144 + cols - 1) / std::max<int64_t>(cols, 1)}));
    size_t off = 0;
    auto take = [&](size_t b) { size_t at = off; off = al256u(off + b); return at; };
    o.rows = take(sizeof(double) * (size_t)std::max<int64_t>(rows, 1));
    o.cols = take(sizeof(double) * (size_t)std::max<int64_t>(cols, 1));
    o.part = take(sizeof(double) * (size_t)o.chunks * (size_t)std::max<int64_t>(cols, 1));
    o.glob = take(sizeof(double) * 2);
    o.total = off;
    return o;
}

__device__ __forceinline__ float am_density(float rel, float p, float eps) {
    return fminf(powf(fmaxf(rel, eps), p), 1.0e6f);
}

// one wave per row: the row's density sum in fp64 (lane partials, then the wave total)
__global__ __launch_bounds__(UN_NT) void am_rows_kernel(const float* __restrict__ rel, int64_t rows, int64_t cols,
                                                        float p, float eps, double* __restrict__ rsum) {
    const int lane = threadIdx.x & 63;
    const int64_t waves = (int64_t)gridDim.x * (UN_NT / 64);
    for (int64_t r = (int64_t)blockIdx.x * (UN_NT / 64) + (threadIdx.x >> 6); r < rows; r += waves) {
        const float* x = rel + r * cols;
        double a = 0.0;
        for (int64_t j = lane; j < cols; j += 64) a += (double)am_density(x[j], p, eps);
        a = wave_total_d(a);   // the total lands in lane 63
        if (lane == 63) rsum[r] = a;
    }
}

// column partial sums over row chunks: part[chunk][col]
__global__ __launch_bounds__(UN_NT) void am_cols_kernel(const float* __restrict__ rel, int64_t rows, int64_t cols,
                                                        int chunks, float p, float eps, double* __restrict__ part) {
    const int64_t j = (int64_t)blockIdx.x * UN_NT + threadIdx.x;
    if (j >= cols) return;
    const int c = blockIdx.y;
    const int64_t per = (rows + chunks - 1) / chunks;
    const int64_t r0 = (int64_t)c * per, r1 = r0 + per < rows ? r0 + per : rows;
    double a = 0.0;
    for (int64_t r = r0; r < r1; ++r) a += (double)am_density(rel[r * cols + j], p, eps);
    part[(size_t)c * cols + j] = a;
}

__global__ __launch_bounds__(UN_NT) void am_colfin_kernel(const double* __restrict__ part, int64_t cols, int chunks,
                                                          double* __restrict__ csum) {
    const int64_t j = (int64_t)blockIdx.x * UN_NT + threadIdx.x;
    if (j >= cols) return;
    double a = 0.0;
    for (int c = 0; c < chunks; ++c) a += part[(size_t)c * cols + j];
    csum[j] = a;
}

// means of the row means and of the column means (one block, fixed order)
__global__ __launch_bounds__(UN_NT) void am_glob_kernel(const double* __restrict__ rsum, const double* __restrict__ csum,
                                                        int64_t rows, int64_t cols, double* __restrict__ glob) {
    __shared__ double red[2 * (UN_NT / 64)];
    double v[2] = {0.0, 0.0};
    for (int64_t i = threadIdx.x; i < rows; i += UN_NT) v[0] += (double)(float)(rsum[i] / (double)cols);
    for (int64_t i = threadIdx.x; i < cols; i += UN_NT) v[1] += (double)(float)(csum[i] / (double)rows);
    block_sum<2>(v, red);
    if (threadIdx.x == 0) {
        glob[0] = v[0] / (double)rows;
        glob[1] = v[1] / (double)cols;
    }
}

__global__ __launch_bounds__(UN_NT) void am_apply_kernel(const double* __restrict__ rsum,
                                                         const double* __restrict__ csum,
                                                         const double* __restrict__ glob, int64_t rows, int64_t cols,
                                                         float k, float eps, float* __restrict__ out) {
    const int64_t n = rows * cols;
    const float gr = fmaxf((float)glob[0], eps), gc = fmaxf((float)glob[1], eps);
    for (int64_t i = (int64_t)blockIdx.x * UN_NT + threadIdx.x; i < n; i += (int64_t)gridDim.x * UN_NT) {
        const int64_t r = i / cols, j = i - r * cols;
        const float rm = (float)(rsum[r] / (double)cols), cm = (float)(csum[j] / (double)rows);
        const float lg = logf(fmaxf(rm / gr, eps)) + logf(fmaxf(cm / gc, eps));
        out[i] = fminf(fmaxf(expf(k * lg), 0.08f), 12.0f);
    }
}

__global__ __launch_bounds__(UN_NT) void am_ones_kernel(int64_t n, float* __restrict__ out) {
    for (int64_t i = (int64_t)blockIdx.x * UN_NT + threadIdx.x; i < n; i += (int64_t)gridDim.x * UN_NT) out[i] = 1.0f;
}

// ---------------------------------------------------------------------------
// rank-level oscillators (one block)
// ---------------------------------------------------------------------------
__global__ void un_metric_update_kernel(float* mq_c, float* mq_s, float* mp_c, float* mp_s, const float* port_c,
                                        const float* port_s, const float* omega, int rank, double dt, double fr) {
    const float damp = (float)fmax(0.0, 1.0 - dt * fr);
    const float fdt = (float)dt;
    for (int r = threadIdx.x; r < rank; r += blockDim.x) {
        const float w2 = omega[r] * omega[r];
        float* mq[2] = {mq_c, mq_s};
        float* mp[2] = {mp_c, mp_s};
        const float* pt[2] = {port_c, port_s};
        for (int k = 0; k < 2; ++k) {
            const float p = fmaf(pt[k][r] - w2 * mq[k][r], fdt, mp[k][r] * damp);
            mp[k][r] = p;
            mq[k][r] = fminf(fmaxf(fmaf(p, fdt, mq[k][r]), -3.0f), 3.0f);
        }
    }
}

__global__ void un_confidence_kernel(float* conf, const float* pc, const float* ps, const float* qc, const float* qs,
                                     int rank, double decay, double epsd) {
    const float eps = (float)epsd;
    for (int r = threadIdx.x; r < rank; r += blockDim.x) {
        const float pe = sqrtf(pc[r] * pc[r] + ps[r] * ps[r] + eps);
        const float qe = sqrtf(qc[r] * qc[r] + qs[r] * qs[r] + eps);
        const float sup = fminf(fmaxf((pc[r] * qc[r] + ps[r] * qs[r]) / (pe * qe + eps), -1.0f), 1.0f);
        conf[r] = fminf(fmaxf(fmaf(sup, (float)(1.0 - decay), conf[r] * (float)decay), -4.0f), 4.0f);
    }
}

struct ContactHyper {
    double dt, refractory_decay, refractory_gain, surprise_gain, surprise_brake, impulse_friction, contact_gain,
        restoring, cubic;
};

// one bank of the contact oscillator (cresso_v5.py:914-943); the block sums
// mean p^2, mean (omega q)^2 and mean(gp p) over the rank in fp64
__global__ __launch_bounds__(UN_NT) void un_contact_kernel(float* q, float* p, const float* port, const float* omega,
                                                           float* calcium, float* action, const float* surprise,
                                                           int rank, ContactHyper c) {
    __shared__ double red[3 * (UN_NT / 64)];
    __shared__ float s_gp[UN_MAXR];
    const float sur = *surprise;
    const float plast = 1.0f + (float)c.surprise_gain * sur / (1.0f + sur);
    const float brake = 1.0f / (1.0f + (float)c.surprise_brake * sur);
    double v[3] = {0.0, 0.0, 0.0};
    for (int r = threadIdx.x; r < rank; r += UN_NT) {
        const float ca = fmaf(fabsf(port[r]), (float)(1.0 - c.refractory_decay), calcium[r] * (float)c.refractory_decay);
        calcium[r] = ca;
        const float gate = 1.0f / (1.0f + (float)c.refractory_gain * ca);
        const float gp = port[r] * gate * plast * brake;
        s_gp[r] = gp;
        const float wq = omega[r] * q[r];
        v[0] += (double)(p[r] * p[r]);
        v[1] += (double)(wq * wq);
        v[2] += (double)(gp * p[r]);
    }
    block_sum<3>(v, red);
    const float energy = 0.5f * ((float)(v[0] / rank) + (float)(v[1] / rank));
    const float power = (float)(v[2] / rank);
    const float fdt = (float)c.dt;
    const float act = fmaf(power - energy, fdt, *action * 0.985f);
    __syncthreads();
    if (threadIdx.x == 0) *action = act;
    const float fr = (float)c.impulse_friction + (float)c.contact_gain * tanhf(fabsf(act));
    const float damp = fmaxf(1.0f - fdt * fr, 0.0f);
    for (int r = threadIdx.x; r < rank; r += UN_NT) {
        const float qv = q[r];
        const float w2 = omega[r] * omega[r];
        const float pn = fmaf(s_gp[r] - (float)c.restoring * w2 * qv - (float)c.cubic * (qv * qv * qv), fdt, p[r] * damp);
        p[r] = pn;
        q[r] = fminf(fmaxf(fmaf(pn, fdt, qv), -8.0f), 8.0f);
    }
}

// ---------------------------------------------------------------------------
// drive shaping and update (cresso_v5.py:1303-1353)
// ---------------------------------------------------------------------------
struct DriveIn {
    const float *t, *pred, *err, *echo, *hp;
    const float* surprise;
    float* drive_energy;
    int64_t n;
    int step, hard;
};

// rat = t/(1+|t|/clip), bnd = clip tanh(t/clip), root = sign(t) sqrt(min(|t|, clip^2) + eps)
__device__ __forceinline__ void un_shape(float t, float clip, float eps, float& rat, float& bnd, float& root) {
    rat = t / (1.0f + fabsf(t) / clip);
    bnd = tanhf(t / clip) * clip;
    root = (t > 0.f ? 1.0f : (t < 0.f ? -1.0f : 0.0f)) * sqrtf(fminf(fabsf(t), clip * clip) + eps);
}

// moments: 0 tt, 1 pp, 2 tp, 3 rr, 4 bb, 5 oo, 6 rb, 7 ro, 8 bo, 9 tr, 10 tb, 11 to, 12 ee, 13 echo^2, 14 hp^2
__global__ __launch_bounds__(UN_NT) void un_drive_moments_kernel(DriveIn in, double clipd, double epsd,
                                                                 double* __restrict__ part) {
    __shared__ double red[UN_DRIVE_V * (UN_NT / 64)];
    const float clip = (float)clipd, eps = (float)epsd;
    double m[UN_DRIVE_V] = {};
    for (int64_t i = (int64_t)blockIdx.x * UN_NT + threadIdx.x; i < in.n; i += (int64_t)gridDim.x * UN_NT) {
        const float t = in.t[i], pr = in.pred[i], e = in.err[i];
        float rat, bnd, root;
        un_shape(t, clip, eps, rat, bnd, root);
        m[0] += (double)(t * t); m[1] += (double)(pr * pr); m[2] += (double)(t * pr);
        m[3] += (double)(rat * rat); m[4] += (double)(bnd * bnd); m[5] += (double)(root * root);
        m[6] += (double)(rat * bnd); m[7] += (double)(rat * root); m[8] += (double)(bnd * root);
        m[9] += (double)(t * rat); m[10] += (double)(t * bnd); m[11] += (double)(t * root);
        m[12] += (double)(e * e);
        if (in.echo) m[13] += (double)(in.echo[i] * in.echo[i]);
        if (in.hp) m[14] += (double)(in.hp[i] * in.hp[i]);
    }
    block_sum<UN_DRIVE_V>(m, red);
    if (threadIdx.x < UN_DRIVE_V) part[(size_t)threadIdx.x * gridDim.x + blockIdx.x] = m[threadIdx.x];
}

// one block: merge the partials in block order, then every coefficient of the drive
// coef: 0 cA(core) 1 mix 2 k_rat 3 k_bnd 4 k_root 5 k_t 6 nov_mix 7 nscale 8 k_res 9 k_echo 10 k_hp 11 clip 12 eps
__global__ __launch_bounds__(UN_NT) void un_drive_coef_kernel(DriveIn in, int nblk, const double* __restrict__ part,
                                                              UnitHead* head, cresso_hyper h) {
    __shared__ double red[UN_DRIVE_V * (UN_NT / 64)];
    double m[UN_DRIVE_V] = {};
    for (int v = 0; v < UN_DRIVE_V; ++v)
        for (int b = threadIdx.x; b < nblk; b += UN_NT) m[v] += part[(size_t)v * nblk + b];
    block_sum<UN_DRIVE_V>(m, red);
    if (threadIdx.x != 0) return;
    const double n = (double)in.n;
    const float eps = (float)h.eps;
    const float S = *in.surprise;
    const float frms = sqrtf((float)(m[0] / n) + eps);
    const float prms = sqrtf((float)(m[1] / n) + eps);
    float align = fminf(fmaxf((float)(m[2] / n) / (frms * prms + eps), -1.0f), 1.0f);
    float agate = fminf(fmaxf((align + 1.0f) * 0.5f, 0.0f), 1.0f);
    if (!(sqrt(m[1] / n + h.eps) > sqrt(h.eps))) agate = 0.0f;   // the predicate in fp64
    const double warm = h.warmup_steps == 0 ? 1.0 : 1.0 - exp(-(double)in.step / (double)std::max(1, h.warmup_steps));
    const float mix = (float)(h.prediction_mix * warm) * agate * (1.0f / (1.0f + S));
    const float rms_rat = sqrtf((float)(m[3] / n) + eps), rms_root = sqrtf((float)(m[5] / n) + eps);
    const float kroot = rms_rat / fmaxf(rms_root, eps);
    const float spike = (float)h.spike_mix / (1.0f + S);
    const float rmix = (in.hard ? (float)h.root_channel_mix : 0.0f) / (1.0f + 0.5f * S);
    // shaped = ar rat + ab bnd + ao root
    const double ar = (double)((1.0f - rmix) * (1.0f - spike)), ab = (double)((1.0f - rmix) * spike),
                 ao = (double)(rmix * kroot);
    const double sh2 = ar * ar * m[3] + ab * ab * m[4] + ao * ao * m[5] + 2.0 * (ar * ab * m[6] + ar * ao * m[7] + ab * ao * m[8]);
    const float srms = sqrtf((float)(sh2 / n) + eps);
    const float dmix = (float)h.direct_force_mix / (1.0f + 0.35f * S);
    const float kdir = srms / fmaxf(frms, eps);
    // core = cr rat + cb bnd + co root + ct t
    const double cr = (1.0 - (double)dmix) * ar, cb = (1.0 - (double)dmix) * ab, co = (1.0 - (double)dmix) * ao;
    const double ct = (double)(dmix * kdir);
    const double core2 = cr * cr * m[3] + cb * cb * m[4] + co * co * m[5] + ct * ct * m[0] +
                         2.0 * (cr * cb * m[6] + cr * co * m[7] + cb * co * m[8] + ct * cr * m[9] + ct * cb * m[10] + ct * co * m[11]);
    const float crms = sqrtf((float)(core2 / n) + eps);
    const float erms = sqrtf((float)(m[12] / n) + eps);
    const float resmix = (float)h.residual_feedback_mix / (1.0f + S);
    float* k = head->coef;
    k[0] = 1.0f - mix;
    k[1] = mix;
    k[2] = (float)cr; k[3] = (float)cb; k[4] = (float)co; k[5] = (float)ct;
    k[6] = (float)h.novelty_mix;
    k[7] = 1.0f / ((float)h.drive_clip * (1.0f + S));
    k[8] = resmix * crms / fmaxf(erms, eps);
    const bool echo_on = in.hard && h.echo_mix != 0.0 && in.echo;
    k[9] = echo_on ? (float)h.echo_mix * srms / fmaxf(sqrtf((float)(m[13] / n) + eps), eps) : 0.0f;
    k[10] = (in.hard && in.hp) ? (float)h.hash_drive_mix * srms / fmaxf(sqrtf((float)(m[14] / n) + eps), eps) : 0.0f;
    k[11] = (float)h.drive_clip;
    k[12] = eps;
}

__device__ __forceinline__ float un_drive_at(const DriveIn& in, const float* k, int64_t i) {
    const float t = in.t[i];
    float rat, bnd, root;
    un_shape(t, k[11], k[12], rat, bnd, root);
    const float core = k[2] * rat + k[3] * bnd + k[4] * root + k[5] * t;
    const float e = in.err[i];
    const float nov = tanhf(e * k[7]) * k[11];
    float d = k[0] * core + k[1] * in.pred[i] + k[6] * nov + k[8] * e;
    if (in.echo) d += k[9] * in.echo[i];
    if (in.hp) d += k[10] * in.hp[i];
    return d;
}

__global__ __launch_bounds__(UN_NT) void un_drive_energy_kernel(DriveIn in, const UnitHead* head,
                                                                double* __restrict__ part) {
    __shared__ double red[UN_NT / 64];
    __shared__ float k[24];
    if (threadIdx.x < 24) k[threadIdx.x] = head->coef[threadIdx.x];
    __syncthreads();
    double v[1] = {0.0};
    for (int64_t i = (int64_t)blockIdx.x * UN_NT + threadIdx.x; i < in.n; i += (int64_t)gridDim.x * UN_NT) {
        const float d = un_drive_at(in, k, i);
        v[0] += (double)(d * d);
    }
    block_sum<1>(v, red);
    if (threadIdx.x == 0) part[blockIdx.x] = v[0];
}

// drive-energy reservoir and gain (one block), then the update
__global__ __launch_bounds__(UN_NT) void un_drive_gain_kernel(DriveIn in, int nblk, const double* __restrict__ part,
                                                              UnitHead* head, cresso_hyper h) {
    __shared__ double red[UN_NT / 64];
    double v[1] = {0.0};
    for (int b = threadIdx.x; b < nblk; b += UN_NT) v[0] += part[b];
    block_sum<1>(v, red);
    if (threadIdx.x != 0) return;
    const float now = (float)(v[0] / (double)in.n);
    const float de = in.step <= 1 ? now : fmaf(now, (float)(1.0 - h.reservoir_decay), *in.drive_energy * (float)h.reservoir_decay);
    *in.drive_energy = de;
    const float gain = fminf(fmaxf((float)h.target_update_rms / sqrtf(de + (float)h.eps), (float)h.min_gain),
                             (float)h.max_gain);
    head->coef[13] = gain;
}

template <typename PT>
__global__ __launch_bounds__(UN_NT) void un_drive_apply_kernel(DriveIn in, const UnitHead* head, PT* __restrict__ param,
                                                               double lr) {
    __shared__ float k[24];
    if (threadIdx.x < 24) k[threadIdx.x] = head->coef[threadIdx.x];
    __syncthreads();
    const float gain = k[13];
    const float nlr = (float)update_alpha<PT>(-lr);
    for (int64_t i = (int64_t)blockIdx.x * UN_NT + threadIdx.x; i < in.n; i += (int64_t)gridDim.x * UN_NT) {
        const float u = to_f(from_w<PT>(un_drive_at(in, k, i) * gain));
        param[i] = from_w<PT>(fmaf(nlr, u, to_f(param[i])));
    }
}

int32_t check_ws(void* ws, size_t ws_bytes, int32_t bins) {
    if (!ws) return fail(CRESSO_E_INVALID, "unit op: null workspace");
    if ((uintptr_t)ws % 256 != 0) return fail(CRESSO_E_INVALID, "unit op: workspace must be 256-byte aligned");
    const size_t need = unit_offs(bins).total;
    if (ws_bytes < need) return fail(CRESSO_E_INVALID, "unit op: workspace of %zu bytes is smaller than %zu", ws_bytes, need);
    return CRESSO_OK;
}

int32_t launched(const char* what) {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? CRESSO_OK : hip_fail(e, what);
}

}  // namespace
}  // namespace cresso

using namespace cresso;

extern "C" size_t cresso_unit_workspace_bytes(int32_t bins) { return unit_offs(bins).total; }

extern "C" int32_t cresso_hash_reduce_mean(const float* x, int64_t numel, int32_t bins, int32_t salt, float* mean_out,
                                           void* workspace, size_t workspace_bytes, void* stream) {
    if (!x || !mean_out) return fail(CRESSO_E_INVALID, "hash reduce mean: null argument");
    if (numel < 1) return fail(CRESSO_E_INVALID, "hash reduce mean: numel must be positive");
    if (bins < 1 || bins > UN_MAXB) return fail(CRESSO_E_INVALID, "hash reduce mean: bins %d outside 1..%d", bins, UN_MAXB);
    if (salt < 0) return fail(CRESSO_E_INVALID, "hash reduce mean: salt must be >= 0");
    int32_t rc = check_ws(workspace, workspace_bytes, bins);
    if (rc != CRESSO_OK) return rc;
    const UnitOffs o = unit_offs(bins);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    UnitHead* head = wat<UnitHead>(workspace, o.head);
    unsigned long long* hist = wat<unsigned long long>(workspace, o.hist);
    unsigned long long* cnt = wat<unsigned long long>(workspace, o.cnt);
    const int nb = nblocks(numel);
    hipLaunchKernelGGL(un_clear_kernel, dim3(1), dim3(UN_NT), 0, s, head, hist, cnt, bins);
    hipLaunchKernelGGL(un_absmax_kernel, dim3(nb), dim3(UN_NT), 0, s, x, numel, head);
    hipLaunchKernelGGL(un_hist_kernel, dim3(nb), dim3(UN_NT), 0, s, x, numel, bins, salt, head, hist, cnt);
    hipLaunchKernelGGL(un_mean_fin_kernel, dim3((bins + UN_NT - 1) / UN_NT), dim3(UN_NT), 0, s, head, numel, bins, hist,
                       cnt, mean_out);
    return launched("hash reduce mean");
}

extern "C" int32_t cresso_hash_gather(const float* values, int32_t bins, int64_t numel, int32_t salt, float* out,
                                      void* stream) {
    if (!values || !out) return fail(CRESSO_E_INVALID, "hash gather: null argument");
    if (numel < 1) return fail(CRESSO_E_INVALID, "hash gather: numel must be positive");
    if (bins < 1) return fail(CRESSO_E_INVALID, "hash gather: values must be non-empty");
    if (salt < 0) return fail(CRESSO_E_INVALID, "hash gather: salt must be >= 0");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int nb = nblocks(numel);
    if (bins <= UN_MAXB)
        hipLaunchKernelGGL(un_gather_kernel, dim3(nb), dim3(UN_NT), 0, s, values, bins, salt, numel, out);
    else
        hipLaunchKernelGGL(un_gather_global_kernel, dim3(nb), dim3(UN_NT), 0, s, values, bins, salt, numel, out);
    return launched("hash gather");
}

extern "C" size_t cresso_instant_axis_metric_2d_workspace_bytes(int64_t rows, int64_t cols) {
    return rows > 0 && cols > 0 ? axis_offs(rows, cols).total : 0;
}

extern "C" int32_t cresso_instant_axis_metric_2d(const float* rel, int64_t rows, int64_t cols, double power,
                                                 double coupling, double eps, float* out, void* workspace,
                                                 size_t workspace_bytes, void* stream) {
    if (!rel || !out) return fail(CRESSO_E_INVALID, "instant axis metric: null argument");
    if (rows < 1 || cols < 1) return fail(CRESSO_E_INVALID, "instant axis metric: requires a non-empty 2D tensor");
    if (cols > ((int64_t)1 << 31) || rows > (((int64_t)1 << 46) / cols))
        return fail(CRESSO_E_INVALID, "instant axis metric: %lld x %lld elements is too large", (long long)rows,
                    (long long)cols);
    if (!std::isfinite(power) || !std::isfinite(coupling)) return fail(CRESSO_E_INVALID, "instant axis metric: power and coupling must be finite");
    if (!(eps > 0.0) || !std::isfinite(eps)) return fail(CRESSO_E_INVALID, "instant axis metric: eps must be positive and finite");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int64_t n = rows * cols;
    const int nb = nblocks(n);
    if (coupling == 0.0 || n <= 1) {   // cresso_v5.py:249-250
        hipLaunchKernelGGL(am_ones_kernel, dim3(nb), dim3(UN_NT), 0, s, n, out);
        return launched("instant axis metric");
    }
    if (!workspace) return fail(CRESSO_E_INVALID, "instant axis metric: null workspace");
    if ((uintptr_t)workspace % 256 != 0) return fail(CRESSO_E_INVALID, "instant axis metric: workspace must be 256-byte aligned");
    const AxisOffs o = axis_offs(rows, cols);
    if (workspace_bytes < o.total)
        return fail(CRESSO_E_INVALID, "instant axis metric: workspace of %zu bytes is smaller than %zu", workspace_bytes, o.total);
    const double p = std::max(power, 0.25);
    double* rsum = wat<double>(workspace, o.rows);
    double* csum = wat<double>(workspace, o.cols);
    double* part = wat<double>(workspace, o.part);
    double* glob = wat<double>(workspace, o.glob);
    const float fe = (float)eps;
    const int rb = (int)std::min<int64_t>(4096, (rows + UN_NT / 64 - 1) / (UN_NT / 64));
    const int cb = (int)((cols + UN_NT - 1) / UN_NT);
    hipLaunchKernelGGL(am_rows_kernel, dim3(rb), dim3(UN_NT), 0, s, rel, rows, cols, (float)p, fe, rsum);
    hipLaunchKernelGGL(am_cols_kernel, dim3(cb, o.chunks), dim3(UN_NT), 0, s, rel, rows, cols, o.chunks, (float)p, fe,
                       part);
    hipLaunchKernelGGL(am_colfin_kernel, dim3(cb), dim3(UN_NT), 0, s, part, cols, o.chunks, csum);
    hipLaunchKernelGGL(am_glob_kernel, dim3(1), dim3(UN_NT), 0, s, rsum, csum, rows, cols, glob);
    hipLaunchKernelGGL(am_apply_kernel, dim3(nb), dim3(UN_NT), 0, s, rsum, csum, glob, rows, cols,
                       (float)(coupling / (2.0 * p)), fe, out);
    return launched("instant axis metric");
}

extern "C" int32_t cresso_hash_metric_update_log(const float* density_source, int64_t numel, float* hash_energy,
                                                 int32_t bins, int32_t salt, int32_t step, double hash_decay,
                                                 double hash_metric_coupling, double energy_power, double eps,
                                                 float* term_out, void* workspace, size_t workspace_bytes,
                                                 void* stream) {
    if (!density_source || !hash_energy || !term_out) return fail(CRESSO_E_INVALID, "hash metric: null argument");
    if (numel < 1) return fail(CRESSO_E_INVALID, "hash metric: numel must be positive");
    if (bins < 1 || bins > UN_MAXB) return fail(CRESSO_E_INVALID, "hash metric: bins %d outside 1..%d", bins, UN_MAXB);
    if (salt < 0) return fail(CRESSO_E_INVALID, "hash metric: salt must be >= 0");
    if (step < 1) return fail(CRESSO_E_INVALID, "hash metric: step must be >= 1 (after the increment)");
    int32_t rc = check_ws(workspace, workspace_bytes, bins);
    if (rc != CRESSO_OK) return rc;
    const UnitOffs o = unit_offs(bins);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    UnitHead* head = wat<UnitHead>(workspace, o.head);
    unsigned long long* hist = wat<unsigned long long>(workspace, o.hist);
    unsigned long long* cnt = wat<unsigned long long>(workspace, o.cnt);
    float* tab = wat<float>(workspace, o.tab);
    const int nb = nblocks(numel);
    hipLaunchKernelGGL(un_clear_kernel, dim3(1), dim3(UN_NT), 0, s, head, hist, cnt, bins);
    hipLaunchKernelGGL(un_absmax_kernel, dim3(nb), dim3(UN_NT), 0, s, density_source, numel, head);
    hipLaunchKernelGGL(un_hist_kernel, dim3(nb), dim3(UN_NT), 0, s, density_source, numel, bins, salt, head, hist, cnt);
    hipLaunchKernelGGL(un_metric_fin_kernel, dim3(1), dim3(UN_NT), 0, s, head, numel, bins, hist, cnt, hash_energy, tab,
                       step, hash_decay, hash_metric_coupling, energy_power, eps);
    hipLaunchKernelGGL(un_gather_kernel, dim3(nb), dim3(UN_NT), 0, s, tab, bins, salt, numel, term_out);
    return launched("hash metric");
}

extern "C" int32_t cresso_hash_impulse_update_gather(const float* port_source, int64_t numel, float* hash_refractory,
                                                     float* hash_impulse, int32_t bins, int32_t salt,
                                                     double hash_decay, double hash_impulse_decay,
                                                     double refractory_gain, float* retrieved_out, void* workspace,
                                                     size_t workspace_bytes, void* stream) {
    if (!port_source || !hash_refractory || !hash_impulse || !retrieved_out)
        return fail(CRESSO_E_INVALID, "hash impulse: null argument");
    if (numel < 1) return fail(CRESSO_E_INVALID, "hash impulse: numel must be positive");
    if (bins < 1 || bins > UN_MAXB) return fail(CRESSO_E_INVALID, "hash impulse: bins %d outside 1..%d", bins, UN_MAXB);
    if (salt < 0) return fail(CRESSO_E_INVALID, "hash impulse: salt must be >= 0");
    int32_t rc = check_ws(workspace, workspace_bytes, bins);
    if (rc != CRESSO_OK) return rc;
    const UnitOffs o = unit_offs(bins);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    UnitHead* head = wat<UnitHead>(workspace, o.head);
    unsigned long long* hist = wat<unsigned long long>(workspace, o.hist);
    unsigned long long* cnt = wat<unsigned long long>(workspace, o.cnt);
    float* tab = wat<float>(workspace, o.tab);
    const int nb = nblocks(numel);
    hipLaunchKernelGGL(un_clear_kernel, dim3(1), dim3(UN_NT), 0, s, head, hist, cnt, bins);
    hipLaunchKernelGGL(un_absmax_kernel, dim3(nb), dim3(UN_NT), 0, s, port_source, numel, head);
    hipLaunchKernelGGL(un_hist_kernel, dim3(nb), dim3(UN_NT), 0, s, port_source, numel, bins, salt, head, hist, cnt);
    hipLaunchKernelGGL(un_impulse_fin_kernel, dim3(1), dim3(UN_NT), 0, s, head, numel, bins, hist, cnt,
                       hash_refractory, hash_impulse, tab, hash_decay, hash_impulse_decay, refractory_gain);
    hipLaunchKernelGGL(un_gather_kernel, dim3(nb), dim3(UN_NT), 0, s, tab, bins, salt, numel, retrieved_out);
    return launched("hash impulse");
}

extern "C" int32_t cresso_metric_update(float* metric_cos, float* metric_sin, float* metric_p_cos, float* metric_p_sin,
                                        const float* mcos_port, const float* msin_port, const float* omega,
                                        int32_t rank, double metric_dt, double metric_friction, void* stream) {
    if (!metric_cos || !metric_sin || !metric_p_cos || !metric_p_sin || !mcos_port || !msin_port || !omega)
        return fail(CRESSO_E_INVALID, "metric update: null argument");
    if (rank < 1 || rank > UN_MAXR) return fail(CRESSO_E_INVALID, "metric update: rank %d outside 1..%d", rank, UN_MAXR);
    hipLaunchKernelGGL(un_metric_update_kernel, dim3(1), dim3(UN_NT), 0, reinterpret_cast<hipStream_t>(stream),
                       metric_cos, metric_sin, metric_p_cos, metric_p_sin, mcos_port, msin_port, omega, rank, metric_dt,
                       metric_friction);
    return launched("metric update");
}

extern "C" int32_t cresso_confidence_update(float* confidence, const float* pcos_port, const float* psin_port,
                                            const float* qcos, const float* qsin, int32_t rank, double confidence_decay,
                                            double eps, void* stream) {
    if (!confidence || !pcos_port || !psin_port || !qcos || !qsin)
        return fail(CRESSO_E_INVALID, "confidence update: null argument");
    if (rank < 1 || rank > UN_MAXR) return fail(CRESSO_E_INVALID, "confidence update: rank %d outside 1..%d", rank, UN_MAXR);
    hipLaunchKernelGGL(un_confidence_kernel, dim3(1), dim3(UN_NT), 0, reinterpret_cast<hipStream_t>(stream), confidence,
                       pcos_port, psin_port, qcos, qsin, rank, confidence_decay, eps);
    return launched("confidence update");
}

extern "C" int32_t cresso_contact_update_pair(float* q, float* p, const float* port, const float* omega, float* calcium,
                                              float* action, const float* surprise, int32_t rank, double dt,
                                              double refractory_decay, double refractory_gain, double surprise_gain,
                                              double surprise_brake, double impulse_friction, double contact_gain,
                                              double restoring, double cubic, void* stream) {
    if (!q || !p || !port || !omega || !calcium || !action || !surprise)
        return fail(CRESSO_E_INVALID, "contact update: null argument");
    if (rank < 1 || rank > UN_MAXR) return fail(CRESSO_E_INVALID, "contact update: rank %d outside 1..%d", rank, UN_MAXR);
    const ContactHyper c{dt, refractory_decay, refractory_gain, surprise_gain, surprise_brake, impulse_friction,
                         contact_gain, restoring, cubic};
    hipLaunchKernelGGL(un_contact_kernel, dim3(1), dim3(UN_NT), 0, reinterpret_cast<hipStream_t>(stream), q, p, port,
                       omega, calcium, action, surprise, rank, c);
    return launched("contact update");
}

extern "C" int32_t cresso_drive_update(void* param, int32_t param_dtype, const float* tangent, const float* pred,
                                       const float* error, const float* echo, const float* hash_pred,
                                       const float* surprise, float* drive_energy, int64_t numel, int32_t step,
                                       int32_t hard, const cresso_hyper* hyper, void* workspace, size_t workspace_bytes,
                                       void* stream) {
    if (!param || !tangent || !pred || !error || !surprise || !drive_energy || !hyper)
        return fail(CRESSO_E_INVALID, "drive update: null argument");
    if (numel < 1) return fail(CRESSO_E_INVALID, "drive update: numel must be positive");
    if (step < 1) return fail(CRESSO_E_INVALID, "drive update: step must be >= 1 (after the increment)");
    if (!(hyper->drive_clip > 0.0)) return fail(CRESSO_E_INVALID, "drive update: drive_clip must be positive");
    if (param_dtype != CRESSO_F32 && param_dtype != CRESSO_BF16 && param_dtype != CRESSO_F16)
        return fail(CRESSO_E_UNSUPPORTED, "drive update: param dtype %d not supported (f32, bf16, f16)", param_dtype);
    int32_t rc = check_ws(workspace, workspace_bytes, 1);
    if (rc != CRESSO_OK) return rc;
    const UnitOffs o = unit_offs(1);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    UnitHead* head = wat<UnitHead>(workspace, o.head);
    double* part = wat<double>(workspace, o.part);
    DriveIn in{tangent, pred, error, echo, hash_pred, surprise, drive_energy, numel, step, hard ? 1 : 0};
    const int nb = nblocks(numel);
    hipLaunchKernelGGL(un_drive_moments_kernel, dim3(nb), dim3(UN_NT), 0, s, in, hyper->drive_clip, hyper->eps, part);
    hipLaunchKernelGGL(un_drive_coef_kernel, dim3(1), dim3(UN_NT), 0, s, in, nb, part, head, *hyper);
    hipLaunchKernelGGL(un_drive_energy_kernel, dim3(nb), dim3(UN_NT), 0, s, in, head, part);
    hipLaunchKernelGGL(un_drive_gain_kernel, dim3(1), dim3(UN_NT), 0, s, in, nb, part, head, *hyper);
    switch (param_dtype) {
        case CRESSO_F32:
            hipLaunchKernelGGL(un_drive_apply_kernel<float>, dim3(nb), dim3(UN_NT), 0, s, in, head, (float*)param, hyper->lr);
            break;
        case CRESSO_BF16:
            hipLaunchKernelGGL(un_drive_apply_kernel<__hip_bfloat16>, dim3(nb), dim3(UN_NT), 0, s, in, head,
                               (__hip_bfloat16*)param, hyper->lr);
            break;
        case CRESSO_F16:
            hipLaunchKernelGGL(un_drive_apply_kernel<__half>, dim3(nb), dim3(UN_NT), 0, s, in, head, (__half*)param,
                               hyper->lr);
            break;
        default:   // rejected above, before any launch
            break;
    }
    return launched("drive update");
}
