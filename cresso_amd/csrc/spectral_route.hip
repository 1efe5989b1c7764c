// Spectral / coordinate-hash route of CRESSO5 on gfx950: plans, workspace set-up
// and the C ABI.  The kernels and the step sequence are in spectral_kernels.hpp;
// the step itself is instantiated per dtype pair in spectral_step_*.hip.
#define CRESSO_SPECTRAL_WS_KERNELS 1
#include "spectral_kernels.hpp"

#include <atomic>
#include <map>
#include <mutex>

namespace cresso {
namespace {

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


size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

int32_t plan_spectral(const int64_t* shape, int32_t ndim, const int64_t* freqs, int32_t rank, int32_t bins,
                      int32_t tables, int32_t work, cresso_spectral_plan& P) {
    if (ndim < 1 || ndim > 8) return fail(CRESSO_E_INVALID, "spectral route: ndim %d outside 1..8", ndim);
    if (work != CRESSO_F32 && work != CRESSO_F64)
        return fail(CRESSO_E_INVALID, "spectral route: work dtype %d is neither CRESSO_F32 nor CRESSO_F64", work);
    P.work = work;
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
    // the same constants in fp64 for the fp64 work dtype (math.pi * f, (math.pi * c) * max(1, f))
    P.axc64.clear();
    if (work == CRESSO_F64)
        for (int r = 0; r < rank; ++r)
            for (int a = 0; a < ndim; ++a) {
                const int64_t f = freqs[(size_t)r * ndim + a];
                AxisConst64 c;
                c.pf = M_PI * (double)f;
                c.pcm = (M_PI * (0.25 + 1.75 * hash_unit_host(r, 17 + a))) * (double)std::max<int64_t>(1, f);
                c.mu = 0.15 + 0.70 * hash_unit_host(r, 101 + a);
                c.sig = 0.18 + 0.20 * hash_unit_host(r, 151 + a);
                c.f = (int32_t)f;
                c.kind = r % 4;
                P.axc64.push_back(c);
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
    P.rmax = rank <= 8 ? 8 : (rank <= 16 ? 16 : 32);
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
    // the matrix-core sweeps take panels of 32 or 64 rows that tile the rows
    // exactly: prefer those from 256 rows on (C5's (512,256,3,3) and
    // (256,256,3,3) conv tensors then take the matrix-core sweeps instead of
    // the general kernels' 16-row panels: C5 1.32 -> 1.28 ms), 64 rows when
    // they tile the rows (measured: (5632,2048) 0.174 -> 0.166 ms a step; a
    // lone (2048,2048) tensor, 256 blocks of 64 rows, is slower, 0.098 ->
    // 0.107 ms, but C4's batches of them fill the GPU and gain: 12.2-12.3 ->
    // 12.0-12.1 ms)
    if (pr >= 16 && g.rows >= 256 && g.rows % 32 == 0) pr = (g.rows % 64 == 0) ? 64 : 32;
    // ranks above 16 run the general sweeps, whose per-block LDS (row
    // coefficients of 2 * 68 + 64 floats per panel row) fits with 32-row panels
    if (rank > 16) pr = std::min<int64_t>(pr, 32);
    // 32-bit element offsets inside a panel: PR * cols < 2^29
    if (g.cols >= ((int64_t)1 << 29))
        return fail(CRESSO_E_UNSUPPORTED, "spectral route: %lld elements per row exceed this build's panel limit",
                    (long long)g.cols);
    pr = std::min<int64_t>(pr, ((int64_t)1 << 29) / g.cols);
    g.PR = (int32_t)std::max<int64_t>(1, pr);
    g.panels = (int32_t)((g.rows + g.PR - 1) / g.PR);
    g.nblk = g.slabs * g.panels;
    // the matrix-core sweeps' histograms: atomic merges (part_reduce's row
    // groups, or every block of a multi-round launch) spread over copies
    g.hcopies = mtables(g) ? SP_HCOPIES : 1;
    // Gram pair sums: one block per ~128 rows/columns of the longer axis, at most 256
    g.nblkg = (int32_t)std::max<int64_t>(1, std::min<int64_t>(256, std::max(g.rows, g.cols) / 128));
    // flat force-RMS sweep and parameter update: contiguous chunks (multiple of 8 elements) per block
    g.nblk1 = (int32_t)std::max<int64_t>(1, std::min<int64_t>(1024, (g.n + 16383) / 16384));
    g.chunk1 = (((g.n + g.nblk1 - 1) / g.nblk1) + 7) & ~(int64_t)7;   // multiples of 8 elements (16-byte loads)
    g.nblk1 = (int32_t)((g.n + g.chunk1 - 1) / g.chunk1);
    // axis density sums: density <= 1e6 per element, sums below 2^62
    g.shrink = 1.0 / std::sqrt(std::fmax(1.0, 0.7 * std::log2((double)g.R + 1.0)));
    g.inv_n = 1.0 / (double)g.n;
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
    o.coltab = take(sizeof(float) * (size_t)(g.KA - 1) * g.cols);   // 2*rmax+1 rows, zero beyond K
    o.stats = take(sizeof(double) * 4 * g.R);
    o.bounds = take(sizeof(double) * 2 * g.R);
    o.gram = take(sizeof(double) * 4 * (size_t)g.R * g.R);
    o.gpart = take(sizeof(double) * (size_t)g.nblkg * (4 * (size_t)g.R * g.R + (size_t)g.K * g.K));
    o.counts = take(sizeof(unsigned long long) * (size_t)g.T * g.B);
    o.cooc = take(cooc_closed(g) ? sizeof(unsigned long long) * (size_t)cooc_pairs(g) * g.B * g.B : 0);
    o.bins = take((size_t)g.binbytes * (size_t)g.n);
    o.tbuf = take(sizeof(float) * (size_t)g.n);
    o.part = take(sizeof(double) * (size_t)NVMAX * std::max(g.nblk, g.nblk1));
    o.part1 = take(sizeof(double) * 2 * (size_t)g.nblk1);   // sweep 1's sums and maxima, read by every block of sweep 2
    o.sums = take(sizeof(double) * (size_t)NVMAX);
    o.hist = take(sizeof(unsigned long long) * (size_t)hist_words(g));   // low-word copies, then the high words
    // per-block histogram partials of the matrix-core sweeps (two or four tables of one-byte bins)
    o.hpart = take(mtables(g) ? sizeof(unsigned long long) * (size_t)g.T * g.B * g.nblk : 0);
    o.lt = take(sizeof(float) * (size_t)g.T * g.B);
    o.imp = take(sizeof(float) * (size_t)g.T * g.B);
    o.rowfx = take(sizeof(unsigned long long) * (size_t)g.rows);
    o.colfx = take(sizeof(unsigned long long) * (size_t)g.cols);
    o.colfac = take(sizeof(float) * (size_t)g.cols);
    int64_t sum_trail = 0;
    for (int a = 0; a < g.ntrail; ++a) sum_trail += g.tdim[a];
    o.terms = take(sizeof(float) * (size_t)std::max<int64_t>(1, sum_trail));
    o.ctrl = take(sizeof(Ctrl));
    o.desc = take(sizeof(cresso_spectral_desc));   // the tensor's descriptor in a batched step
    o.total = work == CRESSO_F64 ? plan_f64_layout(P, off) : off;
    return CRESSO_OK;
}

// The largest bin count of any table (data independent): with it the
// histograms' fixed-point scales keep every bin sum below 2^62.
__global__ void ws_cmax_kernel(const unsigned long long* __restrict__ counts, int64_t tb, int64_t n, int bins_off,
                               Ctrl* __restrict__ ctrl) {
    __shared__ unsigned long long s[256];
    unsigned long long m = 1;
    for (int64_t i = threadIdx.x; i < tb; i += blockDim.x) m = counts[i] > m ? counts[i] : m;
    s[threadIdx.x] = m;
    __syncthreads();
    for (int w = blockDim.x / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w && s[threadIdx.x + w] > s[threadIdx.x]) s[threadIdx.x] = s[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const unsigned long long c = bins_off ? (unsigned long long)n : s[0];
        ctrl->cmax = (double)c;
        ctrl->kq = 62 - (c > 1 ? 64 - __clzll((long long)(c - 1)) : 0);   // 62 - ceil(log2 cmax)
    }
}

__global__ void zero_u64_kernel(unsigned long long* p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0ull;
}

}  // namespace
}  // namespace cresso


using namespace cresso;

extern "C" cresso_spectral_plan* cresso_spectral_plan_create_ex(const int64_t* shape, int32_t ndim,
                                                                const int64_t* freqs, int32_t rank, int32_t hash_bins,
                                                                int32_t hash_tables, int32_t work_dtype) {
    if (!shape || !freqs) {
        fail(CRESSO_E_INVALID, "spectral route: null shape or freqs");
        return nullptr;
    }
    static std::atomic<uint64_t> next_serial{1};
    cresso_spectral_plan* P = new cresso_spectral_plan();
    if (plan_spectral(shape, ndim, freqs, rank, hash_bins, hash_tables, work_dtype, *P) != CRESSO_OK) {
        delete P;
        return nullptr;
    }
    P->serial = next_serial.fetch_add(1);
    return P;
}

extern "C" cresso_spectral_plan* cresso_spectral_plan_create(const int64_t* shape, int32_t ndim, const int64_t* freqs,
                                                             int32_t rank, int32_t hash_bins, int32_t hash_tables) {
    return cresso_spectral_plan_create_ex(shape, ndim, freqs, rank, hash_bins, hash_tables, CRESSO_F32);
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
    hipLaunchKernelGGL(ws_stats_kernel, dim3((unsigned)g.R), dim3(SP_FIN_NT), 0, s, g, meta, at<float>(ws, o.rowtab),
                       at<float>(ws, o.coltab), at<double>(ws, o.stats), at<double>(ws, o.bounds));
    hipLaunchKernelGGL(ws_pairsum_kernel, dim3((unsigned)g.nblkg), dim3(256), 0, s, g, at<float>(ws, o.rowtab),
                       at<float>(ws, o.coltab), at<double>(ws, o.gpart));
    const size_t gram_lds = sizeof(double) * (4 * (size_t)g.R * g.R + (size_t)g.K * g.K);
    if (gram_lds > 64 * 1024) {   // ranks above 16: up to 66.5 KB of pair sums (gfx950: 160 KB per workgroup)
        const hipError_t ea = hipFuncSetAttribute(reinterpret_cast<const void*>(&ws_gram_kernel),
                                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)gram_lds);
        if (ea != hipSuccess) return hip_fail(ea, "spectral route: Gram kernel LDS");
    }
    hipLaunchKernelGGL(ws_gram_kernel, dim3(1), dim3(SP_FIN_NT), gram_lds, s, g, meta, at<double>(ws, o.stats),
                       at<double>(ws, o.gpart), at<double>(ws, o.gram));
    const int64_t TB = (int64_t)g.T * g.B;
    hipLaunchKernelGGL(zero_u64_kernel, dim3((unsigned)((TB + 255) / 256)), dim3(256), 0, s, at<unsigned long long>(ws, o.counts), TB);
    hipLaunchKernelGGL(zero_u64_kernel, dim3((unsigned)((hist_words(g) + 255) / 256)), dim3(256), 0, s,
                       at<unsigned long long>(ws, o.hist), hist_words(g));
    const int64_t bins_blocks = std::max<int64_t>(1, std::min<int64_t>(2048, (g.n + 255) / 256));
    hipLaunchKernelGGL(ws_bins_kernel, dim3((unsigned)bins_blocks), dim3(256), 0, s, g, at<unsigned char>(ws, o.bins),
                       at<unsigned long long>(ws, o.counts));
    hipLaunchKernelGGL(ws_cmax_kernel, dim3(1), dim3(256), 0, s, at<unsigned long long>(ws, o.counts), TB, g.n,
                       P->bins_off, at<Ctrl>(ws, o.ctrl));
    if (cooc_closed(g)) {
        const int64_t BB = (int64_t)cooc_pairs(g) * g.B * g.B;
        hipLaunchKernelGGL(zero_u64_kernel, dim3((unsigned)((BB + 255) / 256)), dim3(256), 0, s,
                           at<unsigned long long>(ws, o.cooc), BB);
        if (g.T == 2)
            hipLaunchKernelGGL(ws_cooc_kernel, dim3((unsigned)bins_blocks), dim3(256), 0, s, g,
                               at<const uint16_t>(ws, o.bins), at<unsigned long long>(ws, o.cooc));
        else {
            // per-block tables in the (not yet used) tangent-field region: as
            // many blocks as fit, at most 256; few elements take the atomics
            const int64_t cells = 6 * (int64_t)g.B * g.B;
            const int64_t nb = std::min<int64_t>(256, (int64_t)(sizeof(float) * (size_t)g.n) / (cells * 4));
            static const hipError_t lds_ok = hipFuncSetAttribute(
                reinterpret_cast<const void*>(&ws_cooc4_part_kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                (int)(sizeof(unsigned int) * WS_COOC4_HALF));
            if (nb >= 16 && lds_ok == hipSuccess) {
                unsigned int* part = at<unsigned int>(ws, o.tbuf);
                const size_t lds = sizeof(unsigned int) * (size_t)std::min<int64_t>(WS_COOC4_HALF, (int64_t)g.B * g.B);
                hipLaunchKernelGGL(ws_cooc4_part_kernel, dim3((unsigned)nb), dim3(WS_COOC4_NT), lds, s, g,
                                   at<const uint32_t>(ws, o.bins), part);
                hipLaunchKernelGGL(ws_cooc4_sum_kernel, dim3((unsigned)((cells + 255) / 256)), dim3(256), 0, s, part,
                                   (int)nb, cells, at<unsigned long long>(ws, o.cooc));
            } else {
                hipLaunchKernelGGL(ws_cooc4_kernel, dim3((unsigned)bins_blocks), dim3(256), 0, s, g,
                                   at<const uint32_t>(ws, o.bins), at<unsigned long long>(ws, o.cooc));
            }
        }
    }
    e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "spectral route: workspace init");
    if (P->work == CRESSO_F64) {
        const int32_t rc = workspace_init_f64(*P, ws, s);
        if (rc != CRESSO_OK) return rc;
    }
    e = hipStreamSynchronize(s);
    return e == hipSuccess ? CRESSO_OK : hip_fail(e, "spectral route: workspace init");
}

namespace {
int32_t check_desc(const cresso_spectral_plan* P, const cresso_spectral_desc* d) {
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
    return CRESSO_OK;
}

// (param dtype, grad dtype) -> the unit that instantiates the step for it
SpectralRunFn find_run(int pt, int gt) {
    static const struct { int pt, gt; SpectralRunFn fn; } table[] = {
        {CRESSO_F32, CRESSO_F32, spectral_run_f32_f32},
        {CRESSO_BF16, CRESSO_BF16, spectral_run_bf16_bf16},
        {CRESSO_F16, CRESSO_F16, spectral_run_f16_f16},
        {CRESSO_F32, CRESSO_BF16, spectral_run_f32_bf16},
        {CRESSO_F32, CRESSO_F16, spectral_run_f32_f16},
    };
    for (const auto& e : table)
        if (e.pt == pt && e.gt == gt) return e.fn;
    fail(CRESSO_E_UNSUPPORTED, "spectral route: param/grad dtype pair (%d,%d) not supported by this build", pt, gt);
    return nullptr;
}

// Layout of a batched workspace: the plan's shape tables once, then `count`
// lanes, each a copy of the single workspace's per-step scratch (from tbuf to
// the end, its device copy of the tensor's descriptor included).
size_t lane_stride(const cresso_spectral_plan* P) { return P->o.total - P->o.tbuf; }
size_t batched_bytes(const cresso_spectral_plan* P, int count) { return P->o.tbuf + (size_t)count * lane_stride(P); }

// The descriptors travel to the device as kernel arguments, DESC_CHUNK per
// launch (no staging buffer, no host synchronization).
constexpr int DESC_CHUNK = 16;
struct DescChunk {
    cresso_spectral_desc d[DESC_CHUNK];
};
static_assert(sizeof(DescChunk) + 16 <= 4096, "descriptor chunk exceeds the kernel argument limit");
static_assert(sizeof(cresso_spectral_desc) % 8 == 0, "descriptor copied as 64-bit words");
__global__ __launch_bounds__(256) void put_descs_kernel(DescChunk c, int n, unsigned char* __restrict__ dst, size_t ls) {
    constexpr int W = (int)(sizeof(cresso_spectral_desc) / 8);
    const unsigned long long* src = reinterpret_cast<const unsigned long long*>(&c.d[0]);
    for (int i = threadIdx.x; i < n * W; i += blockDim.x)
        reinterpret_cast<unsigned long long*>(dst + (size_t)(i / W) * ls)[i % W] = src[i];
}

// Lanes 1.. of a batched workspace start as lane 0 after its set-up: the same
// control block (its data-independent scale bound) and cleared histograms.
__global__ __launch_bounds__(256) void ws_lanes_kernel(unsigned char* __restrict__ lane0, size_t ls, size_t ctrl_off,
                                                       size_t hist_off, int64_t tb) {
    unsigned char* ln = lane0 + (size_t)(blockIdx.x + 1) * ls;
    const unsigned long long* c0 = reinterpret_cast<const unsigned long long*>(lane0 + ctrl_off);
    unsigned long long* c = reinterpret_cast<unsigned long long*>(ln + ctrl_off);
    for (int i = threadIdx.x; i < (int)(sizeof(Ctrl) / 8); i += blockDim.x) c[i] = c0[i];
    unsigned long long* hh = reinterpret_cast<unsigned long long*>(ln + hist_off);
    for (int64_t i = threadIdx.x; i < tb; i += blockDim.x) hh[i] = 0ull;
}
static_assert(sizeof(Ctrl) % 8 == 0, "control block copied as 64-bit words");

}  // namespace

extern "C" int32_t cresso_spectral_step(const cresso_spectral_plan* P, const cresso_spectral_desc* d, void* ws,
                                        size_t ws_bytes, const cresso_hyper* hyper, void* stream) {
    if (!P || !d || !ws || !hyper) return fail(CRESSO_E_INVALID, "spectral route: null argument");
    if (ws_bytes < P->o.total) return fail(CRESSO_E_INVALID, "spectral route: workspace too small");
    const int32_t rc = check_desc(P, d);
    if (rc != CRESSO_OK) return rc;
    if (!(hyper->drive_clip > 0.0)) return fail(CRESSO_E_INVALID, "spectral route: drive_clip must be positive");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (d->param_dtype == CRESSO_F64 || P->work == CRESSO_F64) {
        if (d->param_dtype != CRESSO_F64 || d->grad_dtype != CRESSO_F64 || P->work != CRESSO_F64)
            return fail(CRESSO_E_INVALID, "spectral route: fp64 params and grads need a plan with the fp64 work dtype "
                        "(cresso_spectral_plan_create_ex(..., CRESSO_F64)), and such a plan steps fp64 tensors only");
        return spectral_run_f64(*P, *d, ws, *hyper, s);
    }
    const SpectralRunFn fn = find_run(d->param_dtype, d->grad_dtype);
    if (!fn) return CRESSO_E_UNSUPPORTED;
    return fn(*P, d, 1, nullptr, 0, ws, *hyper, s);
}

extern "C" size_t cresso_spectral_batched_workspace_bytes(const cresso_spectral_plan* P, int32_t count) {
    return P && count >= 1 && P->work == CRESSO_F32 ? batched_bytes(P, count) : 0;
}

extern "C" int32_t cresso_spectral_batched_workspace_init(const cresso_spectral_plan* P, int32_t count, void* ws,
                                                          size_t ws_bytes, const cresso_hyper* hyper, void* stream) {
    if (!P || !ws || !hyper) return fail(CRESSO_E_INVALID, "spectral route: null argument");
    if (count < 1) return fail(CRESSO_E_INVALID, "spectral route: batch of %d tensors", count);
    if (P->work != CRESSO_F32)
        return fail(CRESSO_E_UNSUPPORTED, "spectral route: fp64 plans step one tensor at a time (cresso_spectral_step)");
    if (ws_bytes < batched_bytes(P, count))
        return fail(CRESSO_E_INVALID, "spectral route: batched workspace of %zu bytes is smaller than %zu", ws_bytes,
                    batched_bytes(P, count));
    int32_t rc = cresso_spectral_workspace_init(P, ws, P->o.total, hyper, stream);
    if (rc != CRESSO_OK || count == 1) return rc;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const Offs& o = P->o;
    hipLaunchKernelGGL(ws_lanes_kernel, dim3((unsigned)(count - 1)), dim3(256), 0, s, at<unsigned char>(ws, o.tbuf),
                       lane_stride(P), o.ctrl - o.tbuf, o.hist - o.tbuf, hist_words(P->g));
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    return e == hipSuccess ? CRESSO_OK : hip_fail(e, "spectral route: batched workspace init");
}

extern "C" int32_t cresso_spectral_step_batched(const cresso_spectral_plan* P, const cresso_spectral_desc* descs,
                                                int32_t count, void* ws, size_t ws_bytes, const cresso_hyper* hyper,
                                                void* stream) {
    if (!P || !descs || !ws || !hyper) return fail(CRESSO_E_INVALID, "spectral route: null argument");
    if (count < 1) return fail(CRESSO_E_INVALID, "spectral route: batch of %d tensors", count);
    if (ws_bytes < batched_bytes(P, count))
        return fail(CRESSO_E_INVALID, "spectral route: batched workspace too small for %d tensors", count);
    if (!(hyper->drive_clip > 0.0)) return fail(CRESSO_E_INVALID, "spectral route: drive_clip must be positive");
    const cresso_spectral_desc& d0 = descs[0];
    if (d0.param_dtype == CRESSO_F64 || P->work != CRESSO_F32)
        return fail(CRESSO_E_UNSUPPORTED, "spectral route: fp64 params step one tensor at a time (cresso_spectral_step)");
    for (int i = 0; i < count; ++i) {
        const cresso_spectral_desc& d = descs[i];
        const int32_t rc = check_desc(P, &d);
        if (rc != CRESSO_OK) return rc;
        if (d.param_dtype != d0.param_dtype || d.grad_dtype != d0.grad_dtype)
            return fail(CRESSO_E_INVALID, "spectral route: tensor %d of a batch has other dtypes than tensor 0", i);
        if ((d.hard != 0) != (d0.hard != 0) || (d.hash_energy != nullptr) != (d0.hash_energy != nullptr))
            return fail(CRESSO_E_INVALID, "spectral route: tensor %d of a batch differs from tensor 0 in the hard "
                        "channel or the hash state", i);
    }
    const SpectralRunFn fn = find_run(d0.param_dtype, d0.grad_dtype);
    if (!fn) return CRESSO_E_UNSUPPORTED;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const size_t ls = lane_stride(P);
    for (int i0 = 0; i0 < count; i0 += DESC_CHUNK) {
        DescChunk c;
        const int n = std::min(DESC_CHUNK, count - i0);
        std::memset(&c, 0, sizeof(c));
        std::memcpy(&c.d[0], descs + i0, sizeof(cresso_spectral_desc) * (size_t)n);
        hipLaunchKernelGGL(put_descs_kernel, dim3(1), dim3(256), 0, s, c, n, at<unsigned char>(ws, P->o.desc + i0 * ls), ls);
    }
    return fn(*P, descs, count, at<cresso_spectral_desc>(ws, P->o.desc), ls, ws, *hyper, s);
}

// ---------------------------------------------------------------------------
// cresso_spectral_step_noalloc: the step above with its workspace (carrier
// tables, bins, tangent field and per-step scratch) in a static device array,
// for callers that cannot allocate.  Each GPU the library runs on holds its
// own copy of `scratch` until the process ends.  The array keeps the last
// call's contents: a call whose plan differs from the one whose tables the
// device's copy holds first rebuilds the tables (and clears the histogram
// and count regions) exactly as cresso_spectral_workspace_init does.  Calls
// that overlap on one GPU (two streams, or two host threads) share the array
// and race.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[CRESSO_SPECTRAL_NOALLOC_MAX_BYTES];

namespace {
constexpr int kNoallocMaxDev = 64;
std::mutex g_noalloc_mu;
void* g_noalloc_ptr[kNoallocMaxDev];       // device address of `scratch` per device (hipGetSymbolAddress)
uint64_t g_noalloc_plan[kNoallocMaxDev];   // serial of the plan whose tables that copy holds (0: none)
}  // namespace

extern "C" int32_t cresso_spectral_step_noalloc(const cresso_spectral_plan* P, const cresso_spectral_desc* d,
                                                const cresso_hyper* hyper, void* stream) {
    if (!P || !d || !hyper) return fail(CRESSO_E_INVALID, "spectral route (no-alloc): null argument");
    const size_t need = P->o.total;
    if (need > (size_t)CRESSO_SPECTRAL_NOALLOC_MAX_BYTES)
        return fail(CRESSO_E_INVALID,
                    "spectral route (no-alloc): this plan needs %zu bytes of workspace, above the %zu-byte static "
                    "scratch; use cresso_spectral_step with a caller-allocated workspace",
                    need, (size_t)CRESSO_SPECTRAL_NOALLOC_MAX_BYTES);
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "spectral route (no-alloc): hipGetDevice");
    if (dev < 0 || dev >= kNoallocMaxDev)
        return fail(CRESSO_E_UNSUPPORTED, "spectral route (no-alloc): device %d outside 0..%d", dev, kNoallocMaxDev - 1);
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (!g_noalloc_ptr[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) return hip_fail(e, "spectral route (no-alloc): hipGetSymbolAddress(scratch)");
        g_noalloc_ptr[dev] = ptr;
    }
    void* ws = g_noalloc_ptr[dev];
    if (g_noalloc_plan[dev] != P->serial) {
        // the rebuild copies from host memory and synchronizes the stream,
        // which a stream under graph capture cannot do: refuse before any work
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(reinterpret_cast<hipStream_t>(stream), &cap);
        if (e != hipSuccess) return hip_fail(e, "spectral route (no-alloc): hipStreamIsCapturing");
        if (cap != hipStreamCaptureStatusNone)
            return fail(CRESSO_E_INVALID,
                        "spectral route (no-alloc): the stream is capturing a graph and this plan's tables are not "
                        "resident in the device's static scratch; make one uncaptured call with this plan first");
        g_noalloc_plan[dev] = 0;   // tables unknown until the rebuild below succeeds
        const int32_t rc = cresso_spectral_workspace_init(P, ws, need, hyper, stream);
        if (rc != CRESSO_OK) return rc;
        g_noalloc_plan[dev] = P->serial;
    }
    return cresso_spectral_step(P, d, ws, need, hyper, stream);
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

extern "C" int32_t cresso_spectral_workspace_project(const cresso_spectral_plan* P, void* ws, size_t ws_bytes,
                                                     const float* x, double* out, void* stream) {
    if (!P || !ws || !x || !out) return fail(CRESSO_E_INVALID, "spectral route: null argument");
    if (ws_bytes < P->o.total) return fail(CRESSO_E_INVALID, "spectral route: workspace too small");
    const Geom& g = P->g;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    // the step's partial and sum regions are the scratch (stream order keeps
    // this call and the steps apart)
    const int64_t blocks = std::max<int64_t>(
        1, std::min<int64_t>(std::min<int64_t>(1024, std::max(g.nblk, g.nblk1)), (g.n + 255) / 256));
    double* part = at<double>(ws, P->o.part);
    double* sums = at<double>(ws, P->o.sums);
    hipLaunchKernelGGL(ws_project_kernel, dim3((unsigned)blocks), dim3(256), 0, s, g, at<ModeMeta>(ws, P->o.meta),
                       at<float>(ws, P->o.rowtab), at<float>(ws, P->o.coltab), at<double>(ws, P->o.stats), x, part);
    hipLaunchKernelGGL(part_reduce_kernel, dim3((unsigned)(2 * g.R)), dim3(256), 0, s, part, (int)blocks, 2 * g.R, sums,
                       nullptr, nullptr, 0, Lanes{nullptr, 0});
    hipLaunchKernelGGL(ws_mean_kernel, dim3(1), dim3(64), 0, s, sums, 2 * g.R, 1.0 / (double)g.n, out);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? CRESSO_OK : hip_fail(e, "spectral route: workspace project");
}

extern "C" int32_t cresso_spectral_workspace_reconstruct(const cresso_spectral_plan* P, const void* ws, size_t ws_bytes,
                                                         const float* cc, const float* sc, const float* gates,
                                                         float* out, void* stream) {
    if (!P || !ws || !cc || !sc || !out) return fail(CRESSO_E_INVALID, "spectral route: null argument");
    if (ws_bytes < P->o.total) return fail(CRESSO_E_INVALID, "spectral route: workspace too small");
    const Geom& g = P->g;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    void* w = const_cast<void*>(ws);
    const double shrink = 1.0 / std::sqrt(std::max(1.0, 0.7 * std::log2((double)g.R + 1.0)));
    const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(4096, (g.n + 255) / 256));
    hipLaunchKernelGGL(ws_reconstruct_kernel, dim3((unsigned)blocks), dim3(256), 0, s, g, at<ModeMeta>(w, P->o.meta),
                       at<float>(w, P->o.rowtab), at<float>(w, P->o.coltab), at<double>(w, P->o.stats), cc, sc, gates,
                       shrink, out);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? CRESSO_OK : hip_fail(e, "spectral route: workspace reconstruct");
}

extern "C" int32_t cresso_spectral_workspace_gram(const cresso_spectral_plan* P, const void* ws, size_t ws_bytes,
                                                  double* gram_out, void* stream) {
    if (!P || !ws || !gram_out) return fail(CRESSO_E_INVALID, "spectral route: null argument");
    if (ws_bytes < P->o.total) return fail(CRESSO_E_INVALID, "spectral route: workspace too small");
    const size_t V = 2 * (size_t)P->g.R;
    hipError_t e = hipMemcpyAsync(gram_out, at<double>(const_cast<void*>(ws), P->o.gram), sizeof(double) * V * V,
                                  hipMemcpyDeviceToDevice, reinterpret_cast<hipStream_t>(stream));
    return e == hipSuccess ? CRESSO_OK : hip_fail(e, "spectral route: workspace gram");
}
