// kmeans.hip -- Lloyd k-means on one GPU behind the C ABI.
//
// Replaces CudaKMeansEngine::fit_gpu (vector-cuda/src/kmeans.rs:99-237) and the kernels of
// kmeans.cu.  One iteration is:
//   1. assign   -- fused distance + argmin (MFMA tiles for L2 / dot / cosine in knn_gemm.hip,
//                  VALU tiles for the other metrics in knn_valu.hip); each point also takes an
//                  atomic ticket pos[p] in its cluster's count (integer atomics: exact).  For
//                  squared L2 the points and centroids are held minus a per-dimension shift (the
//                  column means of the points, integers for integer data), which keeps the
//                  GEMM form well conditioned on data away from the origin.  The MFMA assignment
//                  is certified: a point whose best and second-best scores are not separated by
//                  twice its selection error bound goes to a fix-up list instead, and
//   2. fix-up   -- assigns the listed points by the direct-form metric of the unshifted data over
//                  all centroids (knn_valu.hip), so every assignment is the argmin of the direct
//                  form the reference computes (lowest index among equal values);
//   3. scan     -- exclusive scan of the k counts into segment offsets;
//   4. scatter  -- point indices into their cluster segment at offsets[c] + pos[p];
//   5. sums     -- every wave walks a fixed 256-slot window of the cluster-sorted order and adds
//                  the deviations x - c_old of its rows in 64-bit fixed point; at each cluster
//                  boundary it adds the partial sum into the cluster's 64-bit accumulators with
//                  integer atomics.  Integer addition is associative, so the sums -- and every
//                  centroid -- are bit-identical whatever order the atomics handed out the slots
//                  or the windows were scheduled (the reference's float atomics,
//                  kmeans.cu:298-320, and rayon fold, ivf/kmeans.rs:75-118, are
//                  order-dependent).  Each cluster has its own scale 2^E, from its point count and
//                  a bound of its points' deviations, so no sum can overflow and the resolution is
//                  relative to the cluster's own spread (a tight cluster near the origin keeps full
//                  precision next to wide clusters far away).  The same pass writes each point's
//                  squared-L2 inertia in direct form;
//   6. finalize -- one wave per cluster: new = old + deviation sum / count; shift =
//                  sum_d (new - old)^2; an empty cluster keeps its centroid with shift 0
//                  (kmeans.cu:350-356); the accumulators are cleared for the next iteration;
//   7. prepare  -- the centroids' assign rows (shifted), norms and bounds for the next assign.
// With tol < 0 no per-iteration host synchronisation happens.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>

#include "vh_runtime.h"

namespace vh {

bool is_gemm_metric(int m);

// ---- kernels ---------------------------------------------------------------------------
__global__ void k_absmax_partial(const float *__restrict__ x, size_t count, float *__restrict__ partial) {
    __shared__ float red[256];
    float m = 0.0f;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < count; i += (size_t)gridDim.x * blockDim.x)
        m = fmaxf(m, fabsf(x[i]));
    red[threadIdx.x] = m;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + o]);
        __syncthreads();
    }
    if (threadIdx.x == 0) partial[blockIdx.x] = red[0];
}

// Exclusive scan of counts[k] into offsets[k+1]; one workgroup of 1024 threads.
__global__ __launch_bounds__(1024) void k_scan_counts(const int32_t *__restrict__ counts, int k,
                                                      int32_t *__restrict__ offsets) {
    __shared__ int32_t part[1024];
    const int t = threadIdx.x;
    const int per = (k + 1023) / 1024;
    const int b = t * per, e = min(k, b + per);
    int32_t s = 0;
    for (int i = b; i < e; ++i) s += counts[i];
    part[t] = s;
    __syncthreads();
    for (int o = 1; o < 1024; o <<= 1) {
        const int32_t v = t >= o ? part[t - o] : 0;
        __syncthreads();
        part[t] += v;
        __syncthreads();
    }
    int32_t run = t > 0 ? part[t - 1] : 0;
    for (int i = b; i < e; ++i) {
        offsets[i] = run;
        run += counts[i];
    }
    if (t == 1023) offsets[k] = part[1023];
}

__global__ void k_scatter(const int32_t *__restrict__ assign, const int32_t *__restrict__ pos,
                          const int32_t *__restrict__ offsets, int n, int32_t *__restrict__ sorted) {
    const int p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p < n) sorted[offsets[assign[p]] + pos[p]] = p;
}

// ---- update ----------------------------------------------------------------------------
constexpr int kUpdSlotsPerWave = 256;  // sorted slots per wave window
constexpr int kUpdMinSlots = 16;       // the window halves down to this while the waves number
constexpr int kUpdMinWaves = 2048;     // fewer than this

// Largest c in [0, k) with offsets[c] <= i: the (non-empty) cluster whose segment holds slot i.
__device__ __forceinline__ int segment_of(const int32_t *__restrict__ offsets, int k, int i) {
    int lo = 0, hi = k - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (offsets[mid] <= i) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// Fixed-point exponent of each cluster: with every |x_d - c_d| < 2^e1 and count + 1 < 2^e2,
// a deviation sum times 2^E stays below 2^61 for E = 61 - e1 - e2 (at most 60).
__global__ void k_update_scales(int k, const float *__restrict__ devmax, const int32_t *__restrict__ counts,
                                int32_t *__restrict__ exps) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= k) return;
    int E = 60;
    const float dm = devmax[c];
    if (dm > 0.0f && counts[c] > 0) {
        int e1, e2;
        (void)frexpf(dm, &e1);
        (void)frexp((double)counts[c] + 1.0, &e2);
        E = min(60, 61 - e1 - e2);
    }
    exps[c] = E;
}

// Deviation bound of the metrics whose assignment keeps no distance: max|x| + max_d |c_d|.
__global__ void k_dev_bound(int k, float absmax, const float *__restrict__ cabs, float *__restrict__ devmax) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c < k) devmax[c] = (absmax + cabs[c]) * 1.0001f;
}

// S = number of 64-dimension slots per lane (dpad <= 64 * S).  Lane l of a wave owns dimensions
// l, l + 64, ...; the wave adds the deviations x - c of the rows of its window (spw sorted
// slots; integer sums, so the window size does not change them) slot by slot in
// fixed point (the cluster's scale) and flushes the running sum into sums[c] whenever the window
// crosses into the next cluster's segment.  It also writes each point's value against the centroid
// its assignment used, in direct form (lane-strided sums, fixed xor butterfly), by `inertia_mode`:
// 1 the squared distance sum_d (x_d - c_d)^2, 2 -x.c, 3 1 - x.c / (||x|| ||c||) (0 below the
// 1e-9 guard; pnorm and cnorm hold the L2 norms), 0 none (the assignment wrote it).  Lane-strided
// partial sums keep these values exact-to-rounding where a sequential sum drifts: adding odd
// squares to an even running sum above 2^24 rounds each of them down, so a point's product with
// itself as a centroid came out about 6e-6 short of its norm squared at 1024 dimensions of
// integers in [0, 255].
template <int S>
constexpr int upd_unroll() { return S >= 8 ? 4 : (S >= 4 ? 8 : 16); }  // rows in flight per wave

template <int S>
__global__ __launch_bounds__(256) void k_update_sums(const float *__restrict__ pts, const float *__restrict__ cent,
                                                     int dpad, int dim, int n, int k,
                                                     const int32_t *__restrict__ sorted,
                                                     const int32_t *__restrict__ offsets,
                                                     const int32_t *__restrict__ exps,
                                                     unsigned long long *__restrict__ sums, float *__restrict__ inertia,
                                                     int inertia_mode, const float *__restrict__ pnorm,
                                                     const float *__restrict__ cnorm, int spw) {
    constexpr int kUpdUnroll = upd_unroll<S>();
    const int lane = threadIdx.x & 63;
    const int wave = (int)((blockIdx.x * (size_t)blockDim.x + threadIdx.x) >> 6);
    const int s0 = wave * spw;
    if (s0 >= n) return;
    const int s1 = min(n, s0 + spw);
    int c = segment_of(offsets, k, s0);
    int next = offsets[c + 1];
    long long acc[S];
    float cv[S];
    double scale = 1.0;
    auto load_c = [&](int cc) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int d = lane + 64 * s;
            cv[s] = d < dpad ? cent[(size_t)cc * dpad + d] : 0.0f;
        }
        scale = ldexp(1.0, exps[cc]);
    };
#pragma unroll
    for (int s = 0; s < S; ++s) acc[s] = 0;
    load_c(c);
    auto flush = [&](int cc) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int d = lane + 64 * s;
            if (d < dim && acc[s] != 0)
                atomicAdd(sums + (size_t)cc * dpad + d, (unsigned long long)acc[s]);
            acc[s] = 0;
        }
    };
    for (int b = s0; b < s1; b += 64) {
        const int nb = min(64, s1 - b);
        const int mine = lane < nb ? sorted[b + lane] : 0;
        for (int j = 0; j < nb; j += kUpdUnroll) {
            float v[kUpdUnroll][S];
#pragma unroll
            for (int u = 0; u < kUpdUnroll; ++u) {
                const int p = __builtin_amdgcn_readlane(mine, j + u);
                const bool live = j + u < nb;
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    const int d = lane + 64 * s;
                    v[u][s] = (live && d < dpad) ? pts[(size_t)p * dpad + d] : 0.0f;
                }
            }
#pragma unroll
            for (int u = 0; u < kUpdUnroll; ++u) {
                const int i = b + j + u;
                if (i < s1) {
                    if (i >= next) {
                        while (i >= next) {  // offsets[k] = n > i, so c stays below k
                            flush(c);
                            ++c;
                            next = offsets[c + 1];
                        }
                        load_c(c);
                    }
                    float d2 = 0.0f, xc = 0.0f;
#pragma unroll
                    for (int s = 0; s < S; ++s) {
                        acc[s] += llrint(((double)v[u][s] - (double)cv[s]) * scale);
                        const float t = v[u][s] - cv[s];
                        d2 = fmaf(t, t, d2);
                        xc = fmaf(v[u][s], cv[s], xc);
                    }
                    if (inertia_mode) {
                        float r = inertia_mode == 1 ? d2 : xc;
#pragma unroll
                        for (int o = 32; o > 0; o >>= 1) r += __shfl_xor(r, o, 64);
                        const int p = __builtin_amdgcn_readlane(mine, j + u);
                        if (inertia_mode == 2) {
                            r = -r + 0.0f;
                        } else if (inertia_mode == 3) {
                            const float den = pnorm[p] * cnorm[c];
                            r = 1.0f + (den > 1e-9f ? -(r / den) + 0.0f : 0.0f);
                        }
                        if (lane == 0) inertia[p] = r;
                    }
                }
            }
        }
    }
    flush(c);
}

// One wave per cluster: new = old + deviation sum / (2^E count), shift, and the accumulators are
// cleared for the next iteration.  `cent` holds the unshifted centroids.
template <int S>
__global__ __launch_bounds__(256) void k_update_finalize(int k, int dpad, int dim, unsigned long long *__restrict__ sums,
                                                         const int32_t *__restrict__ counts,
                                                         const int32_t *__restrict__ exps, float *__restrict__ cent,
                                                         float *__restrict__ shifts) {
    const int lane = threadIdx.x & 63;
    const int c = (int)((blockIdx.x * (size_t)blockDim.x + threadIdx.x) >> 6);
    if (c >= k) return;
    const int cnt = counts[c];
    const double inv = cnt > 0 ? ldexp(1.0, -exps[c]) / (double)cnt : 0.0;
    float sh = 0.0f;
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int d = lane + 64 * s;
        if (d < dim) {
            unsigned long long *sp = sums + (size_t)c * dpad + d;
            const long long sum = (long long)*sp;
            *sp = 0ull;
            if (cnt > 0) {
                float *cp = cent + (size_t)c * dpad + d;
                const float old = *cp;
                const float nv = (float)((double)old + (double)sum * inv);
                const float diff = nv - old;
                sh = fmaf(diff, diff, sh);
                *cp = nv;
            }
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sh += __shfl_xor(sh, o, 64);
    if (lane == 0) shifts[c] = cnt > 0 ? sh : 0.0f;
}

// Assign rows of the centroids, one wave per row of kpad: cent = craw - shift (shift may be
// null), the norm of that row (norm_kind 1 squared, 2 plain; deterministic lane-strided sum and
// xor butterfly), max_d |craw_d| (cabs), and the largest norm value (cmax, u32 bits of a
// non-negative float, atomic max; cleared by the caller).  Rows past k are NaN, or with pad_big
// (squared L2) zero rows of norm FLT_MAX, whose assign scores are FLT_MAX (finite, so they never
// disturb the best / second-best tracking).
__global__ __launch_bounds__(256) void k_cent_prep(int k, int kpad, int dpad, const float *__restrict__ craw,
                                                   const float *__restrict__ shift, float *__restrict__ cent,
                                                   float *__restrict__ cnorm, int norm_kind, int pad_big,
                                                   float *__restrict__ cabs, uint32_t *__restrict__ cmax) {
    const int lane = threadIdx.x & 63;
    const int c = (int)((blockIdx.x * (size_t)blockDim.x + threadIdx.x) >> 6);
    if (c >= kpad) return;
    float *orow = cent + (size_t)c * dpad;
    if (c >= k) {
        for (int d = lane; d < dpad; d += 64) orow[d] = pad_big ? 0.0f : __builtin_nanf("");
        if (lane == 0) cnorm[c] = pad_big ? 0x1.fffffep127f : __builtin_nanf("");
        return;
    }
    float ss = 0.0f, am = 0.0f;
    for (int d = lane; d < dpad; d += 64) {
        const float x = craw[(size_t)c * dpad + d];
        const float v = shift ? x - shift[d] : x;
        orow[d] = v;
        ss = fmaf(v, v, ss);
        am = fmaxf(am, fabsf(x));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        ss += __shfl_xor(ss, o, 64);
        am = fmaxf(am, __shfl_xor(am, o, 64));
    }
    if (lane == 0) {
        const float nv = norm_kind == 2 ? sqrtf(ss) : ss;
        cnorm[c] = nv;
        cabs[c] = am;
        if (norm_kind) atomicMax(cmax, __float_as_uint(nv));
    }
}

// Deterministic sum: block b sums its contiguous range in double with a fixed tree.
__global__ void k_sum_partial(const float *__restrict__ v, size_t count, size_t chunk, double *__restrict__ partial) {
    __shared__ double red[256];
    const size_t b0 = blockIdx.x * chunk, e0 = min(count, b0 + chunk);
    double s = 0.0;
    for (size_t i = b0 + threadIdx.x; i < e0; i += blockDim.x) s += (double)v[i];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) partial[blockIdx.x] = red[0];
}

// Direct-form metric of each point and its assigned centroid, and optionally the residual
// x - c: the value KMeans::find_nearest_centroid returns (ivf/kmeans.rs:262-309: the engine's
// squared L2, dot product, cosine similarity, ... with the formulas of scalar.rs:14-263) and the
// residual IvfPqIndex::build computes for PQ training (ivf/mod.rs:119-132).  One wave per point:
// a lane-strided sum over the dimensions and a fixed xor butterfly (max for Chebyshev).
__global__ __launch_bounds__(256) void k_coarse_score(const float *__restrict__ pts, int dpad, int dim, int n,
                                                      const float *__restrict__ cent,
                                                      const int32_t *__restrict__ assign, int metric,
                                                      float *__restrict__ score, float *__restrict__ resid) {
    const int lane = threadIdx.x & 63;
    const size_t wave = (blockIdx.x * (size_t)blockDim.x + threadIdx.x) >> 6;
    const size_t nwaves = (gridDim.x * (size_t)blockDim.x) >> 6;
    for (size_t p = wave; p < (size_t)n; p += nwaves) {
        const float *x = pts + p * (size_t)dpad;
        const float *c = cent + (size_t)assign[p] * dpad;
        float a = 0.0f, b = 0.0f, e = 0.0f;
        for (int d = lane; d < dim; d += 64) {
            const float xv = x[d], cv = c[d];
            if (resid) resid[p * (size_t)dim + d] = xv - cv;
            switch (metric) {
                case DOT: a = fmaf(xv, cv, a); break;
                case COS:
                    a = fmaf(xv, cv, a);
                    b = fmaf(xv, xv, b);
                    e = fmaf(cv, cv, e);
                    break;
                case L1: a += fabsf(xv - cv); break;
                case MINK: {
                    const float t = fabsf(xv - cv);
                    a = fmaf(t * t, t, a);
                    break;
                }
                case LINF: a = fmaxf(a, fabsf(xv - cv)); break;
                case HAMF: a += fabsf(xv - cv) > 1e-6f ? 1.0f : 0.0f; break;
                case JACC: {
                    const float ax = fabsf(xv), ac = fabsf(cv);
                    a += fminf(ax, ac);
                    b += fmaxf(ax, ac);
                    break;
                }
                case HELL: {
                    const float t = sqrtf(fabsf(xv)) - sqrtf(fabsf(cv));
                    a = fmaf(t, t, a);
                    break;
                }
                default: {  // L2, MAHA
                    const float t = xv - cv;
                    a = fmaf(t, t, a);
                }
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float oa = __shfl_xor(a, o, 64);
            a = metric == LINF ? fmaxf(a, oa) : a + oa;
            b += __shfl_xor(b, o, 64);
            e += __shfl_xor(e, o, 64);
        }
        if (lane == 0) {
            float v;
            switch (metric) {
                case COS: {
                    const float den = sqrtf(b) * sqrtf(e);
                    v = den <= 1e-9f ? 0.0f : a / den;
                    break;
                }
                case MINK: v = cbrtf(a); break;
                case MAHA: v = sqrtf(a); break;
                case JACC: v = b <= 1e-9f ? 0.0f : 1.0f - a / b; break;
                case HELL: v = sqrtf(0.5f * a); break;
                default: v = a;
            }
            score[p] = v;
        }
    }
}

// Seeded k-means++ on the device (CudaKMeansEngine::init_random, kmeans.rs:409-460).  Each step
// is two or three launches on the state's stream, with no host round trip:
//  * k_kpp_dcc: the squared distance from the newest centre to every earlier one (only when the
//    update prunes);
//  * an update: mind[i] = min(mind[i], ||x_i - c||^2) for the newest centre c, in direct form,
//    and the sum of mind over each block of points (double, fixed order).  A point whose nearest
//    centre so far, a = near[i], lies at ||c_a - c||^2 >= 4 mind[i] (1 + margin) from c cannot
//    come closer to c (triangle inequality: ||x - c|| >= ||c_a - c|| - ||x - c_a|| >=
//    ||x - c_a||), so a pruning update does not read its row; the margin covers the rounding of
//    all three computed squared distances, so the values of mind are exactly those of the
//    unpruned pass.  k_kpp_update serves large point sets: blocks of kKppBlock points, eight
//    lanes a row (each a 16-byte column slice), so each load instruction of a wave reads eight
//    whole 128-byte row pieces.  k_kpp_update_rows serves point sets below kKppRowsMaxN: L lanes
//    a row (L = 8 .. 64 by dimension, so a lane loads at most four 16-byte slices of a row of up
//    to 1024 floats), blocks of 4 (64 / L) `passes` points, so that a small set still spreads
//    over thousands of waves; it prunes only when the points exceed the cache (kKppPruneFloats);
//  * k_kpp_select: one workgroup draws the next centre with probability mind[i] / sum(mind), as
//    the reference's linear scan does (the first i whose running sum reaches u * total), through
//    the block sums and then the chosen block's values, and copies that point into the centres.
// Every sum is in a fixed order, so a seed gives the same centres on every run.
constexpr int kKppBlock = 1024;          // points per k_kpp_update block (256 threads)
constexpr int kKppSelectThreads = 1024;  // at least the points of a block: the select reads one value per thread
constexpr int kKppRowsMaxN = 1 << 20;    // k_kpp_update_rows below this many points
constexpr int kKppRowsMaxBlocks = 4096;  // its blocks per step (the select sums at most 4 per thread)
constexpr size_t kKppPruneFloats = size_t(1) << 24;  // point floats above which k_kpp_update_rows prunes

__device__ __forceinline__ float acc_d2(float d2, float4 x, float4 c) {
    const float a0 = x.x - c.x, a1 = x.y - c.y, a2 = x.z - c.z, a3 = x.w - c.w;
    d2 = fmaf(a0, a0, d2);
    d2 = fmaf(a1, a1, d2);
    d2 = fmaf(a2, a2, d2);
    return fmaf(a3, a3, d2);
}

// ||x - c||^2 over nc4 float4 columns, split over a group of L lanes (sub: this lane's index in
// the group; its columns are sub, sub + L, ...).  Every lane of the group returns the sum.  Four
// column slices are loaded before any is used; a slice past the row end loads the last one (in
// bounds) and is not added.
template <int L>
__device__ __forceinline__ float group_d2(const float4 *__restrict__ x, const float4 *__restrict__ c, int nc4,
                                          int sub) {
    float d2 = 0.0f;
    for (int j = sub; j < nc4; j += 4 * L) {
        float4 xv[4], cv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int jj = min(j + u * L, nc4 - 1);
            xv[u] = x[jj];
            cv[u] = c[jj];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (j + u * L < nc4) d2 = acc_d2(d2, xv[u], cv[u]);
    }
#pragma unroll
    for (int o = L / 2; o > 0; o >>= 1) d2 += __shfl_xor(d2, o, 64);
    return d2;
}

// Lanes per row for a row of nc4 float4 columns.
inline int kpp_lanes(int nc4) { return nc4 <= 32 ? 8 : nc4 <= 64 ? 16 : nc4 <= 128 ? 32 : 64; }

// dcc[a] = ||c_a - c_m||^2 for the m earlier centres, L lanes per centre.
template <int L>
__global__ __launch_bounds__(256) void k_kpp_dcc(const float *__restrict__ cent, int dpad, int m,
                                                 float *__restrict__ dcc) {
    constexpr int R = 64 / L;
    const int lane = threadIdx.x & 63;
    const int a = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R + lane / L;
    const int ac = min(a, m - 1);  // rows past the end repeat the last one, unstored
    const float v = group_d2<L>((const float4 *)(cent + (size_t)ac * dpad), (const float4 *)(cent + (size_t)m * dpad),
                                dpad >> 2, lane & (L - 1));
    if (a < m && (lane & (L - 1)) == 0) dcc[a] = v;
}

// cidx: the newest centre's index (its row is c); prune: 4 (1 + margin), or 0 for no pruning.
// Each wave owns 256 consecutive points of the block.  It first tests all of them (lane l: points
// l, l + 64, l + 128, l + 192; their mind, near and the nearest centre's dcc, three loads in
// flight per point) and lists the points the new centre may come closer to in LDS (ballot
// order); it then reads only the listed rows, 8 G at a time (8 lanes a row, JU column slices of
// each in flight per lane), and leaves each distance in LDS for the lane that owns the point,
// which keeps the smaller of it and mind.  JU = min(4, dpad / 32): the column slices of a row a
// lane has in flight (the row loop steps 32 JU floats); G = 4 rows a lane for JU <= 2 and 2 above,
// which keeps the kernel within 64 VGPRs (8 waves per SIMD, so that the 1,954 blocks of a
// 2,000,000-point step are resident at once).
template <int JU, int G>
__global__ __launch_bounds__(256) void k_kpp_update(const float *__restrict__ pts, int dpad, int n,
                                                    const float *__restrict__ c, int cidx,
                                                    float *__restrict__ mind, int32_t *__restrict__ near,
                                                    const float *__restrict__ dcc, float prune,
                                                    double *__restrict__ partial) {
    extern __shared__ float4 s_c[];  // the centre, dpad / 4 float4
    __shared__ double red[256];
    __shared__ int s_list[4][kKppBlock / 4];    // listed points of each wave (offsets in its 256)
    __shared__ float s_dist[4][kKppBlock / 4];  // their distances to the centre
    const int nc4 = dpad >> 2;
    for (int i = threadIdx.x; i < nc4; i += 256) s_c[i] = ((const float4 *)c)[i];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int b0 = blockIdx.x * kKppBlock + wave * (kKppBlock / 4);
    const int b1 = min(n, b0 + kKppBlock / 4);
    // test the wave's points
    float m[4];
    bool need[4];
    int a[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int r = min(b0 + lane + 64 * q, n - 1);
        m[q] = mind[r];
        a[q] = near[r];
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float dc = dcc[a[q] >= 0 ? a[q] : 0];  // not used when a[q] < 0
        need[q] = b0 + lane + 64 * q < b1 && !(prune > 0.0f && a[q] >= 0 && dc >= prune * m[q]);
    }
    int cnt = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const unsigned long long bal = __ballot(need[q]);
        const int below = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0));
        if (need[q]) s_list[wave][cnt + below] = lane + 64 * q;
        cnt += __popcll(bal);
    }
    __syncthreads();  // s_c and the lists
    // the listed rows, 4 groups of 8 rows per pass
    const int part = lane & 7, slot = lane >> 3;
    for (int it = 0; it < cnt; it += 8 * G) {
        int rl[G];
        const float4 *row[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            rl[g] = s_list[wave][min(it + 8 * g + slot, cnt - 1)];
            row[g] = (const float4 *)(pts + (size_t)(b0 + rl[g]) * dpad);
        }
        float d2[G];
#pragma unroll
        for (int g = 0; g < G; ++g) d2[g] = 0.0f;
        for (int j0 = part; j0 < nc4; j0 += 8 * JU) {
            float4 xv[G][JU];
#pragma unroll
            for (int u = 0; u < JU; ++u) {
                const int j = min(j0 + 8 * u, nc4 - 1);
#pragma unroll
                for (int g = 0; g < G; ++g) xv[g][u] = row[g][j];
            }
#pragma unroll
            for (int u = 0; u < JU; ++u)
                if (j0 + 8 * u < nc4) {
                    const float4 cv = s_c[j0 + 8 * u];
#pragma unroll
                    for (int g = 0; g < G; ++g) d2[g] = acc_d2(d2[g], xv[g][u], cv);
                }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float v = d2[g];
            v += __shfl_xor(v, 1, 64);
            v += __shfl_xor(v, 2, 64);
            v += __shfl_xor(v, 4, 64);
            if (part == 0 && it + 8 * g + slot < cnt) s_dist[wave][rl[g]] = v;
        }
    }
    __syncthreads();  // the distances
    double s = 0.0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int r = b0 + lane + 64 * q;
        if (r < b1) {
            if (need[q]) {
                const float v = s_dist[wave][lane + 64 * q];
                if (v < m[q]) {
                    m[q] = v;
                    mind[r] = v;
                    near[r] = cidx;
                }
            }
            s += (double)m[q];
        }
    }
    red[threadIdx.x] = s;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) partial[blockIdx.x] = red[0];
}

// The update for point sets below kKppRowsMaxN: a wave holds 64 / L rows at a time, L lanes a row,
// and takes `passes` such row groups one after another; a workgroup's 4 waves cover 4 (64 / L)
// passes consecutive points, whose mind values it sums into partial[blockIdx.x] (each lane's
// rows in order, then the wave by a fixed shuffle tree, then the 4 waves in order).  prune as in
// k_kpp_update (0: every row is read and dcc is not).
template <int L>
__global__ __launch_bounds__(256) void k_kpp_update_rows(const float *__restrict__ pts, int dpad, int n,
                                                         const float *__restrict__ c, int cidx,
                                                         float *__restrict__ mind, int32_t *__restrict__ near,
                                                         const float *__restrict__ dcc, float prune, int passes,
                                                         double *__restrict__ partial) {
    constexpr int R = 64 / L;
    __shared__ double red[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, sub = lane & (L - 1);
    const int nc4 = dpad >> 2;
    const int r0 = (blockIdx.x * 4 + wave) * R * passes + lane / L;
    double s = 0.0;
    for (int p = 0; p < passes; ++p) {
        const int r = r0 + p * R;
        if (r < n) {  // uniform over the row's L lanes
            float m = mind[r];
            bool need = true;
            if (prune > 0.0f) {
                const int a = near[r];
                need = !(a >= 0 && dcc[a] >= prune * m);
            }
            if (need) {  // uniform over the row's L lanes, so the group's shuffles stay within it
                const float v = group_d2<L>((const float4 *)(pts + (size_t)r * dpad), (const float4 *)c, nc4, sub);
                if (v < m) {
                    m = v;
                    if (sub == 0) {
                        mind[r] = v;
                        near[r] = cidx;
                    }
                }
            }
            if (sub == 0) s += (double)m;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if (lane == 0) red[wave] = s;
    __syncthreads();
    if (threadIdx.x == 0) partial[blockIdx.x] = ((red[0] + red[1]) + red[2]) + red[3];
}

// Inclusive prefix sum of one double per thread over the workgroup (kKppSelectThreads threads), in
// a fixed order: within each wave by shuffles, then the wave totals; `tmp` holds 16 doubles.
__device__ __forceinline__ double block_scan_incl(double v, double *tmp) {
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const double a = __shfl_up(v, o, 64);
        if (lane >= o) v += a;
    }
    __syncthreads();  // tmp is free (an earlier scan's readers are done)
    if (lane == 63) tmp[w] = v;
    __syncthreads();
    double before = 0.0;
    for (int i = 0; i < w; ++i) before += tmp[i];
    return before + v;
}

// Step j's draw over nb blocks of blk points (partial: their sums).  draw: the step's 64-bit
// random value.  A total weight of at most 1e-6 (every
// point on a centre) takes draw mod n, as the reference takes a uniform index there.  Otherwise
// the threshold is u * total with u = the draw's top 53 bits in [0, 1), and the centre is the
// first point of positive weight whose running sum of mind reaches it: the first run of blocks,
// then block, then point, at which the running sum reaches the threshold.  Should rounding leave
// the running sums short of a threshold near the total, the last run (block, point) of positive
// weight is taken.  Every choice is a minimum or maximum over the threads, so the result does not
// depend on their timing.
__global__ __launch_bounds__(kKppSelectThreads) void k_kpp_select(const double *__restrict__ partial, int nb,
                                                                  int blk, const float *__restrict__ mind, int n,
                                                                  const uint64_t *__restrict__ draws, int j,
                                                                  const float *__restrict__ pts, int dpad,
                                                                  float *__restrict__ cent) {
    __shared__ double tmp[kKppSelectThreads / 64];
    __shared__ int s_run, s_lastrun, s_blk, s_pt, s_last;
    __shared__ double s_before, s_total;
    const int t = threadIdx.x;
    const uint64_t draw = draws[j];
    // block sums: thread t owns a contiguous run of them
    const int per = (nb + kKppSelectThreads - 1) / kKppSelectThreads;
    const int c0 = min(nb, t * per), c1 = min(nb, c0 + per);
    double own = 0.0;
    for (int b = c0; b < c1; ++b) own += partial[b];
    const double incl = block_scan_incl(own, tmp);
    const double excl = incl - own;  // unused for runs of no weight
    if (t == kKppSelectThreads - 1) s_total = incl;
    if (t == 0) {
        s_run = kKppSelectThreads;
        s_lastrun = -1;
        s_pt = 0x7fffffff;
        s_last = -1;
    }
    __syncthreads();
    const double total = s_total;
    int idx;
    if (total <= 1e-6) {
        idx = (int)(draw % (uint64_t)n);
    } else {
        const double thr = (double)(draw >> 11) * (1.0 / 9007199254740992.0) * total;
        if (own > 0.0) {
            if (incl >= thr) atomicMin(&s_run, t);
            atomicMax(&s_lastrun, t);
        }
        __syncthreads();
        // the scan's rounding may leave every run of weight short of a threshold near the total:
        // then the last run of weight
        if (t == (s_run < kKppSelectThreads ? s_run : s_lastrun)) {
            double cum = excl, cum_last = excl;
            int pb = -1, lastb = -1;
            for (int b = c0; b < c1; ++b) {
                const double w = partial[b];
                if (w > 0.0) {
                    if (cum + w >= thr) {
                        pb = b;
                        break;
                    }
                    lastb = b;
                    cum_last = cum;
                }
                cum += w;
            }
            if (pb < 0) {
                pb = lastb;
                cum = cum_last;
            }
            s_blk = pb;
            s_before = cum;
        }
        __syncthreads();
        const int pb = s_blk;
        const int i = pb * blk + t;  // blk <= kKppSelectThreads: one value per thread
        const double w = t < blk && i < n ? (double)mind[i] : 0.0;
        const double ci = s_before + block_scan_incl(w, tmp);
        if (w > 0.0) {
            if (ci >= thr) atomicMin(&s_pt, i);
            atomicMax(&s_last, i);
        }
        __syncthreads();
        idx = s_pt != 0x7fffffff ? s_pt : s_last;
    }
    const float *src = pts + (size_t)idx * dpad;
    float *dst = cent + (size_t)j * dpad;
    for (int d = t; d < dpad; d += kKppSelectThreads) dst[d] = src[d];
}

__global__ void k_fill(float *p, size_t count, float v) {
    const size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (i < count) p[i] = v;
}

}  // namespace vh

struct vhip_kmeans {
    int dev = 0;
    size_t n = 0, n_pad = 0, dim = 0, dpad = 0, k = 0, kpad = 0;
    int metric = 0;
    int grid_cap = 512;
    bool direct_small = true;  // small point sets take the direct-form assignment
    float absmax = 0.0f;     // max |x| over the points
    float err_coeff = 0.0f;  // selection error coefficient of the MFMA assignment
    bool assigned = false;
    bool shifted = false;    // squared L2: pts / cent hold the data minus `shift`
    hipStream_t stream = nullptr;
    // pts: the assign rows of the points (shifted for squared L2), praw the unshifted points when
    // they differ (the update, inertia and fix-up read them); craw: the centroids (the state),
    // cent: their assign rows (shifted, kpad rows with NaN padding)
    vh::DevBuf pts, praw, shift, pnorm, craw, cent, cnorm, cabs, cmax, assign, pos, inertia, counts, offsets, sorted,
        shifts, partial, sums, exps, devmax, fix, nfix, best;
    const float *points() const { return shifted ? praw.as<float>() : pts.as<float>(); }
    vh::PinnedStager stager;
    vh::KernelTimer timer;
    std::mutex mu;
    ~vhip_kmeans() {
        if (stream) {
            (void)hipSetDevice(dev);
            (void)hipStreamSynchronize(stream);
            (void)hipStreamDestroy(stream);
        }
    }
};

namespace vh {

// squared norms for L2 (epilogue and error bound) and dot product (error bound), norms for cosine
static int km_norm_kind(int metric) { return metric == COS ? 2 : ((metric == L2 || metric == DOT) ? 1 : 0); }

// Points given as nseg host segments (segment i: counts[i] rows of dim floats), uploaded one after
// another into one device buffer, so callers with several shards need no concatenated copy.
static int km_create(int ordinal, const float *const *segs, const size_t *counts, size_t nseg, size_t dim, int metric,
                     vhip_kmeans **out) {
    *out = nullptr;
    if (dim == 0) return set_error(VHIP_ERR_INVALID_CONFIG, "dimension must be > 0");
    if (dim > 1024) return set_error(VHIP_ERR_INVALID_CONFIG, "k-means supports dimension <= 1024");
    if (metric < 0 || metric > 9) return set_error(VHIP_ERR_INVALID_CONFIG, "unknown metric code");
    size_t n = 0;
    for (size_t i = 0; i < nseg; ++i) {
        if (counts[i] && !segs[i]) return set_error(VHIP_ERR_INVALID_CONFIG, "a point segment is null");
        n += counts[i];
    }
    if (n == 0) return set_error(VHIP_ERR_INVALID_CONFIG, "k-means needs at least one point");
    if (n > 0x7fffffffull) return set_error(VHIP_ERR_INVALID_CONFIG, "k-means supports n < 2^31 points");
    VH_CHECK(open_device(ordinal));
    std::unique_ptr<vhip_kmeans> K(new vhip_kmeans());
    K->dev = ordinal;
    K->n = n;
    K->n_pad = round_up(n, kTileCols);
    K->dim = dim;
    K->dpad = round_up(dim, kKChunk);
    K->metric = metric;
    K->grid_cap = device_grid_cap(ordinal);
    // VHIP_KMEANS_ASSIGN=mfma keeps small point sets on the MFMA assignment (tests of both paths)
    if (const char *e = std::getenv("VHIP_KMEANS_ASSIGN")) K->direct_small = std::strcmp(e, "mfma") != 0;
    hipStream_t s;
    VH_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    K->stream = s;
    VH_CHECK(K->stager.init(ordinal));
    DevBuf raw;
    VH_CHECK(raw.ensure(ordinal, n * dim * sizeof(float)));
    size_t row = 0;
    for (size_t i = 0; i < nseg; ++i) {
        if (counts[i])
            VH_CHECK(K->stager.h2d(raw.as<float>() + row * dim, segs[i], counts[i] * dim * sizeof(float), s));
        row += counts[i];
    }
    // max |x|: the finiteness check and the deviation bound of the non-L2 metrics' update
    const int nb = 1024;
    VH_CHECK(K->partial.ensure(ordinal, 8192 * sizeof(double)));
    hipLaunchKernelGGL(k_absmax_partial, dim3(nb), dim3(256), 0, s, raw.as<float>(), n * dim, K->partial.as<float>());
    VH_HIP(hipGetLastError());
    std::vector<float> pm(nb);
    VH_HIP(hipMemcpyAsync(pm.data(), K->partial.p, nb * sizeof(float), hipMemcpyDeviceToHost, s));
    VH_HIP(hipStreamSynchronize(s));
    float mx = 0.0f;
    for (float v : pm) mx = std::max(mx, v);
    if (!std::isfinite(mx)) return set_error(VHIP_ERR_INVALID_CONFIG, "data contains non-finite values");
    K->absmax = mx;
    if (metric == L2) {
        // per-dimension shift: the column means (integers for integer data)
        DevBuf part, flag;
        VH_CHECK(part.ensure(ordinal, col_shift_scratch_bytes((int)dim)));
        VH_CHECK(flag.ensure(ordinal, sizeof(uint32_t)));
        VH_CHECK(K->shift.ensure(ordinal, K->dpad * sizeof(float)));
        launch_fill_u32(flag.as<uint32_t>(), 1, 0u, s);
        launch_col_shift(raw.as<float>(), n, (int)dim, (int)K->dpad, part.as<double>(), flag.as<uint32_t>(),
                         K->shift.as<float>(), s);
        VH_HIP(hipGetLastError());
        std::vector<float> mu(K->dpad);
        VH_HIP(hipMemcpyAsync(mu.data(), K->shift.p, K->dpad * sizeof(float), hipMemcpyDeviceToHost, s));
        VH_HIP(hipStreamSynchronize(s));
        for (float v : mu) K->shifted = K->shifted || v != 0.0f;
    }
    // points padded to a multiple of 128 rows with zero rows (their results are never written)
    VH_CHECK(K->pts.ensure(ordinal, K->n_pad * K->dpad * sizeof(float)));
    VH_CHECK(K->pnorm.ensure(ordinal, K->n_pad * sizeof(float)));
    if (K->shifted) VH_CHECK(K->praw.ensure(ordinal, K->n_pad * K->dpad * sizeof(float)));
    RowPrep rp;
    rp.in = raw.as<float>();
    rp.n = n;
    rp.n_out = K->n_pad;
    rp.dim = (int)dim;
    rp.dpad = (int)K->dpad;
    rp.shift = K->shifted ? K->shift.as<float>() : nullptr;
    rp.out = K->pts.as<float>();
    rp.raw_out = K->shifted ? K->praw.as<float>() : nullptr;
    rp.norm = K->pnorm.as<float>();
    rp.norm_kind = km_norm_kind(metric);
    launch_rows_prep(rp, s);
    VH_HIP(hipGetLastError());
    K->err_coeff = sel_err_coeff(metric, (int)K->dpad);
    VH_CHECK(K->assign.ensure(ordinal, n * sizeof(int32_t)));
    VH_CHECK(K->pos.ensure(ordinal, n * sizeof(int32_t)));
    VH_CHECK(K->inertia.ensure(ordinal, n * sizeof(float)));
    VH_CHECK(K->sorted.ensure(ordinal, n * sizeof(int32_t)));
    if (is_gemm_metric(metric)) {
        VH_CHECK(K->fix.ensure(ordinal, n * sizeof(int32_t)));
        VH_CHECK(K->best.ensure(ordinal, n * sizeof(unsigned long long)));
    }
    VH_CHECK(K->nfix.ensure(ordinal, sizeof(uint32_t)));
    VH_CHECK(K->cmax.ensure(ordinal, sizeof(uint32_t)));
    VH_HIP(hipStreamSynchronize(s));  // `raw` is released at return
    *out = K.release();
    return VHIP_OK;
}

// Assign rows, norms and bounds of the current centroids (craw).
static void km_prep_centroids(vhip_kmeans *K) {
    launch_fill_u32(K->cmax.as<uint32_t>(), 1, 0u, K->stream);
    hipLaunchKernelGGL(k_cent_prep, dim3(ceil_div((long)K->kpad, 4)), dim3(256), 0, K->stream, (int)K->k, (int)K->kpad,
                       (int)K->dpad, K->craw.as<float>(), K->shifted ? K->shift.as<float>() : nullptr,
                       K->cent.as<float>(), K->cnorm.as<float>(), km_norm_kind(K->metric), K->metric == L2 ? 1 : 0,
                       K->cabs.as<float>(), K->cmax.as<uint32_t>());
}

// Sets k centroids from device rows d_c (row stride `row_stride` floats: dim, or dpad for rows
// already padded; d_c may be craw itself).  Assign rows are padded to a multiple of 256 with rows
// that never win the argmin: NaN rows (NaN scores), or for squared L2 zero rows of norm FLT_MAX
// (scores FLT_MAX; the assignment also rejects any row past k).
static int km_set_centroids_dev(vhip_kmeans *K, const float *d_c, size_t k, size_t row_stride) {
    const size_t kpad = round_up(k, kRowAlign);
    if (d_c != K->craw.as<float>()) VH_CHECK(K->craw.ensure(K->dev, k * K->dpad * sizeof(float)));
    VH_CHECK(K->cent.ensure(K->dev, kpad * K->dpad * sizeof(float)));
    VH_CHECK(K->cnorm.ensure(K->dev, kpad * sizeof(float)));
    VH_CHECK(K->cabs.ensure(K->dev, k * sizeof(float)));
    VH_CHECK(K->counts.ensure(K->dev, k * sizeof(int32_t)));
    VH_CHECK(K->offsets.ensure(K->dev, (k + 1) * sizeof(int32_t)));
    VH_CHECK(K->shifts.ensure(K->dev, k * sizeof(float)));
    VH_CHECK(K->exps.ensure(K->dev, k * sizeof(int32_t)));
    VH_CHECK(K->devmax.ensure(K->dev, k * sizeof(float)));
    VH_CHECK(K->sums.ensure(K->dev, k * K->dpad * sizeof(unsigned long long)));
    launch_fill_u32(K->sums.as<uint32_t>(), 2 * k * K->dpad, 0u, K->stream);
    if (row_stride == K->dim)
        launch_rows_prep(d_c, k, k, (int)K->dim, (int)K->dpad, nullptr, K->craw.as<float>(), nullptr, 0, 0, 0, 0.0f,
                         K->stream);
    else if (d_c != K->craw.as<float>())
        VH_HIP(hipMemcpyAsync(K->craw.p, d_c, k * K->dpad * sizeof(float), hipMemcpyDeviceToDevice, K->stream));
    VH_HIP(hipGetLastError());
    K->k = k;
    K->kpad = kpad;
    km_prep_centroids(K);
    VH_HIP(hipGetLastError());
    K->assigned = false;
    return VHIP_OK;
}

// Assignment of every point to its nearest centroid, with tickets pos / counts; inertia for all
// metrics but squared L2 (the update writes that one).
static int km_assign(vhip_kmeans *K) {
    hipStream_t s = K->stream;
    const int n = (int)K->n, k = (int)K->k;
    launch_fill_u32(K->counts.as<uint32_t>(), k, 0u, s);
    const int t = K->timer.begin(s);
    // small point sets: the direct form for every point (no MFMA tiles, no fix-up)
    const bool small = is_gemm_metric(K->metric) && K->direct_small &&
                       kmeans_assign_small_ok(n, k, (int)K->dpad, K->grid_cap / 2);
    if (small) {
        launch_fill_u32(K->devmax.as<uint32_t>(), k, 0u, s);
        launch_kmeans_assign_small(K->metric, K->points(), (int)K->dpad, n, K->craw.as<float>(), k,
                                   K->assign.as<int32_t>(), K->inertia.as<float>(), K->pos.as<int32_t>(),
                                   K->counts.as<int32_t>(), K->devmax.as<float>(), s);
    } else if (is_gemm_metric(K->metric)) {
        launch_fill_u32(K->devmax.as<uint32_t>(), k, 0u, s);
        launch_fill_u32(K->nfix.as<uint32_t>(), 1, 0u, s);
        AssignCert cert;
        cert.err_coeff = K->err_coeff;
        cert.cmax = K->cmax.as<float>();
        cert.fix = K->fix.as<int32_t>();
        cert.nfix = K->nfix.as<uint32_t>();
        cert.devmax = K->devmax.as<float>();
        cert.k = (int)K->k;
        launch_kmeans_assign(K->metric, K->cent.as<float>(), K->cnorm.as<float>(), (int)K->kpad, K->pts.as<float>(),
                             K->pnorm.as<float>(), n, (int)K->dpad, K->assign.as<int32_t>(), K->inertia.as<float>(),
                             K->pos.as<int32_t>(), K->counts.as<int32_t>(), cert, K->grid_cap, s);
    } else {
        launch_kmeans_assign_valu(K->metric, K->cent.as<float>(), k, K->pts.as<float>(), n, (int)K->dpad,
                                  K->assign.as<int32_t>(), K->inertia.as<float>(), K->pos.as<int32_t>(),
                                  K->counts.as<int32_t>(), K->grid_cap, s);
    }
    // algorithmic work: 2*n*k*dim flops (MFMA) or n*k*dim element operations; bytes: points + centroids
    const double work = (is_gemm_metric(K->metric) ? 2.0 : 1.0) * (double)n * k * (double)K->dim;
    K->timer.end(t, s, work, ((double)n + k) * K->dim * 4.0);
    VH_HIP(hipGetLastError());
    if (is_gemm_metric(K->metric) && !small) {
        launch_kmeans_fix(K->metric, K->points(), (int)K->dpad, K->fix.as<int32_t>(), K->nfix.as<uint32_t>(),
                          K->craw.as<float>(), k, K->best.as<unsigned long long>(), K->assign.as<int32_t>(),
                          K->inertia.as<float>(), K->pos.as<int32_t>(), K->counts.as<int32_t>(),
                          K->devmax.as<float>(), K->grid_cap, s);
        VH_HIP(hipGetLastError());
    }
    return VHIP_OK;
}

static int km_iterate(vhip_kmeans *K) {
    hipStream_t s = K->stream;
    const int n = (int)K->n, k = (int)K->k;
    VH_CHECK(km_assign(K));
    if (K->metric != L2)
        hipLaunchKernelGGL(k_dev_bound, dim3(ceil_div(k, 256)), dim3(256), 0, s, k, K->absmax, K->cabs.as<float>(),
                           K->devmax.as<float>());
    hipLaunchKernelGGL(k_update_scales, dim3(ceil_div(k, 256)), dim3(256), 0, s, k, K->devmax.as<float>(),
                       K->counts.as<int32_t>(), K->exps.as<int32_t>());
    hipLaunchKernelGGL(k_scan_counts, dim3(1), dim3(1024), 0, s, K->counts.as<int32_t>(), k, K->offsets.as<int32_t>());
    hipLaunchKernelGGL(k_scatter, dim3(ceil_div(n, 256)), dim3(256), 0, s, K->assign.as<int32_t>(),
                       K->pos.as<int32_t>(), K->offsets.as<int32_t>(), n, K->sorted.as<int32_t>());
    const int slots = ceil_div((long)K->dpad, 64);
    int spw = kUpdSlotsPerWave;  // slots per wave: fewer for small point sets, so they fill the GPU
    while (spw > kUpdMinSlots && ceil_div(n, spw) < kUpdMinWaves) spw >>= 1;
    const int waves = ceil_div(n, spw);
    // the per-point values in direct form (kmeans.cu:110-170's squared distance, -dot, 1 - cos);
    // the other metrics' assignment wrote them
    const int mode = K->metric == L2 ? 1 : (K->metric == DOT ? 2 : (K->metric == COS ? 3 : 0));
    unsigned long long *sums = K->sums.as<unsigned long long>();
#define VH_UPD(S)                                                                                                  \
    do {                                                                                                           \
        hipLaunchKernelGGL(k_update_sums<S>, dim3(ceil_div(waves, 4)), dim3(256), 0, s, K->points(),               \
                           K->craw.as<float>(), (int)K->dpad, (int)K->dim, n, k, K->sorted.as<int32_t>(),          \
                           K->offsets.as<int32_t>(), K->exps.as<int32_t>(), sums, K->inertia.as<float>(), mode,         \
                           K->pnorm.as<float>(), K->cnorm.as<float>(), spw);                                        \
        hipLaunchKernelGGL(k_update_finalize<S>, dim3(ceil_div(k, 4)), dim3(256), 0, s, k, (int)K->dpad,          \
                           (int)K->dim, sums, K->counts.as<int32_t>(), K->exps.as<int32_t>(), K->craw.as<float>(), \
                           K->shifts.as<float>());                                                                  \
    } while (0)
    if (slots <= 1) VH_UPD(1);
    else if (slots <= 2) VH_UPD(2);
    else if (slots <= 4) VH_UPD(4);
    else if (slots <= 8) VH_UPD(8);
    else VH_UPD(16);
#undef VH_UPD
    km_prep_centroids(K);
    VH_HIP(hipGetLastError());
    K->assigned = true;
    return VHIP_OK;
}

static int km_total_inertia(vhip_kmeans *K, float *out) {
    const int nb = 256;
    const size_t chunk = (K->n + nb - 1) / nb;
    hipLaunchKernelGGL(k_sum_partial, dim3(nb), dim3(256), 0, K->stream, K->inertia.as<float>(), K->n, chunk,
                       K->partial.as<double>());
    VH_HIP(hipGetLastError());
    std::vector<double> part(nb);
    VH_HIP(hipMemcpyAsync(part.data(), K->partial.p, nb * sizeof(double), hipMemcpyDeviceToHost, K->stream));
    VH_HIP(hipStreamSynchronize(K->stream));
    double s = 0.0;
    for (double v : part) s += v;
    *out = (float)s;
    return VHIP_OK;
}

// Seeded k-means++ (kmeans.rs:409-460): first centre uniform, then each next centre drawn
// with probability proportional to the squared L2 distance to the nearest chosen centre.  The
// draws (one 64-bit splitmix64 value per centre) are made on the host up front; every step then
// runs on the device (k_kpp_dcc, an update kernel, k_kpp_select), with no host round trip.
static int km_init_kmeanspp(vhip_kmeans *K, size_t k, uint64_t seed) {
    hipStream_t s = K->stream;
    const int n = (int)K->n;
    const int dpad = (int)K->dpad;
    VH_CHECK(K->craw.ensure(K->dev, k * K->dpad * sizeof(float)));
    const float *pts = K->points();
    float *cr = K->craw.as<float>();
    // the update's shape: blocks of blk points, nb of them
    const int lanes = kpp_lanes(dpad / 4);
    const bool rows = n < kKppRowsMaxN;
    int passes = 1;
    if (rows)
        while (ceil_div(n, 4 * (64 / lanes) * passes) > kKppRowsMaxBlocks && 4 * (64 / lanes) * passes < kKppBlock)
            passes *= 2;
    const int blk = rows ? 4 * (64 / lanes) * passes : kKppBlock;
    const int nb = ceil_div(n, blk);
    const bool prune_on = !rows || (size_t)n * K->dpad > kKppPruneFloats;
    DevBuf mind, near, part, draws, dcc;
    VH_CHECK(mind.ensure(K->dev, (size_t)n * sizeof(float)));
    VH_CHECK(near.ensure(K->dev, (size_t)n * sizeof(int32_t)));
    VH_CHECK(part.ensure(K->dev, (size_t)nb * sizeof(double)));
    VH_CHECK(draws.ensure(K->dev, k * sizeof(uint64_t)));
    VH_CHECK(dcc.ensure(K->dev, k * sizeof(float)));
    std::vector<uint64_t> dh(k);
    uint64_t st = seed;
    for (size_t j = 0; j < k; ++j) dh[j] = splitmix64(st);
    VH_HIP(hipMemcpyAsync(draws.p, dh.data(), k * sizeof(uint64_t), hipMemcpyHostToDevice, s));
    hipLaunchKernelGGL(k_fill, dim3(ceil_div(n, 256)), dim3(256), 0, s, mind.as<float>(), (size_t)n, 3.4028235e38f);
    launch_fill_u32((uint32_t *)near.as<int32_t>(), (size_t)n, 0xffffffffu, s);
    const size_t idx = dh[0] % (size_t)n;
    VH_HIP(hipMemcpyAsync(cr, pts + idx * K->dpad, K->dpad * sizeof(float), hipMemcpyDeviceToDevice, s));
    // Pruning factor 4 (1 + 64 g), g = gamma_{dpad+2}: each of the three computed squared
    // distances (the centres', the point's to its nearest, the point's to the new centre) is
    // within a factor (1 +- g) of its value, and (1 + 64 g) leaves room for all three.
    const float prune = prune_on ? (float)(4.0 * (1.0 + 64.0 * gamma_n((double)K->dpad + 2.0))) : 0.0f;
    const size_t lds = K->dpad * sizeof(float);
    for (size_t j = 1; j < k; ++j) {
        const int m = (int)j - 1;  // the newest centre
        const float *c = cr + (size_t)m * K->dpad;
        if (prune_on && m > 0) {
            const dim3 g(ceil_div(m, 4 * (64 / lanes)));
            switch (lanes) {
                case 8: hipLaunchKernelGGL(k_kpp_dcc<8>, g, dim3(256), 0, s, cr, dpad, m, dcc.as<float>()); break;
                case 16: hipLaunchKernelGGL(k_kpp_dcc<16>, g, dim3(256), 0, s, cr, dpad, m, dcc.as<float>()); break;
                case 32: hipLaunchKernelGGL(k_kpp_dcc<32>, g, dim3(256), 0, s, cr, dpad, m, dcc.as<float>()); break;
                default: hipLaunchKernelGGL(k_kpp_dcc<64>, g, dim3(256), 0, s, cr, dpad, m, dcc.as<float>()); break;
            }
        }
        if (rows) {
#define VH_KPP_ROWS(LN)                                                                                          \
    hipLaunchKernelGGL(k_kpp_update_rows<LN>, dim3(nb), dim3(256), 0, s, pts, dpad, n, c, m, mind.as<float>(), \
                       near.as<int32_t>(), dcc.as<float>(), prune, passes, part.as<double>())
            switch (lanes) {
                case 8: VH_KPP_ROWS(8); break;
                case 16: VH_KPP_ROWS(16); break;
                case 32: VH_KPP_ROWS(32); break;
                default: VH_KPP_ROWS(64); break;
            }
#undef VH_KPP_ROWS
        } else {
#define VH_KPP_BLOCKS(JU)                                                                                    \
    hipLaunchKernelGGL((k_kpp_update<JU, (JU <= 2 ? 4 : 2)>), dim3(nb), dim3(256), lds, s, pts, dpad, n, c, m, \
                       mind.as<float>(),                                                                     \
                       near.as<int32_t>(), dcc.as<float>(), prune, part.as<double>())
            switch (std::min(4, dpad / 32)) {  // column slices per lane and row in flight
                case 1: VH_KPP_BLOCKS(1); break;
                case 2: VH_KPP_BLOCKS(2); break;
                case 3: VH_KPP_BLOCKS(3); break;
                default: VH_KPP_BLOCKS(4); break;
            }
#undef VH_KPP_BLOCKS
        }
        hipLaunchKernelGGL(k_kpp_select, dim3(1), dim3(kKppSelectThreads), 0, s, part.as<double>(), nb, blk,
                           mind.as<float>(), n, draws.as<uint64_t>(), (int)j, pts, dpad, cr);
    }
    VH_HIP(hipGetLastError());
    VH_HIP(hipStreamSynchronize(s));  // mind, near, part, draws, dcc and dh are released at return
    return km_set_centroids_dev(K, cr, k, K->dpad);
}

}  // namespace vh

using namespace vh;

extern "C" {

int vhip_kmeans_create(int ordinal, const float *data, size_t n, size_t dim, int metric, vhip_kmeans **out) {
    clear_error();
    if (!out) return set_error(VHIP_ERR_INVALID_CONFIG, "out is null");
    return km_create(ordinal, &data, &n, 1, dim, metric, out);
}

int vhip_kmeans_create_segments(int ordinal, const float *const *segments, const size_t *counts, size_t nseg,
                                size_t dim, int metric, vhip_kmeans **out) {
    clear_error();
    if (!out || (nseg && (!segments || !counts))) return set_error(VHIP_ERR_INVALID_CONFIG, "null argument");
    return km_create(ordinal, segments, counts, nseg, dim, metric, out);
}

int vhip_kmeans_set_centroids(vhip_kmeans *K, const float *centroids, size_t k) {
    clear_error();
    if (!K || !centroids || k == 0) return set_error(VHIP_ERR_INVALID_CONFIG, "null state / centroids or k == 0");
    std::lock_guard<std::mutex> lock(K->mu);
    VH_CHECK(open_device(K->dev));
    DevBuf raw;
    VH_CHECK(raw.ensure(K->dev, k * K->dim * sizeof(float)));
    VH_CHECK(K->stager.h2d(raw.p, centroids, k * K->dim * sizeof(float), K->stream));
    VH_CHECK(km_set_centroids_dev(K, raw.as<float>(), k, K->dim));
    VH_HIP(hipStreamSynchronize(K->stream));
    return VHIP_OK;
}

int vhip_kmeans_run(vhip_kmeans *K, size_t iters) {
    clear_error();
    if (!K || K->k == 0) return set_error(VHIP_ERR_INVALID_CONFIG, "centroids not set");
    std::lock_guard<std::mutex> lock(K->mu);
    VH_CHECK(open_device(K->dev));
    for (size_t i = 0; i < iters; ++i) VH_CHECK(km_iterate(K));
    VH_HIP(hipStreamSynchronize(K->stream));
    K->timer.collect();
    return VHIP_OK;
}

int vhip_kmeans_assign_only(vhip_kmeans *K, int32_t *out_assign, float *out_score, float *out_residual) {
    clear_error();
    if (!K || K->k == 0) return set_error(VHIP_ERR_INVALID_CONFIG, "centroids not set");
    std::lock_guard<std::mutex> lock(K->mu);
    VH_CHECK(open_device(K->dev));
    hipStream_t s = K->stream;
    const int n = (int)K->n;
    VH_CHECK(km_assign(K));
    DevBuf score, resid;
    if (out_score || out_residual) {
        VH_CHECK(score.ensure(K->dev, K->n * sizeof(float)));
        if (out_residual) VH_CHECK(resid.ensure(K->dev, K->n * K->dim * sizeof(float)));
        const size_t blocks = std::min<size_t>(65536, (K->n + 3) / 4);
        hipLaunchKernelGGL(k_coarse_score, dim3((unsigned)blocks), dim3(256), 0, s, K->points(), (int)K->dpad,
                           (int)K->dim, n, K->craw.as<float>(), K->assign.as<int32_t>(), K->metric,
                           score.as<float>(), out_residual ? resid.as<float>() : nullptr);
        VH_HIP(hipGetLastError());
    }
    if (out_assign) VH_CHECK(K->stager.d2h(out_assign, K->assign.p, K->n * sizeof(int32_t), s));
    if (out_score) VH_CHECK(K->stager.d2h(out_score, score.p, K->n * sizeof(float), s));
    if (out_residual) VH_CHECK(K->stager.d2h(out_residual, resid.p, K->n * K->dim * sizeof(float), s));
    VH_HIP(hipStreamSynchronize(s));
    K->timer.collect();
    K->assigned = false;  // counts / centroids describe no update
    return VHIP_OK;
}

int vhip_kmeans_read(vhip_kmeans *K, float *centroids, int32_t *assign, int64_t *counts, float *shifts,
                     float *max_shift, float *inertia) {
    clear_error();
    if (!K) return set_error(VHIP_ERR_INVALID_CONFIG, "null state");
    std::lock_guard<std::mutex> lock(K->mu);
    VH_CHECK(open_device(K->dev));
    hipStream_t s = K->stream;
    if (centroids && K->k)
        VH_HIP(hipMemcpy2DAsync(centroids, K->dim * sizeof(float), K->craw.p, K->dpad * sizeof(float),
                                K->dim * sizeof(float), K->k, hipMemcpyDeviceToHost, s));
    if (assign && K->assigned)
        VH_HIP(hipMemcpyAsync(assign, K->assign.p, K->n * sizeof(int32_t), hipMemcpyDeviceToHost, s));
    std::vector<int32_t> c32(K->k);
    std::vector<float> sh(K->k);
    if (K->assigned && K->k) {
        VH_HIP(hipMemcpyAsync(c32.data(), K->counts.p, K->k * sizeof(int32_t), hipMemcpyDeviceToHost, s));
        VH_HIP(hipMemcpyAsync(sh.data(), K->shifts.p, K->k * sizeof(float), hipMemcpyDeviceToHost, s));
    }
    VH_HIP(hipStreamSynchronize(s));
    if (counts)
        for (size_t i = 0; i < K->k; ++i) counts[i] = K->assigned ? c32[i] : 0;
    if (shifts)
        for (size_t i = 0; i < K->k; ++i) shifts[i] = K->assigned ? sh[i] : 0.0f;
    if (max_shift) {
        float m = 0.0f;
        if (K->assigned)
            for (float v : sh) m = std::max(m, v);
        *max_shift = m;
    }
    if (inertia) {
        *inertia = 0.0f;
        if (K->assigned) VH_CHECK(km_total_inertia(K, inertia));
    }
    return VHIP_OK;
}

int vhip_kmeans_profile(vhip_kmeans *K, int enable) {
    if (!K) return set_error(VHIP_ERR_INVALID_CONFIG, "null state");
    std::lock_guard<std::mutex> lock(K->mu);
    K->timer.enabled = enable != 0;
    K->timer.reset();
    return VHIP_OK;
}

int vhip_kmeans_profile_read(vhip_kmeans *K, double *kernel_ms, uint64_t *launches, double *work, double *bytes) {
    if (!K) return set_error(VHIP_ERR_INVALID_CONFIG, "null state");
    std::lock_guard<std::mutex> lock(K->mu);
    if (kernel_ms) *kernel_ms = K->timer.ms;
    if (launches) *launches = K->timer.launches;
    if (work) *work = K->timer.work;
    if (bytes) *bytes = K->timer.bytes;
    return VHIP_OK;
}

void vhip_kmeans_destroy(vhip_kmeans *K) { delete K; }

int vhip_dkmeans_check(size_t num_gpus) {
    clear_error();
    if (num_gpus < 1) return set_error(VHIP_ERR_INVALID_CONFIG, "num_gpus must be at least 1");
    const size_t avail = (size_t)device_count();
    if (num_gpus > avail) {
        set_insufficient(num_gpus, avail);
        return VHIP_ERR_INSUFFICIENT_DEVICES;
    }
    return VHIP_OK;
}

int vhip_kmeans_fit_state(vhip_kmeans *K, size_t k, size_t max_iters, float tol, const float *init_centroids,
                          int init_mode, uint64_t seed, float *out_centroids, int32_t *out_assign,
                          vhip_kmeans_result *result) {
    clear_error();
    if (!K || !result) return set_error(VHIP_ERR_INVALID_CONFIG, "null state or result");
    *result = vhip_kmeans_result{K->dim, 0, 0, 0.0f};
    if (k == 0) return VHIP_OK;  // kmeans.rs:67-76
    const size_t n = K->n, dim = K->dim, ek = std::min(k, n);
    if (!out_centroids) return set_error(VHIP_ERR_INVALID_CONFIG, "out_centroids is null");
    if (init_mode != VHIP_INIT_KMEANSPP && init_mode != VHIP_INIT_SHUFFLE)
        return set_error(VHIP_ERR_INVALID_CONFIG, "unknown init mode");
    if (init_centroids) {
        VH_CHECK(vhip_kmeans_set_centroids(K, init_centroids, ek));
    } else if (init_mode == VHIP_INIT_SHUFFLE) {
        // DistributedKMeansEngine::init_random (distributed_kmeans.rs:524-535), seeded: the first
        // ek indices of a seeded permutation, gathered from the resident points
        std::lock_guard<std::mutex> lock(K->mu);
        VH_CHECK(open_device(K->dev));
        std::vector<uint32_t> idx = row_permutation(n, seed);
        DevBuf didx, rows;
        VH_CHECK(didx.ensure(K->dev, ek * sizeof(uint32_t)));
        VH_CHECK(rows.ensure(K->dev, ek * K->dpad * sizeof(float)));
        VH_HIP(hipMemcpyAsync(didx.p, idx.data(), ek * sizeof(uint32_t), hipMemcpyHostToDevice, K->stream));
        launch_gather_rows(K->points(), didx.as<uint32_t>(), ek, (int)K->dpad, rows.as<float>(), K->stream);
        VH_HIP(hipGetLastError());
        VH_CHECK(km_set_centroids_dev(K, rows.as<float>(), ek, K->dpad));
        VH_HIP(hipStreamSynchronize(K->stream));  // didx/rows/idx are released at scope end
    } else {
        std::lock_guard<std::mutex> lock(K->mu);
        VH_CHECK(open_device(K->dev));
        VH_CHECK(km_init_kmeanspp(K, ek, seed));
    }
    size_t iters = 0;
    {
        std::lock_guard<std::mutex> lock(K->mu);
        VH_CHECK(open_device(K->dev));
        std::vector<float> sh(ek);
        for (size_t it = 0; it < max_iters; ++it) {
            iters = it + 1;
            VH_CHECK(km_iterate(K));
            if (tol >= 0.0f) {  // kmeans.rs:218-223: only K floats cross PCIe per iteration
                VH_HIP(hipMemcpyAsync(sh.data(), K->shifts.p, ek * sizeof(float), hipMemcpyDeviceToHost, K->stream));
                VH_HIP(hipStreamSynchronize(K->stream));
                float m = 0.0f;
                for (float v : sh) m = std::max(m, v);
                if (m <= tol) break;
            }
        }
        VH_HIP(hipStreamSynchronize(K->stream));
    }
    float inertia = 0.0f;
    VH_CHECK(vhip_kmeans_read(K, out_centroids, out_assign, nullptr, nullptr, nullptr, &inertia));
    *result = vhip_kmeans_result{dim, ek, iters, inertia};
    return VHIP_OK;
}

int vhip_kmeans_fit(int ordinal, const float *data, size_t n, size_t dim, size_t k, size_t max_iters, float tol,
                    int metric, const float *init_centroids, int init_mode, uint64_t seed, float *out_centroids,
                    int32_t *out_assign, vhip_kmeans_result *result) {
    clear_error();
    if (!result) return set_error(VHIP_ERR_INVALID_CONFIG, "result is null");
    *result = vhip_kmeans_result{dim, 0, 0, 0.0f};
    if (n == 0 || k == 0) return VHIP_OK;  // kmeans.rs:67-76
    vhip_kmeans *raw = nullptr;
    VH_CHECK(km_create(ordinal, &data, &n, 1, dim, metric, &raw));
    std::unique_ptr<vhip_kmeans> K(raw);
    return vhip_kmeans_fit_state(K.get(), k, max_iters, tol, init_centroids, init_mode, seed, out_centroids,
                                 out_assign, result);
}

}  // extern "C"
