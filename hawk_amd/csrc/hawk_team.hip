// hawk_team.hip — the cross-sample team stages of hawk's gfx950 target,
// written by hand for CDNA4 (wave64, 160 KiB LDS per workgroup, 8 XCDs).
//
// Two reductions whose bits must not depend on the launch: the fixed-tree
// ordered sum (reference hawk/emit/team.py:208-278 `_block_part` and
// :173-192 `_block`, gp form) and the keyed ordered scatter (reference
// hawk/emit/team.py:322-460 with the chunk rule of hawk/_lane_bind.py:111-114).
// Neither uses a floating-point atomic: every addition happens in the order
// the reference's serial host walk makes it, so the results are bit-identical
// to that walk.  Build flags keep -ffp-contract=off.

#include "hawk_core.h"
#include "hawk_internal.h"

#include <hip/hip_runtime.h>
#include <cstdint>
#include <mutex>
#include <string>

namespace {

// ---------------------------------------------------------------------------
// Fixed-tree ordered sum.
// ---------------------------------------------------------------------------
constexpr int kVirtualLanes = 65536;   // reference hawk/emit/team.py:21-23
constexpr int kFoldLanes = 1024;
constexpr int kGroups = 64;            // reference hawk/ir/team.py:649 GROUPS
constexpr int kLaneBlock = 256;
constexpr int kSumUnroll = 32;

// Scratch layout (bytes): lanes[65536] f64 | gp[64] f64 | ticket u32 (+pad).
constexpr size_t kLanesBytes = sizeof(double) * kVirtualLanes;
constexpr size_t kGpBytes = sizeof(double) * kGroups;
constexpr size_t kSumScratch = kLanesBytes + kGpBytes + 256;

// Virtual lane l = blockIdx.x*256 + threadIdx.x adds u[l], u[l+65536], ... in
// order from +0.0.  The loads of kSumUnroll rows are issued before their adds
// so each lane keeps kSumUnroll loads in flight; the adds stay in row order.
// The fold's ticket is cleared here, one launch ahead of the fold that takes
// it, so a sum never depends on what an earlier call left in its scratch.
template <class T>
__global__ __launch_bounds__(kLaneBlock) void hawk_sum_lanes(const T* __restrict__ u,
                                                              long long n,
                                                              T* __restrict__ lanes,
                                                              unsigned* __restrict__ ticket) {
    const long long l = static_cast<long long>(blockIdx.x) * kLaneBlock + threadIdx.x;
    if (l == 0) *ticket = 0u;
    T s = T(0);
    long long r = l;
    constexpr long long kStep = kVirtualLanes;
    for (; r + (kSumUnroll - 1) * kStep < n; r += kSumUnroll * kStep) {
        T a[kSumUnroll];
#pragma unroll
        for (int k = 0; k < kSumUnroll; ++k) a[k] = __builtin_nontemporal_load(u + r + k * kStep);
#pragma unroll
        for (int k = 0; k < kSumUnroll; ++k) s += a[k];
    }
    for (; r < n; r += kStep) s += u[r];
    lanes[l] = s;
}

// Group g of 1024 lanes folded by s[i] += s[i+w], w = 512..1, into gp[g]; the
// last group to finish folds the 64 group values by the same tree, w = 32..1,
// and stores the result.  The ticket is left at zero for the next call.
// Thread t holds lanes t, t+256, t+512 and t+768, so levels 512 and 256 are
// its own adds; levels 128 and 64 cross waves through LDS, and levels 32..1
// run in wave 0, lane i adding lane i+w's value taken by a permute: the same
// additions in the same order as the tree over an LDS array, with two
// barriers in place of ten.
template <class T>
__global__ __launch_bounds__(256) void hawk_sum_fold(const T* __restrict__ lanes,
                                                     T* __restrict__ gp,
                                                     unsigned* __restrict__ ticket,
                                                     T* __restrict__ out) {
    static_assert(kFoldLanes == 1024 && kGroups == 64, "four lanes a thread, one wave of group values");
    __shared__ T up128[128];
    __shared__ T up64[64];
    __shared__ unsigned last;
    const int g = blockIdx.x;
    const int t = threadIdx.x;
    const T* src = lanes + static_cast<long long>(g) * kFoldLanes;
    const T x0 = src[t], x1 = src[t + 256], x2 = src[t + 512], x3 = src[t + 768];
    T a = (x0 + x2) + (x1 + x3);                 // w = 512 (lanes t and t+256), then w = 256
    if (t >= 128) up128[t - 128] = a;
    __syncthreads();
    if (t < 128) a = a + up128[t];               // w = 128
    if (t >= 64 && t < 128) up64[t - 64] = a;
    __syncthreads();
    if (t < 64) {
        a = a + up64[t];                         // w = 64
#pragma unroll
        for (int w = 32; w > 0; w >>= 1) a = a + __shfl_down(a, w, 64);
        if (t == 0) {
            gp[g] = a;
            __threadfence();
            last = atomicAdd(ticket, 1u);
        }
    }
    __syncthreads();
    if (last != kGroups - 1 || t >= 64) return;
    __threadfence();   // acquire: every group's gp store is visible
    T b = __builtin_nontemporal_load(gp + t);
#pragma unroll
    for (int w = 32; w > 0; w >>= 1) b = b + __shfl_down(b, w, 64);
    if (t == 0) {
        *out = b;
        *ticket = 0u;
    }
}

// ---------------------------------------------------------------------------
// Banded reductions (the banded scalar mode; reference hawk/emit/wrapper.py:140
// `BANDED`, hawk/emit/team.py:26-49 and :225-245): every partial is a band, a
// normalised double-double (h, l) with |l| <= ulp(h)/2, folded in the same
// fixed order as the float64 stages, and the stored cell is the final band's
// h.  Two bands join as in Hida, Li and Bailey's QD library: TwoSum of the
// leading and of the low parts and two quick renormalisations; Knuth's TwoSum
// is exact in either operand order, so the add is symmetric.  A virtual
// lane's run of terms accumulates by Neumaier's compensated sum and becomes a
// band at its end (lane_add, lane_band).  A non-finite leading sum drops the
// low part, so Inf and NaN follow IEEE through h.
// ---------------------------------------------------------------------------
struct Band {
    double h, l;
};

__device__ __forceinline__ Band band_two(double a, double b) {
    const double s = a + b;
    const double bb = s - a;
    return Band{s, (a - (s - bb)) + (b - bb)};
}

__device__ __forceinline__ Band band_quick(double a, double b) {
    const double s = a + b;
    return Band{s, b - (s - a)};
}

// A virtual lane's run of rows (the banded ordered sum): Neumaier's
// compensated sum, the running sum s one addition a row and each addition's
// exact error added to c beside it, so a row costs the chain one dependent
// add; renormalised into a band once, at the run's end, by TwoSum of (s, c);
// a non-finite s drops c.
struct LaneSum {
    double s, c;
};

__device__ __forceinline__ void lane_add(LaneSum& a, double x) {
    // the error by TwoSum: the exact error of t = s + x whichever operand is
    // larger, so the same value as Neumaier's branch on |s| >= |x|, without a
    // compare and select
    const double t = a.s + x;
    const double bb = t - a.s;
    a.c = a.c + ((a.s - (t - bb)) + (x - bb));
    a.s = t;
}

__device__ __forceinline__ Band lane_band(LaneSum a) {
    const Band b = band_two(a.s, a.c);
    const bool finite = (a.s - a.s) == 0.0;
    return Band{finite ? b.h : a.s, finite ? b.l : 0.0};
}

__device__ __forceinline__ Band band_add(Band a, Band b) {
    Band s = band_two(a.h, b.h);
    if (!((s.h - s.h) == 0.0)) return Band{s.h, 0.0};
    const Band t = band_two(a.l, b.l);
    s = band_quick(s.h, s.l + t.h);
    return band_quick(s.h, s.l + t.l);
}

// The banded ordered sum's geometry, reference hawk/emit/team.py:26-30
// (BAND_LANES, BAND_VIRTUAL_LANES) and :225-245: group g's 128 virtual lanes
// l = g*128 + t each add rows l, l + 8192, ... as terms of one band.
constexpr int kBandLanes = 128;
constexpr int kBandVirtual = kBandLanes * kGroups;   // 8192
constexpr size_t kBandLanesBytes = sizeof(Band) * kBandVirtual;
constexpr size_t kBandGpBytes = sizeof(Band) * kGroups;
constexpr size_t kBandSumScratch = kBandLanesBytes + kBandGpBytes + 256;

// One workgroup per kBandChains virtual lanes: wave 0 is the chains (lane c
// < kBandChains adds column c of each stage, kBandStage row blocks of
// kBandChains contiguous values, to its lane sum, row after row) and the
// kBandLoaders threads after it read the rows.  A stage reaches the loaders'
// registers kBandAhead stages before the chains add it and their LDS ring
// (kBandSlots stages) two stages before; the chain wave reads each stage into
// registers one stage ahead, so neither the rows' nor the LDS's latency
// meets the chain.  Clears the fold's ticket one launch ahead of the fold.
// Measured on MI355X at N = 2^26: 0.204 ms, against 0.227 for a two-stage
// ring of 64-row stages read after each barrier with 256 loaders, and 0.209
// with 256 loaders here (two loader waves leave the chains' SIMD to them).
// Chains spread over two or four waves measured slower (282 and 358 us
// against 236 in the two-stage form).
constexpr int kBandChains = 32;
constexpr int kBandStage = 32;
constexpr int kBandSlots = 3;
constexpr int kBandAhead = 6;                 // stages a row read has before its chain adds it
constexpr int kBandSets = kBandAhead - 2;     // loader register sets: stage s read at s - 6, stored at s - 2
constexpr int kBandLoaders = 128;
constexpr int kBandThreads = 64 + kBandLoaders;
constexpr int kBandPer = kBandStage * kBandChains / kBandLoaders;   // values a loader reads a stage
static_assert(kBandVirtual % kBandChains == 0 && kBandSets == 4, "whole workgroups of chains, four register sets");

__global__ __launch_bounds__(kBandThreads) void hawk_band_sum_lanes(const double* __restrict__ u, long long n,
                                                                     Band* __restrict__ lanes,
                                                                     unsigned* __restrict__ ticket) {
    __shared__ double buf[kBandSlots][kBandStage * kBandChains];
    const int t = threadIdx.x;
    const bool loader = t >= 64;
    const int lt = t - 64;
    const bool chain = t < kBandChains;
    const long long l0 = static_cast<long long>(blockIdx.x) * kBandChains;
    if (blockIdx.x == 0 && t == 0) *ticket = 0u;
    // row blocks of lane l0, the workgroup's longest lane, and its stages
    const long long blocks = n > l0 ? (n - l0 + kBandVirtual - 1) / kBandVirtual : 0;
    const long long stages = (blocks + kBandStage - 1) / kBandStage;
    double ld[kBandSets][kBandPer];
    auto load = [&](long long st, double (&reg)[kBandPer]) {
        if (!loader || st >= stages) return;
#pragma unroll
        for (int q = 0; q < kBandPer; ++q) {
            const int i = lt + q * kBandLoaders;
            const long long r = (st * kBandStage + i / kBandChains) * kBandVirtual + l0 + i % kBandChains;
            reg[q] = r < n ? __builtin_nontemporal_load(u + r) : 0.0;
        }
    };
    auto store = [&](long long st, const double (&reg)[kBandPer]) {
        if (!loader || st >= stages) return;
        double* slot = buf[st % kBandSlots];
#pragma unroll
        for (int q = 0; q < kBandPer; ++q) slot[lt + q * kBandLoaders] = reg[q];
    };
    const long long mine = chain && l0 + t < n ? (n - l0 - t + kBandVirtual - 1) / kBandVirtual : 0;
    LaneSum acc{0.0, 0.0};
    double v[2][kBandStage];
    auto fetch = [&](long long st, double (&v)[kBandStage]) {
        if (!chain || st >= stages) return;
        const double* slot = buf[st % kBandSlots];
#pragma unroll
        for (int k = 0; k < kBandStage; ++k) v[k] = slot[k * kBandChains + t];
    };
    auto add = [&](long long st, const double (&v)[kBandStage]) {
        if (!chain) return;
        const long long left = mine - st * kBandStage;
        if (left >= kBandStage) {
#pragma unroll
            for (int k = 0; k < kBandStage; ++k) lane_add(acc, v[k]);
        } else {
#pragma unroll
            for (int k = 0; k < kBandStage; ++k)
                if (k < left) lane_add(acc, v[k]);
        }
    };
    // stages 0 .. 3 into the loaders' registers, 0 and 1 into the ring
#pragma unroll
    for (int j = 0; j < kBandSets; ++j) load(j, ld[j]);
    store(0, ld[0]);
    store(1, ld[1]);
    load(kBandSets, ld[0]);
    load(kBandSets + 1, ld[1]);
    __syncthreads();
    fetch(0, v[0]);
    // iteration s: the chains read stage s + 1 and add stage s; the loaders
    // store stage s + 2 (set (s + 2) % 4) and read stage s + 6 into that set
    for (long long s0 = 0; s0 < stages; s0 += kBandSets) {
#pragma unroll
        for (int j = 0; j < kBandSets; ++j) {
            const long long s = s0 + j;
            if (s < stages) {
                fetch(s + 1, v[(j + 1) & 1]);
                add(s, v[j & 1]);
                store(s + 2, ld[(j + 2) % kBandSets]);
                load(s + kBandAhead, ld[(j + 2) % kBandSets]);
            }
            __syncthreads();
        }
    }
    if (chain) lanes[l0 + t] = lane_band(acc);
}

// Group g's 128 lane bands by the halving tree into gp[g]; the last group
// to finish folds the 64 group bands by the same tree and stores h.
__global__ __launch_bounds__(256) void hawk_band_sum_fold(const Band* __restrict__ lanes, Band* __restrict__ gp,
                                                          unsigned* __restrict__ ticket, double* __restrict__ out) {
    __shared__ Band sh[kBandLanes];
    __shared__ unsigned last;
    const int g = blockIdx.x;
    const int t = threadIdx.x;
    for (int i = t; i < kBandLanes; i += 256) sh[i] = lanes[g * kBandLanes + i];
    __syncthreads();
    for (int w = kBandLanes / 2; w > 0; w >>= 1) {
        for (int i = t; i < w; i += 256) sh[i] = band_add(sh[i], sh[i + w]);
        __syncthreads();
    }
    if (t == 0) {
        gp[g] = sh[0];
        __threadfence();
        last = atomicAdd(ticket, 1u);
    }
    __syncthreads();
    if (last != kGroups - 1) return;
    __threadfence();
    if (t < kGroups) {
        sh[t].h = __builtin_nontemporal_load(&gp[t].h);
        sh[t].l = __builtin_nontemporal_load(&gp[t].l);
    }
    __syncthreads();
    for (int w = kGroups / 2; w > 0; w >>= 1) {
        if (t < w) sh[t] = band_add(sh[t], sh[t + w]);
        __syncthreads();
    }
    if (t == 0) {
        *out = sh[0].h;
        *ticket = 0u;
    }
}

// ---------------------------------------------------------------------------
// The default-policy sample sum's finish.  The per-sample stage leaves one
// compensated (hi, comp) pair per row of 32 samples; the cell is those rows
// folded in the canonical ordered tree of reference hawk/_cells.py:71-119:
// leaves of 4096 rows, each leaf's 256 slots adding rows slot, slot + 256,
// ... (16 terms) with Neumaier's compensated add, the leaf's slots folded by
// the halving tree, then the leaves folded pairwise level by level (an odd
// last one carried up), and hi + comp at the end.  A non-finite partial drops
// its compensation, so Inf and NaN follow IEEE through hi.
// ---------------------------------------------------------------------------
constexpr int kRowSlots = 256;
constexpr int kRowTerms = 16;
constexpr long long kRowLeaf = static_cast<long long>(kRowSlots) * kRowTerms;

template <class T>
__device__ __forceinline__ bool finite_bits(T x) { return (x - x) == T(0); }

// The exact residual of s == a + b, a zero residual +0, NaN when s is not
// finite (reference hawk/_cells.py:46-52, Fast2Sum on the operands ordered by
// magnitude).  Knuth's TwoSum gives the same exact residual for any finite
// a and b without the ordering's compare and selects.
template <class T>
__device__ __forceinline__ T two_sum_err(T a, T b, T s) {
    const T bb = s - a;
    return finite_bits(s) ? ((a - (s - bb)) + (b - bb)) + T(0) : T(__builtin_nan(""));
}

// Neumaier's add of (x, xc) onto (h, c) (reference hawk/_cells.py:55-58).
template <class T>
__device__ __forceinline__ void neumaier_add(T& h, T& c, T x, T xc) {
    const T s = h + x;
    const bool fin = finite_bits(s);
    c = fin ? c + two_sum_err(h, x, s) : T(0);
    c = fin ? c + xc : T(0);
    h = s;
}

// Two partials combined (reference hawk/_cells.py:61-63).
template <class T>
__device__ __forceinline__ void pair_add(T& h, T& c, T h2, T c2) {
    const T s = h + h2;
    c = finite_bits(s) ? (c + c2) + two_sum_err(h, h2, s) : T(0);
    h = s;
}

// Leaf j: rows [j*4096, min((j+1)*4096, rows)).  T is the rows' type: the
// finish runs in it, as the reference's finish runs in the rows' dtype.
template <class T>
__global__ __launch_bounds__(kRowSlots) void hawk_rows_leaves(const T* __restrict__ hi, const T* __restrict__ comp,
                                                              long long rows, T* __restrict__ leaf_h,
                                                              T* __restrict__ leaf_c) {
    __shared__ T sh[kRowSlots], sc[kRowSlots];
    const int s = threadIdx.x;
    const long long lo = static_cast<long long>(blockIdx.x) * kRowLeaf;
    const long long rest = rows - lo;
    const int cnt = rest < kRowLeaf ? static_cast<int>(rest) : static_cast<int>(kRowLeaf);
    const int live = cnt < kRowSlots ? cnt : kRowSlots;
    if (s < live) {
        T h = hi[lo + s];
        T c = finite_bits(h) ? comp[lo + s] : T(0);
        for (int k = 1; k < kRowTerms; ++k) {
            const int m = live < cnt - k * kRowSlots ? live : cnt - k * kRowSlots;
            if (m <= 0 || s >= m) break;
            neumaier_add(h, c, hi[lo + k * kRowSlots + s], comp[lo + k * kRowSlots + s]);
        }
        sh[s] = h;
        sc[s] = c;
    }
    __syncthreads();
    for (int off = kRowSlots / 2; off > 0; off >>= 1) {
        const int lim = live > off ? (off < live - off ? off : live - off) : 0;
        if (s < lim) {
            T h = sh[s], c = sc[s];
            pair_add(h, c, sh[s + off], sc[s + off]);
            sh[s] = h;
            sc[s] = c;
        }
        __syncthreads();
    }
    if (s == 0) {
        leaf_h[blockIdx.x] = sh[0];
        leaf_c[blockIdx.x] = sc[0];
    }
}

// The leaves folded pairwise level by level by one workgroup, ping-ponging
// between the two halves of the scratch; the cell gets hi + comp (hi alone
// when it is not finite).
template <class T>
__global__ __launch_bounds__(256) void hawk_rows_levels(T* __restrict__ buf, long long leaves, T* __restrict__ out) {
    T* vh = buf;
    T* vc = buf + leaves;
    T* nh = buf + 2 * leaves;
    T* nc = buf + 3 * leaves;
    long long m = leaves;
    while (m > 1) {
        const long long pairs = m / 2;
        for (long long p = threadIdx.x; p < pairs; p += 256) {
            T h = vh[2 * p], c = vc[2 * p];
            pair_add(h, c, vh[2 * p + 1], vc[2 * p + 1]);
            nh[p] = h;
            nc[p] = c;
        }
        if ((m & 1) && threadIdx.x == 0) {
            nh[pairs] = vh[m - 1];
            nc[pairs] = vc[m - 1];
        }
        __syncthreads();
        T* th = vh; vh = nh; nh = th;
        T* tc = vc; vc = nc; nc = tc;
        m = pairs + (m & 1);
    }
    if (threadIdx.x == 0) *out = finite_bits(vh[0]) ? vh[0] + vc[0] : vh[0];
}

// The rows' finish of hawk.max / hawk.min (reference hawk/_cells.py:66-71 and
// `finish`): the same tree, every add the extreme a > b ? a : b (max) or
// a < b ? a : b (min) of (the earlier partial, the later); exact, and a NaN
// partial on the left gives way to the right one.  OP 1 is max, 2 min.
template <int OP, class T>
__device__ __forceinline__ T tree_extreme(T a, T b) {
    return OP == 1 ? (a > b ? a : b) : (a < b ? a : b);
}

template <class T, int OP>
__global__ __launch_bounds__(kRowSlots) void hawk_rows_ext_leaves(const T* __restrict__ hi, long long rows,
                                                                  T* __restrict__ leaf_h) {
    __shared__ T sh[kRowSlots];
    const int s = threadIdx.x;
    const long long lo = static_cast<long long>(blockIdx.x) * kRowLeaf;
    const long long rest = rows - lo;
    const int cnt = rest < kRowLeaf ? static_cast<int>(rest) : static_cast<int>(kRowLeaf);
    const int live = cnt < kRowSlots ? cnt : kRowSlots;
    if (s < live) {
        T h = hi[lo + s];
        for (int k = 1; k < kRowTerms; ++k) {
            const int m = live < cnt - k * kRowSlots ? live : cnt - k * kRowSlots;
            if (m <= 0 || s >= m) break;
            h = tree_extreme<OP>(h, hi[lo + k * kRowSlots + s]);
        }
        sh[s] = h;
    }
    __syncthreads();
    for (int off = kRowSlots / 2; off > 0; off >>= 1) {
        const int lim = live > off ? (off < live - off ? off : live - off) : 0;
        if (s < lim) sh[s] = tree_extreme<OP>(sh[s], sh[s + off]);
        __syncthreads();
    }
    if (s == 0) leaf_h[blockIdx.x] = sh[0];
}

template <class T, int OP>
__global__ __launch_bounds__(256) void hawk_rows_ext_levels(T* __restrict__ buf, long long leaves,
                                                            T* __restrict__ out) {
    T* vh = buf;
    T* nh = buf + leaves;
    long long m = leaves;
    while (m > 1) {
        const long long pairs = m / 2;
        for (long long p = threadIdx.x; p < pairs; p += 256) nh[p] = tree_extreme<OP>(vh[2 * p], vh[2 * p + 1]);
        if ((m & 1) && threadIdx.x == 0) nh[pairs] = vh[m - 1];
        __syncthreads();
        T* th = vh; vh = nh; nh = th;
        m = pairs + (m & 1);
    }
    if (threadIdx.x == 0) *out = vh[0];
}

// The banded rows' finish: the canonical tree above (leaves of 4096 rows over
// 256 slots, the in-leaf halving tree, the leaves pairwise level by level)
// with every add a band add; the cell is the final band's h.  Row r of the
// stage is the band (hi[r], lo[r]).
__global__ __launch_bounds__(kRowSlots) void hawk_band_rows_leaves(const double* __restrict__ hi,
                                                                   const double* __restrict__ lo, long long rows,
                                                                   double* __restrict__ leaf_h,
                                                                   double* __restrict__ leaf_l) {
    __shared__ Band sh[kRowSlots];
    const int s = threadIdx.x;
    const long long first = static_cast<long long>(blockIdx.x) * kRowLeaf;
    const long long rest = rows - first;
    const int cnt = rest < kRowLeaf ? static_cast<int>(rest) : static_cast<int>(kRowLeaf);
    const int live = cnt < kRowSlots ? cnt : kRowSlots;
    if (s < live) {
        Band b{hi[first + s], lo[first + s]};
        for (int k = 1; k < kRowTerms; ++k) {
            const int m = live < cnt - k * kRowSlots ? live : cnt - k * kRowSlots;
            if (m <= 0 || s >= m) break;
            b = band_add(b, Band{hi[first + k * kRowSlots + s], lo[first + k * kRowSlots + s]});
        }
        sh[s] = b;
    }
    __syncthreads();
    for (int off = kRowSlots / 2; off > 0; off >>= 1) {
        const int lim = live > off ? (off < live - off ? off : live - off) : 0;
        if (s < lim) sh[s] = band_add(sh[s], sh[s + off]);
        __syncthreads();
    }
    if (s == 0) {
        leaf_h[blockIdx.x] = sh[0].h;
        leaf_l[blockIdx.x] = sh[0].l;
    }
}

__global__ __launch_bounds__(256) void hawk_band_rows_levels(double* __restrict__ buf, long long leaves,
                                                             double* __restrict__ out) {
    double* vh = buf;
    double* vl = buf + leaves;
    double* nh = buf + 2 * leaves;
    double* nl = buf + 3 * leaves;
    long long m = leaves;
    while (m > 1) {
        const long long pairs = m / 2;
        for (long long p = threadIdx.x; p < pairs; p += 256) {
            const Band b = band_add(Band{vh[2 * p], vl[2 * p]}, Band{vh[2 * p + 1], vl[2 * p + 1]});
            nh[p] = b.h;
            nl[p] = b.l;
        }
        if ((m & 1) && threadIdx.x == 0) {
            nh[pairs] = vh[m - 1];
            nl[pairs] = vl[m - 1];
        }
        __syncthreads();
        double* th = vh; vh = nh; nh = th;
        double* tl = vl; vl = nl; nl = tl;
        m = pairs + (m & 1);
    }
    if (threadIdx.x == 0) *out = vh[0];
}

// hawk.sum(x, over=<trailing lane axes>) under the default policy: key k's
// `group` consecutive values are summed as a sample sum of their own.  Rows
// of 32 run from the key's first value (a ragged last row padded with +0),
// each a compensated (hi, comp) pair by the pairs (l, l ^ 16), ..., (l, l ^ 1)
// of a half-wave; the rows fold in the canonical tree above (leaves of 4096
// rows over 256 slots with Neumaier's add, the halving tree, the leaves
// pairwise level by level) and the key's cell is hi + comp.  One workgroup a
// key; row r lands in slot r % 256 and every slot adds its rows in order.
constexpr long long kKeyedCompLeaves = kRowSlots;        // leaves a key may span

template <class T>
__device__ __forceinline__ void row_pair_sum(T& h, T& c) {
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) {
        const T h2 = __shfl_xor(h, off, 64);
        const T c2 = __shfl_xor(c, off, 64);
        const T s = h + h2;
        c = finite_bits(s) ? (c + c2) + two_sum_err(h, h2, s) : T(0);
        h = s;
    }
}

template <class T>
__global__ __launch_bounds__(kRowSlots) void hawk_keyed_comp(const T* __restrict__ u, long long group,
                                                             T* __restrict__ out) {
    __shared__ T sh[kRowSlots], sc[kRowSlots], lh[kKeyedCompLeaves], lc[kKeyedCompLeaves];
    const int t = threadIdx.x, half = t >> 5, l = t & 31;
    const T* __restrict__ mine = u + static_cast<long long>(blockIdx.x) * group;
    const long long rows = (group + 31) / 32;
    const long long leaves = (rows + kRowLeaf - 1) / kRowLeaf;
    for (long long j = 0; j < leaves; ++j) {
        const long long lo = j * kRowLeaf;
        const int cnt = static_cast<int>(rows - lo < kRowLeaf ? rows - lo : kRowLeaf);
        const int live = cnt < kRowSlots ? cnt : kRowSlots;
        // Half-wave `half` takes rows half, half + 8, ... in increasing order.
        // Slot s gets rows s, s + 256, ..., all from the one half-wave (256 is
        // a multiple of 8), so each slot's adds keep row order with no
        // barrier; four rows' loads are in flight at a time.
        for (int rb0 = 0; rb0 < cnt; rb0 += 32) {       // the same trips for every lane
            const int rb = rb0 + half;
            T x[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int r = rb + 8 * q;
                const long long at = (lo + r) * 32 + l;
                x[q] = (r < cnt && at < group) ? __builtin_nontemporal_load(mine + at) : T(0);
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int r = rb + 8 * q;
                T h = x[q], c = T(0);
                row_pair_sum<T>(h, c);
                if (l == 0 && r < cnt) {
                    const int slot = r & (kRowSlots - 1);
                    if (r < kRowSlots) {
                        sh[slot] = h;
                        sc[slot] = finite_bits(h) ? c : T(0);
                    } else {
                        T a = sh[slot], b = sc[slot];
                        neumaier_add(a, b, h, c);
                        sh[slot] = a;
                        sc[slot] = b;
                    }
                }
            }
        }
        __syncthreads();
        for (int off = kRowSlots / 2; off > 0; off >>= 1) {
            const int lim = live > off ? (off < live - off ? off : live - off) : 0;
            if (t < lim) {
                T h = sh[t], c = sc[t];
                pair_add(h, c, sh[t + off], sc[t + off]);
                sh[t] = h;
                sc[t] = c;
            }
            __syncthreads();
        }
        if (t == 0) {
            lh[j] = sh[0];
            lc[j] = sc[0];
        }
        __syncthreads();
    }
    if (t == 0) {
        long long m = leaves;
        while (m > 1) {               // in place: pair p reads slots 2p, 2p + 1 >= p
            const long long pairs = m / 2;
            for (long long p = 0; p < pairs; ++p) {
                T h = lh[2 * p], c = lc[2 * p];
                pair_add(h, c, lh[2 * p + 1], lc[2 * p + 1]);
                lh[p] = h;
                lc[p] = c;
            }
            if (m & 1) {
                lh[pairs] = lh[m - 1];
                lc[pairs] = lc[m - 1];
            }
            m = pairs + (m & 1);
        }
        out[blockIdx.x] = finite_bits(lh[0]) ? lh[0] + lc[0] : lh[0];
    }
}

// Keys of at most 64 rows (2048 samples): one wave a key, four keys a block.
// The wave's halves sum two rows a step into the wave's slots (row r in slot
// r: fewer than 256 rows, so no slot takes a second row), then the halving
// tree over the R live slots, as the leaf above: the same bits.  A wave past
// the last key computes nothing but meets every barrier.
template <class T>
__global__ __launch_bounds__(256) void hawk_keyed_comp_wave(const T* __restrict__ u, long long group,
                                                            long long keys, T* __restrict__ out) {
    __shared__ T sh[4][64], sc[4][64];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, half = lane >> 5, l = lane & 31;
    const long long k = static_cast<long long>(blockIdx.x) * 4 + w;
    const bool live = k < keys;
    const T* __restrict__ mine = u + (live ? k : 0) * group;
    const int rows = static_cast<int>((group + 31) / 32);
    for (int rb = 0; rb < rows; rb += 2) {
        const int r = rb + half;
        const long long at = static_cast<long long>(r) * 32 + l;
        T h = (live && r < rows && at < group) ? __builtin_nontemporal_load(mine + at) : T(0), c = T(0);
        row_pair_sum<T>(h, c);
        if (l == 0 && r < rows) {
            sh[w][r] = h;
            sc[w][r] = finite_bits(h) ? c : T(0);
        }
    }
    __syncthreads();
    for (int off = 32; off > 0; off >>= 1) {
        const int lim = rows > off ? (off < rows - off ? off : rows - off) : 0;
        T h = T(0), c = T(0);
        if (lane < lim) {
            h = sh[w][lane];
            c = sc[w][lane];
            pair_add(h, c, sh[w][lane + off], sc[w][lane + off]);
        }
        __syncthreads();
        if (lane < lim) {
            sh[w][lane] = h;
            sc[w][lane] = c;
        }
        __syncthreads();
    }
    if (live && lane == 0) out[k] = finite_bits(sh[w][0]) ? sh[w][0] + sc[w][0] : sh[w][0];
}

// ---------------------------------------------------------------------------
// Keyed fixed-tree sum: hawk.sum(x, over=<trailing lane axes>, policy=
// "ordered").  Key k's rows are the `group` consecutive values
// u[k*group .. (k+1)*group), and each key takes the ordered sum's tree
// (reference hawk/emit/team.py:115-205 with its gp stage): virtual lane l of
// 65536 adds rows l, l + 65536, ... from +0.0, groups of 1024 lanes fold by
// the halving tree, then the 64 group values by the same tree.
//
// Only the first lv = min(group, 65536) lanes of a key can hold rows; the
// others are +0.0, and so are the groups past ceil(lv / 1024).  No lane value
// or tree sum is ever -0.0 (each starts at +0.0; a round-to-nearest sum is
// -0.0 only from two -0.0 operands), so adding +0.0 is the identity and the
// trees need only their first P = min(1024, 2^ceil(log2 lv)) lanes and first
// Q = 2^ceil(log2 groups) group values: the bits of the full trees.
// ---------------------------------------------------------------------------
template <class T>
__global__ __launch_bounds__(256) void hawk_keyed_lanes(const T* __restrict__ u, long long group, long long lv,
                                                        long long total, T* __restrict__ lanes) {
    for (long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x; i < total;
         i += static_cast<long long>(gridDim.x) * 256) {
        const long long k = i / lv, l = i - k * lv;
        const T* row = u + k * group;
        T part = T(0);
        for (long long r = l; r < group; r += kVirtualLanes) part = part + __builtin_nontemporal_load(row + r);
        lanes[i] = part;
    }
}

__host__ __device__ __forceinline__ int pow2_at_least(long long x) {
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}

// The halving tree s[i] += s[i + w], w = P/2 .. 1, of P <= 1024 values (a
// power of 2; zeros past the data) held by a 256-thread workgroup as
// s[t + 256j] = v[j]: the levels w = 512 and 256 pair values of one thread,
// w = 128 and 64 go through LDS, w = 32 .. 1 through the first wave's
// shuffles (lane i reads lane i + w; only lanes below w carry on).  The
// same pairs, in the same order, as the tree over LDS.  Thread 0 returns s[0].
template <class T>
__device__ __forceinline__ T block_tree(T (&v)[4], int P, T* sh) {
    const int t = threadIdx.x;
    if (P > 512) { v[0] = v[0] + v[2]; v[1] = v[1] + v[3]; }
    if (P > 256) v[0] = v[0] + v[1];
    T x = v[0];
    if (P > 64) {
        sh[t] = x;
        __syncthreads();
        if (P > 128 && t < 128) sh[t] = sh[t] + sh[t + 128];
        __syncthreads();
        if (t < 64) x = sh[t] + sh[t + 64];
    }
    if (t < 64) {
#pragma unroll
        for (int w = 32; w >= 1; w >>= 1) {
            const T y = __shfl_down(x, w, 64);
            if (P > w) x = x + y;
        }
    }
    __syncthreads();                      // sh is free for the next tree
    return x;
}

// The 64 group values' tree over Q = 2^ceil(log2 used) of them, in the first wave.
template <class T>
__device__ __forceinline__ T group_tree(const T* gp, int used) {
    const int t = threadIdx.x;
    const int q = pow2_at_least(used);
    T x = t < used ? gp[t] : T(0);
#pragma unroll
    for (int w = 32; w >= 1; w >>= 1) {
        const T y = __shfl_down(x, w, 64);
        if (q > w) x = x + y;
    }
    return x;
}

// One workgroup per key whose lanes are already folded into `lanes` (groups
// of more than 65536 rows): the used groups' trees, then the group values'.
template <class T>
__global__ __launch_bounds__(256) void hawk_keyed_fold(const T* __restrict__ lanes, long long lv,
                                                       T* __restrict__ out) {
    __shared__ T sh[256];
    __shared__ T gp[kGroups];
    const long long k = blockIdx.x;
    const int t = threadIdx.x;
    const int used = static_cast<int>((lv + kFoldLanes - 1) / kFoldLanes);     // <= 64
    const int width = lv >= kFoldLanes ? kFoldLanes : pow2_at_least(lv);
    const T* mine = lanes + k * lv;
    for (int g = 0; g < used; ++g) {
        T v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const long long at = static_cast<long long>(g) * kFoldLanes + t + 256 * j;
            v[j] = at < lv ? mine[at] : T(0);
        }
        const T s = block_tree<T>(v, width, sh);
        if (t == 0) gp[g] = s;
    }
    __syncthreads();
    const T total = t < 64 ? group_tree<T>(gp, used) : T(0);
    if (t == 0) out[k] = total;
}

// One workgroup per key of at most 65536 rows: virtual lane l holds row l
// alone (0.0 + u[l], the add from +0.0), so the trees read u directly.
template <class T>
__global__ __launch_bounds__(256) void hawk_keyed_rows(const T* __restrict__ u, long long group,
                                                       T* __restrict__ out) {
    __shared__ T sh[256];
    __shared__ T gp[kGroups];
    const long long k = blockIdx.x;
    const int t = threadIdx.x;
    const int used = static_cast<int>((group + kFoldLanes - 1) / kFoldLanes);
    const int width = group >= kFoldLanes ? kFoldLanes : pow2_at_least(group);
    const T* mine = u + k * group;
    T nxt[4];                        // the next group's rows, loaded during this group's tree
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const long long at = t + 256 * j;
        nxt[j] = at < group ? __builtin_nontemporal_load(mine + at) : T(0);
    }
    for (int g = 0; g < used; ++g) {
        T v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const long long at = static_cast<long long>(g) * kFoldLanes + t + 256 * j;
            v[j] = at < group ? T(0) + nxt[j] : T(0);
        }
        if (g + 1 < used) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const long long at = static_cast<long long>(g + 1) * kFoldLanes + t + 256 * j;
                nxt[j] = at < group ? __builtin_nontemporal_load(mine + at) : T(0);
            }
        }
        const T s = block_tree<T>(v, width, sh);
        if (t == 0) gp[g] = s;
    }
    __syncthreads();
    const T total = t < 64 ? group_tree<T>(gp, used) : T(0);
    if (t == 0) out[k] = total;
}

// Keys of at most 64 rows: a wave holds 64 / P keys, P = 2^ceil(log2 group),
// in segments of P lanes (lane j of a segment holds row j, 0.0 + u, or +0.0
// past the key's rows), and each segment runs the halving tree by shuffles
// (lane j adds lane j + w for w = P/2 .. 1; only lanes below w carry on): the
// pairs of the tree over P values.  The group tree has one value, which it
// returns unchanged.
template <class T>
__global__ __launch_bounds__(256) void hawk_keyed_small(const T* __restrict__ u, long long group, int P,
                                                        long long keys, T* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    const long long per_wave = 64 / P;
    const long long k = (static_cast<long long>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * per_wave + lane / P;
    const int j = lane & (P - 1);
    T x = T(0);
    if (k < keys && j < group) x = T(0) + __builtin_nontemporal_load(u + k * group + j);
#pragma unroll
    for (int w = 32; w >= 1; w >>= 1) {
        const T y = __shfl_down(x, w, 64);
        if (P > w) x = x + y;
    }
    if (j == 0 && k < keys) out[k] = x;
}

// ---------------------------------------------------------------------------
// Keyed ordered scatter.
//
// parts[b][k] is the in-lane-order sum (from +0.0) of chunk b's values with
// key k; cell k then adds parts[0][k], parts[1][k], ... in chunk order from
// +0.0 and adds that onto target[k].  Up to 65536 cells the split walk below
// makes those additions.  Past that, one 1024-thread workgroup walks one chunk
// in tiles of 4096 lanes: each tile is sorted stably by key in LDS (LSD radix,
// 8-bit digits), so every key's lanes form one run in lane order, and the
// run's owner thread adds them one by one onto the key's accumulator — the
// additions the serial walk makes, in its order.  Accumulators of keys below
// kAccKeys live in LDS, the others in the zero-filled parts[b] (only this
// workgroup touches that row).
// ---------------------------------------------------------------------------
constexpr int kScatterChunks = 256;    // reference hawk/_lane_bind.py:108
constexpr int kWalkThreads = 1024;
constexpr int kWalkWaves = kWalkThreads / 64;
constexpr int kWalkItems = 4;                      // lanes per thread per tile
constexpr int kTile = kWalkThreads * kWalkItems;   // 4096 lanes per tile
constexpr int kPosBits = 12;                       // 2^12 == kTile
constexpr unsigned kPosMask = (1u << kPosBits) - 1u;
constexpr unsigned kInvalid = 0x80000000u;         // a skipped (-1), bad or padding lane
constexpr int kMaxKeyBits = 31 - kPosBits;         // key field: bits 12..30
constexpr int kDigitBits = 8;
constexpr int kDigits = 1 << kDigitBits;
constexpr int kHistRow = kWalkWaves + 1;          // one digit's per-wave counts, padded: rows in different banks
constexpr int kAccKeys = 4096;                     // keys whose accumulators live in LDS
constexpr int kFoldUnroll = 8;

static_assert(kTile == 1 << kPosBits, "tile positions fill the position field");

// Inclusive scan over the 64 lanes of a wave in DPP moves, no LDS: within
// each row of 16 lanes by row shifts 1, 2, 4, 8 (a lane past the row's start
// adds 0), then row 15's total into rows 1 and 3 and lane 31's into rows 2
// and 3 (row broadcasts).
__device__ __forceinline__ unsigned wave_inclusive_scan(unsigned x) {
    x += __builtin_amdgcn_update_dpp(0u, x, 0x111, 0xf, 0xf, false);   // row_shr:1
    x += __builtin_amdgcn_update_dpp(0u, x, 0x112, 0xf, 0xf, false);   // row_shr:2
    x += __builtin_amdgcn_update_dpp(0u, x, 0x114, 0xf, 0xf, false);   // row_shr:4
    x += __builtin_amdgcn_update_dpp(0u, x, 0x118, 0xf, 0xf, false);   // row_shr:8
    x += __builtin_amdgcn_update_dpp(0u, x, 0x142, 0xa, 0xf, false);   // row_bcast:15 into rows 1, 3
    x += __builtin_amdgcn_update_dpp(0u, x, 0x143, 0xc, 0xf, false);   // row_bcast:31 into rows 2, 3
    return x;
}

template <class T>
struct WalkShared {
    T vals[kTile];                               // 32 KiB: the tile's values, lane order
    unsigned ent[2][kTile];                           // 32 KiB: (key << 12) | position | invalid
    unsigned hist[kDigits][kHistRow];                 // 17 KiB: [digit][wave] counts, then offsets
    union {
        unsigned long long peer[kWalkWaves][kDigits]; // 32 KiB: per-wave lane masks of one digit (sort)
        T sv[kTile];                             //         the tile's values in sorted order (fold)
    };
    T acc[kAccKeys];                             // 32 KiB: accumulators of keys < kAccKeys
    unsigned long long starts[kTile / 64];            // run heads of the sorted tile
    unsigned wsum[kWalkWaves];
};

// Stable LSD radix sort of the tile's entries by the key field (bits
// 12..12+key_bits), 8 bits a pass, ping-ponging ent[0] <-> ent[1]; returns the
// buffer holding the result.  Wave w ranks its 256 entries w*256 + j*64 + lane
// window by window (j = 0..3, in order): the lanes of a window holding digit d
// find each other through one LDS OR into peer[w][d]; the lowest of them adds
// the group's size onto hist[d][w] after all of them read it.  The exclusive
// scan of hist in (digit, wave) order then places every wave's group after
// the earlier waves' groups of the same digit, so each pass keeps input order
// within a digit.
template <class T>
__device__ int walk_sort(WalkShared<T>& sh, int key_bits) {
    const int t = threadIdx.x;
    const int wave = t >> 6;
    const int lane = t & 63;
    const unsigned long long me = 1ull << lane;
    int src = 0;
    for (int lo = 0; lo < key_bits; lo += kDigitBits) {
        const int width = key_bits - lo < kDigitBits ? key_bits - lo : kDigitBits;
        const unsigned dmask = (1u << width) - 1u;
        const int shift = kPosBits + lo;
        const unsigned* in = sh.ent[src];
        unsigned* out = sh.ent[src ^ 1];
        for (int d = lane; d < kDigits; d += 64) sh.hist[d][wave] = 0u;
        __builtin_amdgcn_wave_barrier();
        unsigned item[kWalkItems], digit[kWalkItems], rank[kWalkItems];
#pragma unroll
        for (int j = 0; j < kWalkItems; ++j) item[j] = in[wave * (kWalkItems * 64) + j * 64 + lane];
#pragma unroll
        for (int j = 0; j < kWalkItems; ++j) {
            digit[j] = (item[j] >> shift) & dmask;
            atomicOr(&sh.peer[wave][digit[j]], me);
            __builtin_amdgcn_wave_barrier();
            const unsigned long long peers = sh.peer[wave][digit[j]];
            const unsigned below = __builtin_amdgcn_mbcnt_hi(static_cast<unsigned>(peers >> 32),
                                                             __builtin_amdgcn_mbcnt_lo(static_cast<unsigned>(peers), 0u));
            const unsigned old = sh.hist[digit[j]][wave];
            rank[j] = old + below;
            __builtin_amdgcn_wave_barrier();
            if (below == 0u) {
                sh.hist[digit[j]][wave] = old + static_cast<unsigned>(__popcll(peers));
                sh.peer[wave][digit[j]] = 0ull;
            }
            __builtin_amdgcn_wave_barrier();
        }
        __syncthreads();
        // Exclusive scan over f = digit*16 + wave: thread t owns f = 4t .. 4t+3.
        const int d = t >> 2;
        const int w0 = (t & 3) * 4;
        const unsigned c0 = sh.hist[d][w0], c1 = sh.hist[d][w0 + 1];
        const unsigned c2 = sh.hist[d][w0 + 2], c3 = sh.hist[d][w0 + 3];
        const unsigned mine = c0 + c1 + c2 + c3;
        const unsigned incl = wave_inclusive_scan(mine);
        if (lane == 63) sh.wsum[wave] = incl;
        __syncthreads();
        unsigned before = 0u;
        for (int w = 0; w < wave; ++w) before += sh.wsum[w];
        const unsigned base = incl - mine + before;
        sh.hist[d][w0] = base;
        sh.hist[d][w0 + 1] = base + c0;
        sh.hist[d][w0 + 2] = base + c0 + c1;
        sh.hist[d][w0 + 3] = base + c0 + c1 + c2;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kWalkItems; ++j) out[sh.hist[digit[j]][wave] + rank[j]] = item[j];
        __syncthreads();
        src ^= 1;
    }
    return src;
}

// Lane base + wave*256 + j*64 + lane goes to thread slot j: every load
// instruction of a wave reads 64 consecutive lanes.  Lanes past `hi` read as
// the skip key -1.
template <class T>
__device__ __forceinline__ void walk_load(const int* __restrict__ key, const T* __restrict__ v, long long base,
                                          long long hi, int (&kk)[kWalkItems], T (&vv)[kWalkItems]) {
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < kWalkItems; ++j) {
        const long long i = base + wave * (kWalkItems * 64) + j * 64 + lane;
        const bool in = i < hi;
        kk[j] = in ? __builtin_nontemporal_load(key + i) : -1;
        vv[j] = in ? __builtin_nontemporal_load(v + i) : T(0);
    }
}

// The first run head after position i of the sorted tile (kTile if none).
template <class T>
__device__ __forceinline__ int next_head(const WalkShared<T>& sh, int i) {
    int wi = i >> 6;
    const int bit = i & 63;
    unsigned long long m = bit == 63 ? 0ull : (sh.starts[wi] & (~0ull << (bit + 1)));
    while (m == 0ull && ++wi < kTile / 64) m = sh.starts[wi];
    return m ? (wi << 6) + __builtin_ctzll(m) : kTile;
}

// a + x[s] + x[s+1] + ... + x[e-1], one addition at a time in that order; the
// next eight values are in flight while the current eight are added.
template <class T>
__device__ __forceinline__ T fold_run(const T* x, int s, int e, T a) {
    int m = s;
    if (e - m >= 2 * kFoldUnroll) {
        T cur[kFoldUnroll];
#pragma unroll
        for (int q = 0; q < kFoldUnroll; ++q) cur[q] = x[m + q];
        m += kFoldUnroll;
        for (; m + kFoldUnroll <= e; m += kFoldUnroll) {
            T nxt[kFoldUnroll];
#pragma unroll
            for (int q = 0; q < kFoldUnroll; ++q) nxt[q] = x[m + q];
#pragma unroll
            for (int q = 0; q < kFoldUnroll; ++q) a = a + cur[q];
#pragma unroll
            for (int q = 0; q < kFoldUnroll; ++q) cur[q] = nxt[q];
        }
#pragma unroll
        for (int q = 0; q < kFoldUnroll; ++q) a = a + cur[q];
    }
    for (; m < e; ++m) a = a + x[m];
    return a;
}

// Accumulators outside LDS are read and written at agent scope, so a value
// one thread stores in a tile is what another thread of the workgroup loads
// after the tile's closing barrier.
template <class T>
__device__ __forceinline__ T acc_load(const T* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ void acc_store(T* p, T x) {
    __hip_atomic_store(p, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One workgroup per chunk b: lanes [b*span, min((b+1)*span, n)); parts
// arrives zero-filled.
template <class T>
__global__ __launch_bounds__(kWalkThreads) void hawk_scatter_walk(
        const int* __restrict__ key, const T* __restrict__ v, long long n, long long cells, long long span,
        int key_bits, T* __restrict__ parts, int* __restrict__ status) {
    __shared__ WalkShared<T> sh;
    const int t = threadIdx.x;
    const int wave = t >> 6;
    const int lane = t & 63;
    const int b = blockIdx.x;
    const long long lo = static_cast<long long>(b) * span;
    const long long hi = lo + span < n ? lo + span : n;
    const int acc_n = cells < kAccKeys ? static_cast<int>(cells) : kAccKeys;
    const unsigned kmask = (1u << key_bits) - 1u;
    const unsigned sentinel = kmask;          // the key field of an invalid lane
    T* row = parts + static_cast<long long>(b) * cells;

    for (int k = t; k < acc_n; k += kWalkThreads) sh.acc[k] = T(0);
    bool bad = false;
    int nk[kWalkItems];
    T nv[kWalkItems];
    if (lo < hi) walk_load(key, v, lo, hi, nk, nv);
    __syncthreads();
    for (long long base = lo; base < hi; base += kTile) {
        int kk[kWalkItems];
        T vv[kWalkItems];
#pragma unroll
        for (int j = 0; j < kWalkItems; ++j) { kk[j] = nk[j]; vv[j] = nv[j]; }
        if (base + kTile < hi) walk_load(key, v, base + kTile, hi, nk, nv);
#pragma unroll
        for (int j = 0; j < kWalkItems; ++j) {
            const unsigned p = static_cast<unsigned>(wave * (kWalkItems * 64) + j * 64 + lane);
            const bool valid = kk[j] >= 0 && kk[j] < cells;
            bad = bad || (kk[j] != -1 && !valid);
            const unsigned field = valid ? static_cast<unsigned>(kk[j]) : sentinel;
            sh.ent[0][p] = (field << kPosBits) | p | (valid ? 0u : kInvalid);
            sh.vals[p] = vv[j];
            // the previous tile's sorted values share LDS with the sort's peer
            // masks, which must start at zero
            (&sh.peer[0][0])[p] = 0ull;
        }
        __syncthreads();
        const unsigned* sorted = sh.ent[walk_sort(sh, key_bits)];
        // The values in sorted order (an invalid lane's as +0.0) and the run
        // heads, one ballot per 64 entries.
        bool head[kWalkItems];
#pragma unroll
        for (int j = 0; j < kWalkItems; ++j) {
            const int i = j * kWalkThreads + t;
            const unsigned e = sorted[i];
            sh.sv[i] = (e & kInvalid) ? T(0) : sh.vals[e & kPosMask];
            const unsigned k = (e >> kPosBits) & kmask;
            head[j] = i == 0 || k != ((sorted[i - (i > 0)] >> kPosBits) & kmask);
            const unsigned long long m = __ballot(head[j]);
            if (lane == 0) sh.starts[(j * kWalkThreads + wave * 64) >> 6] = m;
        }
        __syncthreads();
        // Every run's owner: its accumulator first (the loads of all its runs
        // in flight together), then its lanes in order, then the store.
        int rs[kWalkItems], re[kWalkItems];
        unsigned rk[kWalkItems];
        bool load[kWalkItems];
#pragma unroll
        for (int j = 0; j < kWalkItems; ++j) {
            rs[j] = j * kWalkThreads + t;
            rk[j] = (sorted[rs[j]] >> kPosBits) & kmask;
            re[j] = 0;
            load[j] = false;
            if (!head[j] || rk[j] >= cells) continue;
            re[j] = next_head(sh, rs[j]);
            const unsigned k = rk[j];
            load[j] = k >= static_cast<unsigned>(acc_n);
        }
        T ra[kWalkItems];
#pragma unroll
        for (int j = 0; j < kWalkItems; ++j) {
            const unsigned k = rk[j] < static_cast<unsigned>(acc_n) ? rk[j] : 0u;
            ra[j] = load[j] ? acc_load(row + rk[j])
                            : (re[j] != 0 && rk[j] < static_cast<unsigned>(acc_n) ? sh.acc[k] : T(0));
        }
#pragma unroll 1
        for (int j = 0; j < kWalkItems; ++j) {
            if (re[j] == 0) continue;
            const unsigned k = rk[j];
            T a = ra[j];
            bool any = true;
            if (k == sentinel) {
                // The one run that can hold invalid lanes: skip them.
                any = false;
                for (int m = rs[j]; m < re[j]; ++m) {
                    if (sorted[m] & kInvalid) continue;
                    a = a + sh.sv[m];
                    any = true;
                }
            } else {
                a = fold_run(sh.sv, rs[j], re[j], a);
            }
            if (!any) continue;
            if (k < static_cast<unsigned>(acc_n)) sh.acc[k] = a;
            else acc_store(row + k, a);
        }
        __syncthreads();
    }
    for (int k = t; k < acc_n; k += kWalkThreads) row[k] = sh.acc[k];
    if (bad) status[1 + b] = 1;
}

// More keys than the sort's key field holds: one thread per chunk walks its
// lanes in order onto the zero-filled parts[b] (the reference's serial walk).
template <class T>
__global__ __launch_bounds__(64) void hawk_scatter_serial(const int* __restrict__ key, const T* __restrict__ v,
                                                          long long n, long long cells, long long span,
                                                          T* __restrict__ parts, int* __restrict__ status) {
    if (threadIdx.x != 0) return;
    const int b = blockIdx.x;
    const long long lo = static_cast<long long>(b) * span;
    const long long hi = lo + span < n ? lo + span : n;
    T* row = parts + static_cast<long long>(b) * cells;
    bool bad = false;
    for (long long i = lo; i < hi; ++i) {
        const int k = key[i];
        if (k == -1) continue;
        if (k < 0 || k >= cells) { bad = true; continue; }
        row[k] = row[k] + v[i];
    }
    if (bad) status[1 + b] = 1;
}

template <class T>
__global__ __launch_bounds__(256) void hawk_fill_zero(T* __restrict__ p, long long count) {
    for (long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x; i < count;
         i += static_cast<long long>(gridDim.x) * 256)
        p[i] = T(0);
}

// Cell c adds its chunk partials in chunk order from +0.0, then onto the
// target: target[c] += sum (reference hawk/emit/team.py:437-460).  Two blocks
// of kAhead chunks are in flight while a third is added: 64 loads a thread,
// since a grid of one thread per cell (65536 at the split walk's largest)
// holds only a wave or two per SIMD to cover HBM's latency.
template <class T>
__global__ __launch_bounds__(256) void hawk_scatter_cells(const T* __restrict__ parts, long long cells,
                                                          int chunks, T* __restrict__ target) {
    const long long c = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    if (c >= cells) return;
    constexpr int kAhead = 32;
    auto fetch = [&](int b, T (&x)[kAhead]) {
#pragma unroll
        for (int q = 0; q < kAhead; ++q) {
            // past the last chunk a partial reads as +0.0, which adds nothing
            // to a sum that is never -0.0
            const int bq = b + q < chunks ? b + q : chunks - 1;
            const T p = parts[static_cast<long long>(bq) * cells + c];
            x[q] = b + q < chunks ? p : T(0);
        }
    };
    T x0[kAhead], x1[kAhead];
    fetch(0, x0);
    fetch(kAhead, x1);
    T s = T(0);
    for (int b = 0; b < chunks; b += kAhead) {
        T x2[kAhead];
        fetch(b + 2 * kAhead, x2);
#pragma unroll
        for (int q = 0; q < kAhead; ++q) s = s + x0[q];
#pragma unroll
        for (int q = 0; q < kAhead; ++q) {
            x0[q] = x1[q];
            x1[q] = x2[q];
        }
    }
    target[c] = target[c] + s;
}

__global__ void hawk_scatter_status(int* status, long long cells) {
    const int t = threadIdx.x;
    if (t == 0) status[0] = static_cast<int>(cells);
    if (t < kScatterChunks) status[1 + t] = 0;
}

// ---- the split walk: the ordered scatter into at most 65536 cells ----------
// The same additions as hawk_scatter_walk (each (chunk, key) sum in lane order
// from +0.0), with every accumulator in LDS, so no partial is read back from
// memory while a chunk is walked:
//
// * hawk_split_hot: one workgroup per chunk, keys [0, kSplitHot) in LDS.  Each
//   tile of 4096 lanes is split stably into buckets in one pass: window keys
//   0..31 each a bucket of their own, keys 32..kSplitHot-1 fifteen classes by
//   (key - 32) % 15, and keys from kSplitHot up one bucket per tail range of
//   kTailRange keys.  Wave 0 then folds the head buckets (lane c the chain of
//   key c over its contiguous run) and wave w class w - 1 (64 entries at a
//   time: equal keys find each other, and the lowest lane adds its group in
//   lane order onto the key's accumulator; a wave's LDS operations complete in
//   issue order, so a key's groups meet the accumulator window after window).
//   The tail buckets go from registers to the tile's slot of the chunk's bin,
//   with the offset of each range.
// * hawk_split_tail: one workgroup of 8 waves per (chunk, tail range), the
//   range's keys in LDS, two workgroups a CU; it reads the range's segment of
//   every slot in tile order (lane order), a batch of 2048 entries at a time,
//   and folds them in eight classes by key & 7 as above.
//
// Both write every key's accumulator of their window to parts[b] (+0.0 for a
// key no lane named); hawk_scatter_cells then adds the partials in chunk order.
constexpr int kSplitHot = 12288;                 // keys hawk_split_hot keeps in LDS (96 KiB of accumulators)
constexpr int kTailRange = 6144;                 // keys a hawk_split_tail workgroup keeps in LDS (48 KiB)
constexpr long long kSplitCells = 65536;         // the split walk's largest cell count
constexpr int kSplitMaxRanges = static_cast<int>((kSplitCells - kSplitHot + kTailRange - 1) / kTailRange);  // 9
constexpr int kSplitHeads = 32;                  // buckets 0..31: window keys 0..31, a chain each
constexpr int kSplitClassBase = kSplitHeads;     // classes from bucket 32 (hot: 32..46; tail: 32..39)
constexpr int kSplitTailBase = kSplitClassBase + 16;   // 48..56: hawk_split_hot's tail ranges
constexpr int kSplitNone = 63;                   // a lane that adds nothing (skip key, bad key, padding)
constexpr int kHotStride = kSplitTailBase + kSplitMaxRanges + 3;   // 60: a wave's row of bucket counts
constexpr int kTailClassBits = 3;                // hawk_split_tail's classes: key & 7
constexpr int kTailClasses = 1 << kTailClassBits;
constexpr int kTailStride = kSplitClassBase + kTailClasses + 8;   // 48
constexpr int kTailKeys = kTailRange >> kTailClassBits;   // 768 keys a class
constexpr int kTailWaves = kTailClasses;         // a wave per class
constexpr int kTailThreads = 64 * kTailWaves;
constexpr int kTailBatch = kTailThreads * kWalkItems;   // 2048 entries a batch

static_assert(kSplitHot - kSplitHeads < (1 << 15), "hot_class_index is exact below 2^15");
static_assert((kSplitHot - kSplitHeads) / 15 < 1024 && (kTailRange >> kTailClassBits) <= 1024,
              "class matching covers a class index of ten bits");
static_assert(kHotStride >= kSplitTailBase + kSplitMaxRanges + 1, "bucket starts need one past the last bucket");
static_assert(kTailStride >= kSplitClassBase + kTailClasses + 1, "bucket starts need one past the last bucket");
static_assert(kSplitNone >= kHotStride && kSplitNone >= kTailStride, "the no-bucket code is outside the count rows");
static_assert(kTailRange < (1 << 16), "bins hold window-local keys as u16");

constexpr int kSplitPad = 72;                    // entries read (and ignored) past a run's end
constexpr unsigned kPeerSlots = 128;             // a class fold's match slots: class-index bits 0..6
constexpr int kHeadBlock = 8;                    // a head chain's reads in flight: four blocks of kHeadBlock
static_assert(4 * kHeadBlock <= kSplitPad, "a head chain reads at most kSplitPad entries past its run");

// A split walk workgroup's LDS: Waves waves, Window accumulators, count rows
// of Stride buckets, and the split tile (Waves * 256 entries).
template <class T, int Waves, int Window, int Stride>
struct SplitShared {
    static constexpr int kWaves = Waves;
    static constexpr int kStride = Stride;
    static constexpr int kSpan = Waves * 64 * kWalkItems;
    T acc[Window];                              // the window's accumulators
    T val[kSpan + kSplitPad];                   // the tile's values, bucket order
    unsigned short key[kSpan + kSplitPad];      // their window-local keys
    union {                                     // one phase at a time:
        unsigned long long win[Waves][Stride];                 // split: a match table per wave
        struct {
            unsigned long long peer[Waves][kPeerSlots];        // fold: per-wave match masks
        } f;
    };
    unsigned cnt[Waves][Stride];                // bucket counts, a row per wave (lane b reads word b)
    unsigned bstart[Stride + 1];                // bucket d holds [bstart[d], bstart[d+1])
};
template <class T>
using HotShared = SplitShared<T, kWalkWaves, kSplitHot, kHotStride>;      // 157 KiB (float64)
template <class T>
using TailShared = SplitShared<T, kTailWaves, kTailRange, kTailStride>;   // 78 KiB (float64): two a CU
static_assert(sizeof(TailShared<double>) <= 80 * 1024, "two tail workgroups share a CU's 160 KiB");

// The bucket of window-local key kl (0 <= kl < window) in hawk_split_hot:
// keys 0..31 a head bucket each; keys from 32 up one of fifteen classes by
// (kl - 32) % 15, so the fifteen class waves share the window evenly.
__device__ __forceinline__ unsigned hot_class_index(unsigned kl) {   // (kl - 32) / 15, exact below 2^15
    return ((kl - static_cast<unsigned>(kSplitHeads)) * 34953u) >> 19;
}
// hawk_split_tail keeps a class's accumulators together (class c = kl & 7 at
// [768c, 768c + 768), key index m = kl >> 3), so a class wave's reads and
// writes of distinct keys spread over the LDS banks; in key order all of a
// class's keys sit 64 bytes apart, on four bank positions.  m is XORed with
// 8c, which keeps it below 768 and turns the final store's reads (eight
// classes a wave) from eight-way bank conflicts into two-way ones.
__device__ __forceinline__ unsigned tail_slot(unsigned kl) {
    const unsigned c = kl & (kTailClasses - 1u);
    return c * static_cast<unsigned>(kTailKeys) + ((kl >> kTailClassBits) ^ (c << 3));
}
__device__ __forceinline__ int split_bucket(unsigned kl) {
    const unsigned u = kl - static_cast<unsigned>(kSplitHeads);
    return kl < static_cast<unsigned>(kSplitHeads) ? static_cast<int>(kl)
                                                   : kSplitClassBase + static_cast<int>(u - 15u * hot_class_index(kl));
}

// Where hawk_split_hot's split puts the tile's tail entries: straight from
// registers into the tile's slot of the chunk's bin, in bucket order, with
// the offset of each tail range in the tile's row of bin_off.
template <class T>
struct TailSink {
    unsigned short* key = nullptr;
    T* val = nullptr;
    unsigned* off = nullptr;
    int ranges = 0;
};

// Stable split of the tile held in registers (thread slot j of wave w is tile
// position w*256 + j*64 + lane) into nb buckets: sh.key/sh.val in bucket order,
// lane order within a bucket; bucket bounds in sh.bstart.  Each wave matches
// its four windows one after another in one table, so a lane's rank is the
// count of its bucket in the wave's earlier windows plus the lanes below it
// in its own.  Every wave then forms its own positions from all waves'
// counts.  With Sink, entries of a tail bucket go to the sink instead of LDS.
// Starts and ends with every thread of the workgroup.
template <class T, class Sh, bool Sink>
__device__ void split_tile(Sh& sh, const unsigned (&kl)[kWalkItems], const int (&d)[kWalkItems],
                           const T (&vv)[kWalkItems], int nb, const TailSink<T>& sink) {
    const int t = threadIdx.x;
    const int wave = t >> 6;
    const int lane = t & 63;
    const unsigned long long me = 1ull << lane;
    unsigned long long own[kWalkItems], mine[kWalkItems];
    // Window j: clear the table, OR every lane's bit into its bucket's slot,
    // read the lane's own slot and (lane b) slot b.  The four windows' LDS
    // operations run back to back: a wave's LDS operations complete in issue
    // order, so each window's reads see its own ORs and precede the next
    // window's clear.
    unsigned long long* tab = sh.win[wave];
    const int b = lane < Sh::kStride ? lane : 0;
#pragma unroll
    for (int j = 0; j < kWalkItems; ++j) {
        if (lane < Sh::kStride) tab[lane] = 0ull;
        __builtin_amdgcn_wave_barrier();
        if (d[j] != kSplitNone) atomicOr(&tab[d[j]], me);
        __builtin_amdgcn_wave_barrier();
        own[j] = tab[d[j] != kSplitNone ? d[j] : 0];
        mine[j] = tab[b];
        __builtin_amdgcn_wave_barrier();
    }
    // lane b: bucket b's count in each window and the running count before
    // each; each item later takes its bucket's position from lane d (a
    // permute) and adds the lanes below it in its window
    unsigned run[kWalkItems], below[kWalkItems];
    unsigned total = 0u;
#pragma unroll
    for (int j = 0; j < kWalkItems; ++j) {
        run[j] = total;
        total += static_cast<unsigned>(__popcll(mine[j]));
        below[j] = __builtin_amdgcn_mbcnt_hi(static_cast<unsigned>(own[j] >> 32),
                                             __builtin_amdgcn_mbcnt_lo(static_cast<unsigned>(own[j]), 0u));
    }
    if (lane < Sh::kStride) sh.cnt[wave][lane] = total;
    __syncthreads();
    // lane b: bucket b's total over the waves, the earlier waves' share of it,
    // and (a scan over the lanes) where bucket b starts
    unsigned before = 0u, sum = 0u;
    if (lane < nb) {
        // word b of every wave's row: consecutive lanes, consecutive banks
#pragma unroll
        for (int w = 0; w < Sh::kWaves; ++w) {
            const unsigned c = sh.cnt[w][lane];
            before += w < wave ? c : 0u;
            sum += c;
        }
    }
    const unsigned start = wave_inclusive_scan(sum) - sum;
    if (wave == 0 && lane <= nb) sh.bstart[lane] = start;
    const unsigned base = start + before;
    unsigned ts = 0u;
    if constexpr (Sink) {
        ts = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(start), kSplitTailBase));
        if (sink.ranges > 0 && wave == 0 && lane >= kSplitTailBase && lane <= kSplitTailBase + sink.ranges)
            sink.off[lane - kSplitTailBase] = start - ts;
    }
#pragma unroll
    for (int j = 0; j < kWalkItems; ++j) {
        const int dj = d[j] != kSplitNone ? d[j] : 0;
        const unsigned p =
                static_cast<unsigned>(__builtin_amdgcn_ds_bpermute(dj << 2, static_cast<int>(base + run[j]))) + below[j];
        if (d[j] != kSplitNone) {
            if (Sink && d[j] >= kSplitTailBase) {
                sink.key[p - ts] = static_cast<unsigned short>(kl[j]);
                sink.val[p - ts] = vv[j];
            } else {
                sh.key[p] = static_cast<unsigned short>(kl[j]);
                sh.val[p] = vv[j];
            }
        }
    }
    __syncthreads();
}

// Lane `lane`'s T, to every lane (two readlanes: the lane select is uniform).
__device__ __forceinline__ double lane_value(double x, int lane) {
    const long long bits = __double_as_longlong(x);
    const int lo = __builtin_amdgcn_readlane(static_cast<int>(bits), lane);
    const int hi = __builtin_amdgcn_readlane(static_cast<int>(bits >> 32), lane);
    return __longlong_as_double((static_cast<long long>(hi) << 32) | static_cast<unsigned>(lo));
}
__device__ __forceinline__ float lane_value(float x, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

// The head keys' chains, by one wave: lane c (c < kSplitHeads) adds bucket c
// (window key c: one contiguous run, lane order) onto acc[c], one addition at
// a time from its own registers.  Its reads run 32 values ahead of its adds
// in four rotating blocks of 8, so the chain waits on the adds' latency, not
// on the LDS.  A lane's loop ends with its run; the wave runs as long as the
// longest run.  Reads go at most 63 entries past a run's end (the padding).
template <class T>
__device__ __forceinline__ void head_block(T (&r)[kHeadBlock], T& a, const T* src) {
#pragma unroll
    for (int q = 0; q < kHeadBlock; ++q) a = a + r[q];
    // the block's next reads go into the registers its adds just used: no
    // copies, so the other blocks' reads stay in flight
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < kHeadBlock; ++q) r[q] = src[q];
    __builtin_amdgcn_sched_barrier(0);
}

template <class T, class Sh>
__device__ void fold_heads(Sh& sh) {
    const int lane = threadIdx.x & 63;
    if (lane >= kSplitHeads) return;
    const int s = static_cast<int>(sh.bstart[lane]);
    const int e = static_cast<int>(sh.bstart[lane + 1]);
    if (s >= e) return;
    T a = sh.acc[lane];
    T r0[kHeadBlock], r1[kHeadBlock], r2[kHeadBlock], r3[kHeadBlock];
    const T* x = sh.val + s;
    // the first reads in block order, as the loop issues them: the loop's
    // waits count LDS operations, and on its entry they follow this order
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < kHeadBlock; ++q) r0[q] = x[q];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < kHeadBlock; ++q) r1[q] = x[kHeadBlock + q];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < kHeadBlock; ++q) r2[q] = x[2 * kHeadBlock + q];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < kHeadBlock; ++q) r3[q] = x[3 * kHeadBlock + q];
    __builtin_amdgcn_sched_barrier(0);
    constexpr int kAhead = 4 * kHeadBlock;
    int left = e - s;
    for (; left >= kAhead; left -= kAhead, x += kAhead) {
        head_block(r0, a, x + kAhead);
        head_block(r1, a, x + kAhead + kHeadBlock);
        head_block(r2, a, x + kAhead + 2 * kHeadBlock);
        head_block(r3, a, x + kAhead + 3 * kHeadBlock);
    }
    // fewer than kAhead left, held in r0..r3 in order
#pragma unroll
    for (int q = 0; q < kHeadBlock; ++q)
        if (q < left) a = a + r0[q];
#pragma unroll
    for (int q = 0; q < kHeadBlock; ++q)
        if (kHeadBlock + q < left) a = a + r1[q];
#pragma unroll
    for (int q = 0; q < kHeadBlock; ++q)
        if (2 * kHeadBlock + q < left) a = a + r2[q];
#pragma unroll
    for (int q = 0; q < kHeadBlock; ++q)
        if (3 * kHeadBlock + q < left) a = a + r3[q];
    sh.acc[lane] = a;
}

// The caller's wave folds class c of the split tile, 64 entries a window in
// lane order.  Within a class a key is named by its index m (hot: (kl - 32)
// / 15; tail: kl >> 3), below 1024.  Equal keys of a window find each other
// through the wave's match table: bits 0..6 of m pick one of kPeerSlots
// slots, every lane ORs its bit into its slot, and three ballots over bits
// 7..9 keep the lanes whose whole key is equal.  The lowest lane of each key
// adds its own value and then its peers' (read back from the class's run, in
// lane order) onto the accumulator it read with the match.  A wave's LDS
// operations complete in issue order, so a key's windows meet its
// accumulator one after another.
template <class T, class Sh, bool Hot>
__device__ void fold_class(Sh& sh, int c) {
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const unsigned long long me = 1ull << lane;
    const int s = static_cast<int>(sh.bstart[kSplitClassBase + c]);
    const int e = static_cast<int>(sh.bstart[kSplitClassBase + c + 1]);
    if (s >= e) return;
    unsigned long long* peer = sh.f.peer[wave];
    unsigned k = sh.key[s + lane];
    T x = sh.val[s + lane];
    for (int base = s; base < e; base += 64) {
        const bool valid = base + lane < e;
        unsigned nk = 0u;
        T nx = T(0);
        if (base + 64 < e) {
            nk = sh.key[base + 64 + lane];
            nx = sh.val[base + 64 + lane];
        }
        const unsigned kv = valid ? k : 0u;
        const unsigned m = Hot ? hot_class_index(kv) : (kv >> kTailClassBits);
        const unsigned h = m & (kPeerSlots - 1u);
        if (valid) atomicOr(&peer[h], me);
        __builtin_amdgcn_wave_barrier();
        unsigned long long pm = valid ? peer[h] : 0ull;
        const unsigned ai = Hot ? kv : tail_slot(kv);
        const T a0 = valid ? sh.acc[ai] : T(0);
        __builtin_amdgcn_wave_barrier();
        if (valid) peer[h] = 0ull;
#pragma unroll
        for (int bit = 7; bit < 10; ++bit) {
            const bool one = (m >> bit) & 1u;
            const unsigned long long ones = __ballot(valid && one);
            pm &= one ? ones : ~ones;
        }
        if (valid && (pm & (me - 1ull)) == 0ull) {
            // the key's lowest lane: its value, then its peers' in lane order
            T a = a0 + x;
            unsigned long long rest = pm & ~me;
            while (rest != 0ull) {
                T y[8];
                int got = 0;
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    if (rest != 0ull) {
                        y[q] = sh.val[base + static_cast<int>(__builtin_ctzll(rest))];
                        rest &= rest - 1ull;
                        got = q + 1;
                    }
                }
#pragma unroll
                for (int q = 0; q < 8; ++q)
                    if (q < got) a = a + y[q];
            }
            sh.acc[ai] = a;
        }
        __builtin_amdgcn_wave_barrier();
        k = nk;
        x = nx;
    }
}

// The split tile's folds in hawk_split_hot: wave 0 the head keys' chains,
// wave w (1..15) class w - 1.  A class wave first clears its match table (it
// shares LDS with the split's tables); each window leaves it clear.
template <class T>
__device__ void split_fold(HotShared<T>& sh) {
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    if (wave == 0) {
        fold_heads<T>(sh);
        return;
    }
#pragma unroll
    for (unsigned i = 0; i < kPeerSlots; i += 64) sh.f.peer[wave][i + lane] = 0ull;
    __builtin_amdgcn_wave_barrier();
    fold_class<T, HotShared<T>, true>(sh, wave - 1);
}

// hawk_split_tail's folds: wave w folds class w (keys with kl & 7 == w).
template <class T>
__device__ void split_fold_tail(TailShared<T>& sh) {
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (unsigned i = 0; i < kPeerSlots; i += 64) sh.f.peer[wave][i + lane] = 0ull;
    __builtin_amdgcn_wave_barrier();
    fold_class<T, TailShared<T>, false>(sh, wave);
}

// The window's partials of chunk b, every key [klo, klo+window): a key no
// lane named holds +0.0, the walk's starting value.
template <class T, class Sh>
__device__ void split_store(Sh& sh, long long b, long long cells, long long klo, int window,
                            T* __restrict__ parts) {
    __syncthreads();
    T* row = parts + b * cells + klo;
    for (int k = threadIdx.x; k < window; k += Sh::kWaves * 64) row[k] = sh.acc[k];
}

template <class T, class Sh>
__device__ void split_clear(Sh& sh, int window) {
    for (int k = threadIdx.x; k < window; k += Sh::kWaves * 64) sh.acc[k] = T(0);
    __syncthreads();
}

// Chunk b = blockIdx.x: lanes [b*span, min((b+1)*span, n)), keys below
// kSplitHot folded here, the others written to the chunk's bin (slot = tile,
// offsets of the `ranges` tail ranges in bin_off[b][tile][0..ranges]).
template <class T>
__global__ __launch_bounds__(kWalkThreads) void hawk_split_hot(
        const int* __restrict__ key, const T* __restrict__ v, long long n, long long cells, long long span,
        int tiles, int ranges, unsigned short* __restrict__ bin_key, T* __restrict__ bin_val,
        unsigned* __restrict__ bin_off, T* __restrict__ parts, int* __restrict__ status) {
    __shared__ HotShared<T> sh;
    const int t = threadIdx.x;
    const long long b = blockIdx.x;
    const long long lo = b * span;
    const long long hi = lo + span < n ? lo + span : n;
    const int window = cells < kSplitHot ? static_cast<int>(cells) : kSplitHot;
    const int nb = kSplitTailBase + ranges;
    split_clear<T>(sh, window);
    bool bad = false;
    int nk[kWalkItems];
    T nv[kWalkItems];
    if (lo < hi) walk_load(key, v, lo, hi, nk, nv);
    int tile = 0;
    for (long long base = lo; base < hi; base += kTile, ++tile) {
        unsigned kl[kWalkItems];
        int d[kWalkItems];
        T vv[kWalkItems];
        // each lane's bucket, without branches: a skip or bad key none, a
        // window key its head bucket or class, a tail key its range
#pragma unroll
        for (int j = 0; j < kWalkItems; ++j) {
            const unsigned u = static_cast<unsigned>(nk[j]);
            vv[j] = nv[j];
            const bool valid = u < static_cast<unsigned>(cells);
            bad = bad | ((nk[j] != -1) & !valid);
            const unsigned tl = u - static_cast<unsigned>(kSplitHot);
            const unsigned r = tl / static_cast<unsigned>(kTailRange);
            const bool in_win = u < static_cast<unsigned>(window);
            const int dw = split_bucket(u);
            d[j] = !valid ? kSplitNone : in_win ? dw : kSplitTailBase + static_cast<int>(r);
            kl[j] = in_win ? u : tl - r * static_cast<unsigned>(kTailRange);
        }
        if (base + kTile < hi) walk_load(key, v, base + kTile, hi, nk, nv);
        {
            TailSink<T> sink;
            if (ranges > 0) {
                const long long slot = (b * tiles + tile) * kTile;
                sink.key = bin_key + slot;
                sink.val = bin_val + slot;
                sink.off = bin_off + (b * tiles + tile) * (ranges + 1);
                sink.ranges = ranges;
            }
            split_tile<T, HotShared<T>, true>(sh, kl, d, vv, nb, sink);
        }
        split_fold(sh);
        __syncthreads();
    }
    // a chunk with fewer tiles than `tiles` (the last, short one) leaves its
    // later slots empty
    if (ranges > 0)
        for (int i = t; i < (tiles - tile) * (ranges + 1); i += kWalkThreads)
            bin_off[(b * tiles + tile) * (ranges + 1) + i] = 0u;
    split_store<T>(sh, b, cells, 0, window, parts);
    // the status plane (hawk_scatter_status's values, written here in the
    // split walk): chunk b's flag, and from chunk 0 the cell count and the
    // flags of the chunks past the last
    const int any = __syncthreads_or(bad ? 1 : 0);
    if (t == 0) status[1 + b] = any ? 1 : 0;
    if (b == 0) {
        if (t == 0) status[0] = static_cast<int>(cells);
        for (int i = static_cast<int>(gridDim.x) + t; i < kScatterChunks; i += kWalkThreads) status[1 + i] = 0;
    }
}

// The tail ranges' stream: for workgroup (chunk b, range r), the range's
// segment of each tile slot of the chunk, slot after slot (lane order).  Each
// wave holds a group of up to kTailGroup segments in registers: lane l,
// register k describes segment g = 64k + l by its first stream position
// P[k] and the offset that turns a stream position q of it into its bin
// entry, base + A[k] + q (base: the group's first slot).  Segments past the group's end start at the group's
// length, so no position of the group falls in them.
constexpr int kTailGroup = 128;

struct TailSegs {
    unsigned P[kTailGroup / 64];
    int A[kTailGroup / 64];
    long long base;        // the group's first slot
    unsigned count;        // entries in the group
    int n;                 // segments in the group
};

__device__ __forceinline__ unsigned tail_reg(const unsigned (&x)[kTailGroup / 64], int m) {
    static_assert(kTailGroup == 128, "two registers a lane");
    const unsigned v = m < 64 ? x[0] : x[1];
    return static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(v), m & 63));
}
__device__ __forceinline__ int tail_reg(const int (&x)[kTailGroup / 64], int m) {
    const int v = m < 64 ? x[0] : x[1];
    return __builtin_amdgcn_readlane(v, m & 63);
}

// Group [g0, g0 + gn) of chunk b's slots, range r: every wave reads the
// group's bounds (hawk_split_hot wrote 0 <= o[r] <= o[r+1] <= 4096; the
// clamps keep every read inside its slot whatever the plane holds).
__device__ __forceinline__ TailSegs tail_segs(const unsigned* __restrict__ bin_off, long long b, int tiles, int ranges,
                                              int r, int g0, int gn) {
    const int lane = threadIdx.x & 63;
    TailSegs S;
    unsigned carry = 0u;
#pragma unroll
    for (int k = 0; k < kTailGroup / 64; ++k) {
        const int g = k * 64 + lane;
        unsigned lo = 0u, hi = 0u;
        if (g < gn) {
            const unsigned* o = bin_off + (b * tiles + g0 + g) * (ranges + 1);
            const unsigned a = o[r], z = o[r + 1];
            lo = a < static_cast<unsigned>(kTile) ? a : static_cast<unsigned>(kTile);
            hi = z < lo ? lo : (z < static_cast<unsigned>(kTile) ? z : static_cast<unsigned>(kTile));
        }
        const unsigned c = hi - lo;
        const unsigned incl = wave_inclusive_scan(c) + carry;
        S.P[k] = incl - c;
        S.A[k] = g * kTile + static_cast<int>(lo) - static_cast<int>(S.P[k]);
        carry = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(incl), 63));
    }
    S.count = carry;
    S.n = gn;
    S.base = (b * tiles + g0) * kTile;
#pragma unroll
    for (int k = 0; k < kTailGroup / 64; ++k)
        if (k * 64 + lane >= gn) S.P[k] = carry;
    return S;
}

// The batch at stream position qb: thread slot j of wave w takes position
// qb + w*256 + j*64 + lane (positions past the group's end read as nothing).
// Each window of 64 positions finds the segment of its first position with
// two ballots, then steps over the segments that start inside it.
template <class T>
__device__ __forceinline__ void tail_load(const TailSegs& S, const unsigned short* __restrict__ bin_key,
                                          const T* __restrict__ bin_val, unsigned qb, unsigned (&kk)[kWalkItems],
                                          T (&vv)[kWalkItems]) {
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < kWalkItems; ++j) {
        const unsigned qw = qb + static_cast<unsigned>(wave * (kWalkItems * 64) + j * 64);
        const unsigned q = qw + static_cast<unsigned>(lane);
        kk[j] = 0u;
        vv[j] = T(0);
        if (qw >= S.count) continue;
        int g = -1;
#pragma unroll
        for (int k = 0; k < kTailGroup / 64; ++k) g += __popcll(__ballot(S.P[k] <= qw));
        int a = tail_reg(S.A, g);
        for (int m = g + 1; m < S.n; ++m) {
            // both reads with every lane active: the lane read from must
            // have computed its register select
            const unsigned pm = tail_reg(S.P, m);
            if (pm > qw + 63u) break;
            const int am = tail_reg(S.A, m);
            a = q >= pm ? am : a;
        }
        if (q < S.count) {
            const long long at = S.base + a + static_cast<long long>(q);
            kk[j] = bin_key[at];
            vv[j] = bin_val[at];
        }
    }
}

// (chunk b, tail range r) = (blockIdx.x / ranges, blockIdx.x % ranges): keys
// [kSplitHot + kTailRange*r, +kTailRange) of chunk b, read as a stream from the
// bin's slots in tile order, kTailBatch entries a batch, the next batch's reads
// in flight while a batch is split and folded.
template <class T>
__global__ __launch_bounds__(kTailThreads, 2) void hawk_split_tail(
        long long cells, int tiles, int ranges, const unsigned short* __restrict__ bin_key,
        const T* __restrict__ bin_val, const unsigned* __restrict__ bin_off, T* __restrict__ parts) {
    __shared__ TailShared<T> sh;
    const long long b = blockIdx.x / ranges;
    const int r = static_cast<int>(blockIdx.x % ranges);
    const long long klo = kSplitHot + static_cast<long long>(kTailRange) * r;
    const int window = cells - klo < kTailRange ? static_cast<int>(cells - klo) : kTailRange;
    split_clear<T>(sh, kTailRange);
    for (int g0 = 0; g0 < tiles; g0 += kTailGroup) {
        const int gn = tiles - g0 < kTailGroup ? tiles - g0 : kTailGroup;
        const TailSegs S = tail_segs(bin_off, b, tiles, ranges, r, g0, gn);
        unsigned nk[kWalkItems];
        T nv[kWalkItems];
        if (S.count > 0u) tail_load(S, bin_key, bin_val, 0u, nk, nv);
        for (unsigned qb = 0; qb < S.count; qb += kTailBatch) {
            unsigned kl[kWalkItems];
            int d[kWalkItems];
            T vv[kWalkItems];
#pragma unroll
            for (int j = 0; j < kWalkItems; ++j) {
                const unsigned q = qb + static_cast<unsigned>((threadIdx.x >> 6) * (kWalkItems * 64) + j * 64 +
                                                              (threadIdx.x & 63));
                kl[j] = nk[j];
                vv[j] = nv[j];
                d[j] = q < S.count ? kSplitClassBase + static_cast<int>(kl[j] & (kTailClasses - 1u)) : kSplitNone;
            }
            if (qb + kTailBatch < S.count) tail_load(S, bin_key, bin_val, qb + kTailBatch, nk, nv);
            split_tile<T, TailShared<T>, false>(sh, kl, d, vv, kSplitClassBase + kTailClasses, TailSink<T>());
            split_fold_tail(sh);
            __syncthreads();
        }
    }
    __syncthreads();
    T* row = parts + b * cells + klo;
    for (int k = threadIdx.x; k < window; k += kTailThreads) row[k] = sh.acc[tail_slot(static_cast<unsigned>(k))];
}

// The ordered scatter's scratch, in this order (each part 256-byte aligned):
// parts[chunks][cells] f64; and for the split walk with tail ranges, the bin
// offsets [chunks][tiles][ranges+1] u32, the bin keys [chunks][tiles][4096]
// u16 and the bin values [chunks][tiles][4096] f64.
struct ScatterLayout {
    int chunks = 1;
    long long span = 0;
    bool split = false;
    int tiles = 0;
    int ranges = 0;
    size_t parts = 0, bin_off = 0, bin_key = 0, bin_val = 0, bytes = 0;
};

size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

ScatterLayout scatter_layout(int64_t n, int64_t cells, int chunks) {
    ScatterLayout L;
    L.chunks = chunks;
    L.span = (n + chunks - 1) / chunks;
    L.split = cells <= kSplitCells;
    const size_t c = static_cast<size_t>(chunks);
    size_t at = 0;
    L.parts = at;
    at += align256(sizeof(double) * c * static_cast<size_t>(cells));
    if (L.split) {
        const long long tiles = (L.span + kTile - 1) / kTile;
        L.tiles = static_cast<int>(tiles < 1 ? 1 : tiles);
        L.ranges = cells > kSplitHot ? static_cast<int>((cells - kSplitHot + kTailRange - 1) / kTailRange) : 0;
        if (L.ranges > 0) {
            const size_t slots = c * static_cast<size_t>(L.tiles);
            L.bin_off = at;
            at += align256(sizeof(unsigned) * slots * static_cast<size_t>(L.ranges + 1));
            L.bin_key = at;
            at += align256(sizeof(unsigned short) * slots * kTile);
            L.bin_val = at;
            at += align256(sizeof(double) * slots * kTile);
        }
    }
    L.bytes = at;
    return L;
}

// ---- the ordered gradient's log fold ----------------------------------------
// reference hawk/emit/team.py:281-312 (`_fold`) and hawk/ir/team.py:684-693
// (`fold_spec`): pair (key k, slot e) adds the key's `rows` contributions
// v[e * stride + k * rows + r], r = 0, 1, ..., in lane order from +0.0, and
// STORES the sum into out[cell_of[e * keys + k]].  Pairs run slot-major
// (pair = e * keys + k), so neighbouring pairs read neighbouring runs of one
// component plane.  A cell outside [0, cells) is not stored and sets status
// bit 0; a cell that a second pair names sets bit 1 and lowers status[1] to
// it (claims counts the pairs naming each cell): such stores race, as they do
// in the reference, and the caller is told.

template <class T>
__device__ __forceinline__ void log_fold_store(T s, int c, long long cells, T* __restrict__ out,
                                               int* __restrict__ claims, int* __restrict__ status) {
    if (c < 0 || c >= cells) {
        atomicOr(status, 1);
        return;
    }
    if (atomicAdd(claims + c, 1) != 0) {
        atomicOr(status, 2);
        atomicMin(status + 1, c);
    }
    out[c] = s;
}

// One thread per pair: the thread reads its run 16 rows at a time (then 8,
// then one), each batch's loads in flight before its adds.  Measured on
// MI355X over 805 MB of log: 4.6 TB/s at 64 rows a run, against 4.0 with
// batches of 8; staging the runs through LDS, or a wave reading whole lines,
// did no better.
template <class T>
__global__ __launch_bounds__(256) void hawk_log_fold_lanes(const T* __restrict__ v, long long stride,
                                                           const int* __restrict__ cell_of, long long keys,
                                                           long long rows, long long pairs,
                                                           T* __restrict__ out, long long cells,
                                                           int* __restrict__ claims, int* __restrict__ status) {
    const long long t = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    if (t >= pairs) return;
    const long long e = t / keys, k = t - e * keys;
    const T* __restrict__ p = v + e * stride + k * rows;
    T s = T(0);
    long long r = 0;
    for (; r + 16 <= rows; r += 16) {
        T x[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) x[q] = p[r + q];
#pragma unroll
        for (int q = 0; q < 16; ++q) s = s + x[q];
    }
    if (r + 8 <= rows) {
        T x[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) x[q] = p[r + q];
#pragma unroll
        for (int q = 0; q < 8; ++q) s = s + x[q];
        r += 8;
    }
    for (; r < rows; ++r) s = s + p[r];
    log_fold_store(s, cell_of[t], cells, out, claims, status);
}

// One wave per pair, for long runs of few pairs: the wave loads 64 consecutive rows (one
// 512-byte read) while it adds the previous 64 in lane order, every lane
// holding the same running sum; lane 0 stores it.
template <class T>
__global__ __launch_bounds__(256) void hawk_log_fold_waves(const T* __restrict__ v, long long stride,
                                                           const int* __restrict__ cell_of, long long keys,
                                                           long long rows, long long pairs,
                                                           T* __restrict__ out, long long cells,
                                                           int* __restrict__ claims, int* __restrict__ status) {
    const long long pair = static_cast<long long>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (pair >= pairs) return;                 // the whole wave
    const int lane = threadIdx.x & 63;
    const long long e = pair / keys, k = pair - e * keys;
    const T* __restrict__ p = v + e * stride + k * rows;
    T s = T(0);
    T x = lane < rows ? p[lane] : T(0);
    long long r0 = 0;
    for (; r0 + 64 <= rows; r0 += 64) {
        const T cur = x;
        x = r0 + 64 + lane < rows ? p[r0 + 64 + lane] : T(0);
#pragma unroll
        for (int j = 0; j < 64; ++j) s = s + lane_value(cur, j);
    }
    const int tail = static_cast<int>(rows - r0);
    for (int j = 0; j < tail; ++j) s = s + lane_value(x, j);
    if (lane == 0) log_fold_store(s, cell_of[pair], cells, out, claims, status);
}

__global__ __launch_bounds__(256) void hawk_log_fold_clear(int* __restrict__ claims, long long cells,
                                                           int* __restrict__ status) {
    const long long i0 = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    if (i0 == 0) {
        status[0] = 0;
        status[1] = 0x7fffffff;
    }
    for (long long i = i0; i < cells; i += static_cast<long long>(gridDim.x) * 256) claims[i] = 0;
}

int launch_error(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hawk_internal::set_hip_error(what, e);
    return HK_OK;
}

int bits_for(long long max_value) {
    int b = 1;
    while ((1LL << b) <= max_value) ++b;
    return b;
}

}  // namespace

// The scratch of hk_ordered_sum_f64_noalloc: the ordered sum's 65536 lane
// partials, 64 group values and ticket, kSumScratch bytes (512 KiB + 768 B)
// whatever the number of samples.  Each GPU the library runs on holds its own
// copy until the process ends.  In host code `scratch` names a host-side
// stand-in, never the device memory: launches take the per-device address
// that scratch_of() obtains with hipGetSymbolAddress.
static __device__ __align__(256) unsigned char scratch[kSumScratch];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the GPU that runs `stream` (the current
// device for the null stream), looked up once per device with that device
// current.
int scratch_of(hipStream_t stream, void** out) {
    int dev = 0;
    hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
    if (e != hipSuccess) return hawk_internal::set_hip_error("hk_ordered_sum_f64_noalloc: the stream's device", e);
    if (dev < 0 || dev >= kMaxDevices)
        return hawk_internal::set_error(HK_EVALUE, "hk_ordered_sum_f64_noalloc: device " + std::to_string(dev) +
                                                       " is past the " + std::to_string(kMaxDevices) +
                                                       " devices it keeps a scratch address for");
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        int current = 0;
        e = hipGetDevice(&current);
        if (e != hipSuccess) return hawk_internal::set_hip_error("hk_ordered_sum_f64_noalloc: hipGetDevice", e);
        if (current != dev && (e = hipSetDevice(dev)) != hipSuccess)
            return hawk_internal::set_hip_error("hk_ordered_sum_f64_noalloc: hipSetDevice", e);
        void* ptr = nullptr;
        const hipError_t got = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (current != dev && (e = hipSetDevice(current)) != hipSuccess)
            return hawk_internal::set_hip_error("hk_ordered_sum_f64_noalloc: hipSetDevice", e);
        if (got != hipSuccess)
            return hawk_internal::set_hip_error("hk_ordered_sum_f64_noalloc: hipGetSymbolAddress(scratch)", got);
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return HK_OK;
}

// The ordered sum in T (hk_ordered_sum_f64 / _f32): the lanes, then the fold.
// A float sum keeps the double layout's offsets, its data in the front of
// each region.
template <class T>
int ordered_sum(const T* u, int64_t n, T* out, void* scratch, void* stream, const char* name) {
    if (n < 0) return hawk_internal::set_error(HK_EVALUE, std::string(name) + ": n must be >= 0");
    if ((n > 0 && !u) || !out || !scratch)
        return hawk_internal::set_error(HK_EVALUE, std::string(name) + ": u, out and scratch are required");
    auto* base = static_cast<unsigned char*>(scratch);
    auto* lanes = reinterpret_cast<T*>(base);
    auto* gp = reinterpret_cast<T*>(base + kLanesBytes);
    auto* ticket = reinterpret_cast<unsigned*>(base + kLanesBytes + kGpBytes);
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(hawk_sum_lanes<T>, dim3(kVirtualLanes / kLaneBlock), dim3(kLaneBlock), 0, s, u,
                       static_cast<long long>(n), lanes, ticket);
    int rc = launch_error("hawk_sum_lanes launch");
    if (rc != HK_OK) return rc;
    hipLaunchKernelGGL(hawk_sum_fold<T>, dim3(kGroups), dim3(256), 0, s, lanes, gp, ticket, out);
    return launch_error("hawk_sum_fold launch");
}

// The keyed ordered sum in T (hk_keyed_ordered_sum_f64 / _f32).
template <class T>
int keyed_ordered_sum(const T* u, int64_t n, int64_t group, T* out, void* scratch, void* stream, const char* name) {
    const std::string who(name);
    if (n < 0 || group <= 0) return hawk_internal::set_error(HK_EVALUE, who + ": n must be >= 0 and group >= 1");
    if (n % group != 0)
        return hawk_internal::set_error(HK_EVALUE, who + ": n (" + std::to_string(n) +
                                                       ") is not a whole number of groups of " + std::to_string(group));
    if (n == 0) return HK_OK;
    if (!u || !out || !scratch) return hawk_internal::set_error(HK_EVALUE, who + ": u, out and scratch are required");
    if (n == group) return ordered_sum<T>(u, n, out, scratch, stream, name);    // one key: the ordered sum
    const long long keys = n / group;
    if (keys > 0x7fffffffLL) return hawk_internal::set_error(HK_EVALUE, who + ": too many keys");
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (group <= 64) {
        const int P = pow2_at_least(group);
        const long long waves = (keys + 64 / P - 1) / (64 / P);
        hipLaunchKernelGGL(hawk_keyed_small<T>, dim3(static_cast<unsigned>((waves + 3) / 4)), dim3(256), 0, s, u,
                           static_cast<long long>(group), P, keys, out);
        return launch_error("hawk_keyed_small launch");
    }
    if (group <= kVirtualLanes) {
        hipLaunchKernelGGL(hawk_keyed_rows<T>, dim3(static_cast<unsigned>(keys)), dim3(256), 0, s, u,
                           static_cast<long long>(group), out);
        return launch_error("hawk_keyed_rows launch");
    }
    const long long lv = group < kVirtualLanes ? group : kVirtualLanes;
    const long long total = keys * lv;
    auto* lanes = static_cast<T*>(scratch);
    long long blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(hawk_keyed_lanes<T>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, u,
                       static_cast<long long>(group), lv, total, lanes);
    int rc = launch_error("hawk_keyed_lanes launch");
    if (rc != HK_OK) return rc;
    hipLaunchKernelGGL(hawk_keyed_fold<T>, dim3(static_cast<unsigned>(keys)), dim3(256), 0, s, lanes, lv, out);
    return launch_error("hawk_keyed_fold launch");
}

// The rows' finish in T: the leaves, then the levels into *out.
template <class T>
int rows_finish(const T* hi, const T* comp, int64_t rows, T* out, void* scratch, void* stream, const char* name) {
    if (rows < 1) return hawk_internal::set_error(HK_EVALUE, std::string(name) + ": rows must be >= 1");
    if (!hi || !comp || !out || !scratch)
        return hawk_internal::set_error(HK_EVALUE, std::string(name) + ": hi, comp, out and scratch are required");
    const long long leaves = (rows + kRowLeaf - 1) / kRowLeaf;
    if (leaves > 0x7fffffffLL) return hawk_internal::set_error(HK_EVALUE, std::string(name) + ": too many rows");
    auto* buf = static_cast<T*>(scratch);
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(hawk_rows_leaves<T>, dim3(static_cast<unsigned>(leaves)), dim3(kRowSlots), 0, s, hi, comp,
                       static_cast<long long>(rows), buf, buf + leaves);
    int rc = launch_error("hawk_rows_leaves launch");
    if (rc != HK_OK) return rc;
    hipLaunchKernelGGL(hawk_rows_levels<T>, dim3(1), dim3(256), 0, s, buf, leaves, out);
    return launch_error("hawk_rows_levels launch");
}

// The rows' extreme in T (op 1 max, 2 min): the leaves, then the levels.
template <class T>
int rows_extreme(const T* hi, int64_t rows, int32_t op, T* out, void* scratch, void* stream, const char* name) {
    const std::string who(name);
    if (rows < 1) return hawk_internal::set_error(HK_EVALUE, who + ": rows must be >= 1");
    if (op != 1 && op != 2) return hawk_internal::set_error(HK_EVALUE, who + ": op must be 1 (max) or 2 (min)");
    if (!hi || !out || !scratch) return hawk_internal::set_error(HK_EVALUE, who + ": hi, out and scratch are required");
    const long long leaves = (rows + kRowLeaf - 1) / kRowLeaf;
    if (leaves > 0x7fffffffLL) return hawk_internal::set_error(HK_EVALUE, who + ": too many rows");
    auto* buf = static_cast<T*>(scratch);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (op == 1)
        hipLaunchKernelGGL((hawk_rows_ext_leaves<T, 1>), dim3(static_cast<unsigned>(leaves)), dim3(kRowSlots), 0, s,
                           hi, static_cast<long long>(rows), buf);
    else
        hipLaunchKernelGGL((hawk_rows_ext_leaves<T, 2>), dim3(static_cast<unsigned>(leaves)), dim3(kRowSlots), 0, s,
                           hi, static_cast<long long>(rows), buf);
    int rc = launch_error("hawk_rows_ext_leaves launch");
    if (rc != HK_OK) return rc;
    if (op == 1)
        hipLaunchKernelGGL((hawk_rows_ext_levels<T, 1>), dim3(1), dim3(256), 0, s, buf, leaves, out);
    else
        hipLaunchKernelGGL((hawk_rows_ext_levels<T, 2>), dim3(1), dim3(256), 0, s, buf, leaves, out);
    return launch_error("hawk_rows_ext_levels launch");
}

// The keyed default-policy sum in T (hk_keyed_sample_sum_f64 / _f32).
template <class T>
int keyed_sample_sum(const T* u, int64_t n, int64_t group, T* out, void* stream, const char* name) {
    const std::string who(name);
    if (n < 0 || group <= 0)
        return hawk_internal::set_error(HK_EVALUE, who + ": n must be >= 0 and group >= 1");
    if (n % group != 0)
        return hawk_internal::set_error(HK_EVALUE, who + ": n (" + std::to_string(n) +
                                                       ") is not a whole number of groups of " + std::to_string(group));
    if ((group + 31) / 32 > kRowLeaf * kKeyedCompLeaves)
        return hawk_internal::set_error(HK_EVALUE, who + ": a key of " + std::to_string(group) +
                                                       " samples spans more than 256 leaves of 4096 rows; sum it "
                                                       "with policy='ordered'");
    if (n == 0) return HK_OK;
    if (!u || !out) return hawk_internal::set_error(HK_EVALUE, who + ": u and out are required");
    const long long keys = n / group;
    if (keys > 0x7fffffffLL) return hawk_internal::set_error(HK_EVALUE, who + ": too many keys");
    if (group <= 64 * 32) {
        hipLaunchKernelGGL(hawk_keyed_comp_wave<T>, dim3(static_cast<unsigned>((keys + 3) / 4)), dim3(256), 0,
                           static_cast<hipStream_t>(stream), u, static_cast<long long>(group), keys, out);
        return launch_error("hawk_keyed_comp_wave launch");
    }
    hipLaunchKernelGGL(hawk_keyed_comp<T>, dim3(static_cast<unsigned>(keys)), dim3(kRowSlots), 0,
                       static_cast<hipStream_t>(stream), u, static_cast<long long>(group), out);
    return launch_error("hawk_keyed_comp launch");
}

// The ordered gradient's log fold in T (hk_keyed_log_fold_f64 / _f32).
template <class T>
int keyed_log_fold(const T* values, int64_t stride, const int32_t* cells_log, int64_t keys, int64_t rows,
                   int32_t width, T* out, int64_t cells, void* scratch, int32_t* status, void* stream,
                   const char* name) {
    const std::string who(name);
    if (keys < 0 || rows < 1 || width < 1 || cells < 0)
        return hawk_internal::set_error(HK_EVALUE, who + ": keys and cells must be >= 0, rows and width >= 1");
    if (stride < keys * rows)
        return hawk_internal::set_error(HK_EVALUE, who + ": stride (" + std::to_string(stride) +
                                                       ") is shorter than keys * rows (" +
                                                       std::to_string(keys * rows) + ")");
    if (!status) return hawk_internal::set_error(HK_EVALUE, who + ": status is required");
    const long long pairs = keys * static_cast<long long>(width);
    if (pairs > 0 && (!values || !cells_log || !out || (cells > 0 && !scratch)))
        return hawk_internal::set_error(HK_EVALUE,
                                        who + ": values, cells_log, out and scratch are required");
    if (cells > 0x7fffffffLL)
        return hawk_internal::set_error(HK_EVALUE, who + ": more than 2^31-1 cells");
    hipStream_t s = static_cast<hipStream_t>(stream);
    auto* claims = static_cast<int*>(scratch);
    const long long clear = (cells + 255) / 256 < 1 ? 1 : ((cells + 255) / 256 < 4096 ? (cells + 255) / 256 : 4096);
    hipLaunchKernelGGL(hawk_log_fold_clear, dim3(static_cast<unsigned>(clear)), dim3(256), 0, s, claims,
                       static_cast<long long>(cells), status);
    int rc = launch_error("hawk_log_fold_clear launch");
    if (rc != HK_OK || pairs == 0) return rc;
    if (rows <= 64 || pairs >= 65536) {          // enough pairs for a thread each to fill the chip
        const long long blocks = (pairs + 255) / 256;
        if (blocks > 0x7fffffffLL) return hawk_internal::set_error(HK_EVALUE, who + ": too many pairs");
        hipLaunchKernelGGL(hawk_log_fold_lanes<T>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, values,
                           static_cast<long long>(stride), cells_log, static_cast<long long>(keys),
                           static_cast<long long>(rows), pairs, out, static_cast<long long>(cells), claims, status);
        return launch_error("hawk_log_fold_lanes launch");
    }
    const long long blocks = (pairs + 3) / 4;
    if (blocks > 0x7fffffffLL) return hawk_internal::set_error(HK_EVALUE, who + ": too many pairs");
    hipLaunchKernelGGL(hawk_log_fold_waves<T>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, values,
                       static_cast<long long>(stride), cells_log, static_cast<long long>(keys),
                       static_cast<long long>(rows), pairs, out, static_cast<long long>(cells), claims, status);
    return launch_error("hawk_log_fold_waves launch");
}

// The ordered scatter in T (hk_ordered_scatter_f64 / _f32).
template <class T>
int ordered_scatter(const int32_t* key, const T* v, int64_t n, T* target, int64_t cells, void* scratch,
                    int32_t* status, void* stream, const char* name) {
    const std::string who(name);
    if (n < 0 || cells < 0)
        return hawk_internal::set_error(HK_EVALUE, who + ": n and cells must be >= 0");
    if (cells == 0) return HK_OK;   // a scatter into no cells adds nothing (reference hawk/runtime.py:727)
    if ((n > 0 && (!key || !v)) || !target || !scratch || !status)
        return hawk_internal::set_error(HK_EVALUE,
                                        who + ": key, v, target, scratch and status are required");
    if (cells > 0x7fffffffLL)
        return hawk_internal::set_error(HK_EVALUE, who + ": more than 2^31-1 cells");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int chunks = hk_scatter_chunks(n, cells);
    const ScatterLayout L = scatter_layout(n, cells, chunks);
    unsigned char* base = static_cast<unsigned char*>(scratch);
    auto* parts = reinterpret_cast<T*>(base + L.parts);     // a float scatter uses the front of each region
    int rc = HK_OK;
    if (!L.split) {
        hipLaunchKernelGGL(hawk_scatter_status, dim3(1), dim3(kScatterChunks + 64), 0, s, status,
                           static_cast<long long>(cells));
        rc = launch_error("hawk_scatter_status launch");
        if (rc != HK_OK) return rc;
    }
    if (L.split) {
        auto* bin_off = reinterpret_cast<unsigned*>(base + L.bin_off);
        auto* bin_key = reinterpret_cast<unsigned short*>(base + L.bin_key);
        auto* bin_val = reinterpret_cast<T*>(base + L.bin_val);
        hipLaunchKernelGGL(hawk_split_hot<T>, dim3(static_cast<unsigned>(chunks)), dim3(kWalkThreads), 0, s, key, v,
                           static_cast<long long>(n), static_cast<long long>(cells), L.span, L.tiles, L.ranges,
                           bin_key, bin_val, bin_off, parts, status);
        rc = launch_error("hawk_split_hot launch");
        if (rc != HK_OK) return rc;
        if (L.ranges > 0) {
            hipLaunchKernelGGL(hawk_split_tail<T>, dim3(static_cast<unsigned>(chunks * L.ranges)), dim3(kTailThreads),
                               0, s, static_cast<long long>(cells), L.tiles, L.ranges, bin_key, bin_val, bin_off,
                               parts);
            rc = launch_error("hawk_split_tail launch");
            if (rc != HK_OK) return rc;
        }
    } else {
        // more cells than the split walk's windows cover: parts arrives
        // zero-filled and the sorted walk (or, past its key field, the serial
        // walk) adds onto it
        const long long count = static_cast<long long>(chunks) * cells;
        const long long blocks = (count + 255) / 256 < 4096 ? (count + 255) / 256 : 4096;
        hipLaunchKernelGGL(hawk_fill_zero<T>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, parts, count);
        rc = launch_error("hawk_fill_zero launch");
        if (rc != HK_OK) return rc;
        const int key_bits = bits_for(cells - 1);
        if (key_bits <= kMaxKeyBits) {
            hipLaunchKernelGGL(hawk_scatter_walk<T>, dim3(static_cast<unsigned>(chunks)), dim3(kWalkThreads), 0, s,
                               key, v, static_cast<long long>(n), static_cast<long long>(cells), L.span, key_bits,
                               parts, status);
            rc = launch_error("hawk_scatter_walk launch");
        } else {
            hipLaunchKernelGGL(hawk_scatter_serial<T>, dim3(static_cast<unsigned>(chunks)), dim3(64), 0, s, key, v,
                               static_cast<long long>(n), static_cast<long long>(cells), L.span, parts, status);
            rc = launch_error("hawk_scatter_serial launch");
        }
        if (rc != HK_OK) return rc;
    }
    const long long grid = (cells + 255) / 256;
    hipLaunchKernelGGL(hawk_scatter_cells<T>, dim3(static_cast<unsigned>(grid)), dim3(256), 0, s, parts,
                       static_cast<long long>(cells), chunks, target);
    return launch_error("hawk_scatter_cells launch");
}

}  // namespace

extern "C" {

size_t hk_ordered_sum_scratch_bytes(void) { return kSumScratch; }

int hk_ordered_fold_f64(const double* lanes, double* out, void* scratch, void* stream) {
    if (!lanes || !out || !scratch)
        return hawk_internal::set_error(HK_EVALUE, "hk_ordered_fold_f64: lanes, out and scratch are required");
    auto* base = static_cast<unsigned char*>(scratch);
    auto* gp = reinterpret_cast<double*>(base + kLanesBytes);
    auto* ticket = reinterpret_cast<unsigned*>(base + kLanesBytes + kGpBytes);
    hipLaunchKernelGGL(hawk_sum_fold<double>, dim3(kGroups), dim3(256), 0, static_cast<hipStream_t>(stream),
                       lanes, gp, ticket, out);
    return launch_error("hawk_sum_fold launch");
}

int hk_ordered_sum_f64(const double* u, int64_t n, double* out, void* scratch, void* stream) {
    return ordered_sum<double>(u, n, out, scratch, stream, "hk_ordered_sum_f64");
}

int hk_ordered_sum_f32(const float* u, int64_t n, float* out, void* scratch, void* stream) {
    return ordered_sum<float>(u, n, out, scratch, stream, "hk_ordered_sum_f32");
}

size_t hk_ordered_sum_noalloc_scratch_bytes(void) { return kSumScratch; }

int hk_ordered_sum_f64_noalloc(const double* u, int64_t n, double* out, void* stream) {
    if (n < 0) return hawk_internal::set_error(HK_EVALUE, "hk_ordered_sum_f64_noalloc: n must be >= 0");
    if ((n > 0 && !u) || !out)
        return hawk_internal::set_error(HK_EVALUE, "hk_ordered_sum_f64_noalloc: u and out are required");
    void* ptr = nullptr;
    const int rc = scratch_of(static_cast<hipStream_t>(stream), &ptr);
    if (rc != HK_OK) return rc;
    return hk_ordered_sum_f64(u, n, out, ptr, stream);    // the same kernels, on the static scratch
}

size_t hk_keyed_ordered_sum_scratch_bytes(int64_t n, int64_t group) {
    if (n <= 0 || group <= 0 || n % group != 0) return 0;
    if (n == group) return kSumScratch;
    if (group <= kVirtualLanes) return 256;                  // the keys read their rows directly
    const long long lv = group < kVirtualLanes ? group : kVirtualLanes;
    return sizeof(double) * static_cast<size_t>(n / group) * static_cast<size_t>(lv) + 256;
}

int hk_keyed_ordered_sum_f64(const double* u, int64_t n, int64_t group, double* out, void* scratch, void* stream) {
    return keyed_ordered_sum<double>(u, n, group, out, scratch, stream, "hk_keyed_ordered_sum_f64");
}

int hk_keyed_ordered_sum_f32(const float* u, int64_t n, int64_t group, float* out, void* scratch, void* stream) {
    return keyed_ordered_sum<float>(u, n, group, out, scratch, stream, "hk_keyed_ordered_sum_f32");
}

int hk_keyed_sample_sum_f64(const double* u, int64_t n, int64_t group, double* out, void* stream) {
    return keyed_sample_sum<double>(u, n, group, out, stream, "hk_keyed_sample_sum_f64");
}

int hk_keyed_sample_sum_f32(const float* u, int64_t n, int64_t group, float* out, void* stream) {
    return keyed_sample_sum<float>(u, n, group, out, stream, "hk_keyed_sample_sum_f32");
}

size_t hk_rows_finish_scratch_bytes(int64_t rows) {
    if (rows <= 0) return 0;
    const long long leaves = (rows + kRowLeaf - 1) / kRowLeaf;
    return sizeof(double) * 4 * static_cast<size_t>(leaves);
}

int hk_rows_finish_f64(const double* hi, const double* comp, int64_t rows, double* out, void* scratch,
                       void* stream) {
    return rows_finish(hi, comp, rows, out, scratch, stream, "hk_rows_finish_f64");
}

int hk_rows_finish_f32(const float* hi, const float* comp, int64_t rows, float* out, void* scratch,
                       void* stream) {
    return rows_finish(hi, comp, rows, out, scratch, stream, "hk_rows_finish_f32");
}

int hk_rows_extreme_f64(const double* hi, int64_t rows, int32_t op, double* out, void* scratch, void* stream) {
    return rows_extreme(hi, rows, op, out, scratch, stream, "hk_rows_extreme_f64");
}

int hk_rows_extreme_f32(const float* hi, int64_t rows, int32_t op, float* out, void* scratch, void* stream) {
    return rows_extreme(hi, rows, op, out, scratch, stream, "hk_rows_extreme_f32");
}

size_t hk_band_rows_finish_scratch_bytes(int64_t rows) { return hk_rows_finish_scratch_bytes(rows); }

int hk_band_rows_finish_f64(const double* hi, const double* lo, int64_t rows, double* out, void* scratch,
                            void* stream) {
    if (rows < 1) return hawk_internal::set_error(HK_EVALUE, "hk_band_rows_finish_f64: rows must be >= 1");
    if (!hi || !lo || !out || !scratch)
        return hawk_internal::set_error(HK_EVALUE, "hk_band_rows_finish_f64: hi, lo, out and scratch are required");
    const long long leaves = (rows + kRowLeaf - 1) / kRowLeaf;
    if (leaves > 0x7fffffffLL) return hawk_internal::set_error(HK_EVALUE, "hk_band_rows_finish_f64: too many rows");
    auto* buf = static_cast<double*>(scratch);
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(hawk_band_rows_leaves, dim3(static_cast<unsigned>(leaves)), dim3(kRowSlots), 0, s, hi, lo,
                       static_cast<long long>(rows), buf, buf + leaves);
    int rc = launch_error("hawk_band_rows_leaves launch");
    if (rc != HK_OK) return rc;
    hipLaunchKernelGGL(hawk_band_rows_levels, dim3(1), dim3(256), 0, s, buf, leaves, out);
    return launch_error("hawk_band_rows_levels launch");
}

size_t hk_band_ordered_sum_scratch_bytes(void) { return kBandSumScratch; }

int hk_band_ordered_sum_f64(const double* u, int64_t n, double* out, void* scratch, void* stream) {
    if (n < 0) return hawk_internal::set_error(HK_EVALUE, "hk_band_ordered_sum_f64: n must be >= 0");
    if ((n > 0 && !u) || !out || !scratch)
        return hawk_internal::set_error(HK_EVALUE, "hk_band_ordered_sum_f64: u, out and scratch are required");
    auto* base = static_cast<unsigned char*>(scratch);
    auto* lanes = reinterpret_cast<Band*>(base);
    auto* gp = reinterpret_cast<Band*>(base + kBandLanesBytes);
    auto* ticket = reinterpret_cast<unsigned*>(base + kBandLanesBytes + kBandGpBytes);
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(hawk_band_sum_lanes, dim3(kBandVirtual / kBandChains), dim3(kBandThreads), 0, s, u,
                       static_cast<long long>(n), lanes, ticket);
    int rc = launch_error("hawk_band_sum_lanes launch");
    if (rc != HK_OK) return rc;
    hipLaunchKernelGGL(hawk_band_sum_fold, dim3(kGroups), dim3(256), 0, s, lanes, gp, ticket, out);
    return launch_error("hawk_band_sum_fold launch");
}

int hk_scatter_chunks(int64_t n, int64_t cells) {
    if (n <= 0) return 1;
    const int64_t fit = n / (cells < 1 ? 1 : cells);
    return static_cast<int>(fit < 1 ? 1 : (fit > kScatterChunks ? kScatterChunks : fit));
}

size_t hk_ordered_scatter_scratch_bytes(int64_t n, int64_t cells) {
    if (cells <= 0) return 0;
    return scatter_layout(n, cells, hk_scatter_chunks(n, cells)).bytes;
}

int hk_ordered_scatter_f64(const int32_t* key, const double* v, int64_t n, double* target, int64_t cells,
                           void* scratch, int32_t* status, void* stream) {
    return ordered_scatter<double>(key, v, n, target, cells, scratch, status, stream, "hk_ordered_scatter_f64");
}

int hk_ordered_scatter_f32(const int32_t* key, const float* v, int64_t n, float* target, int64_t cells,
                           void* scratch, int32_t* status, void* stream) {
    return ordered_scatter<float>(key, v, n, target, cells, scratch, status, stream, "hk_ordered_scatter_f32");
}

size_t hk_keyed_log_fold_scratch_bytes(int64_t cells) {
    return cells <= 0 ? 0 : sizeof(int) * static_cast<size_t>(cells);
}

int hk_keyed_log_fold_f64(const double* values, int64_t stride, const int32_t* cells_log, int64_t keys,
                          int64_t rows, int32_t width, double* out, int64_t cells, void* scratch,
                          int32_t* status, void* stream) {
    return keyed_log_fold<double>(values, stride, cells_log, keys, rows, width, out, cells, scratch, status, stream,
                                  "hk_keyed_log_fold_f64");
}

int hk_keyed_log_fold_f32(const float* values, int64_t stride, const int32_t* cells_log, int64_t keys,
                          int64_t rows, int32_t width, float* out, int64_t cells, void* scratch,
                          int32_t* status, void* stream) {
    return keyed_log_fold<float>(values, stride, cells_log, keys, rows, width, out, cells, scratch, status, stream,
                                 "hk_keyed_log_fold_f32");
}

}  // extern "C"
