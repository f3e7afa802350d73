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
__global__ __launch_bounds__(kLaneBlock) void hawk_sum_lanes(const double* __restrict__ u,
                                                              long long n,
                                                              double* __restrict__ lanes) {
    const long long l = static_cast<long long>(blockIdx.x) * kLaneBlock + threadIdx.x;
    double s = 0.0;
    long long r = l;
    constexpr long long kStep = kVirtualLanes;
    for (; r + (kSumUnroll - 1) * kStep < n; r += kSumUnroll * kStep) {
        double a[kSumUnroll];
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
__global__ __launch_bounds__(256) void hawk_sum_fold(const double* __restrict__ lanes,
                                                     double* __restrict__ gp,
                                                     unsigned* __restrict__ ticket,
                                                     double* __restrict__ out) {
    __shared__ double sh[kFoldLanes];
    __shared__ unsigned last;
    const int g = blockIdx.x;
    const int t = threadIdx.x;
    for (int i = t; i < kFoldLanes; i += 256) sh[i] = lanes[g * kFoldLanes + i];
    __syncthreads();
    for (int w = kFoldLanes / 2; w > 0; w >>= 1) {
        for (int i = t; i < w; i += 256) sh[i] = sh[i] + sh[i + w];
        __syncthreads();
    }
    if (t == 0) {
        gp[g] = sh[0];
        __threadfence();
        last = atomicAdd(ticket, 1u);
    }
    __syncthreads();
    if (last != kGroups - 1) return;
    __threadfence();   // acquire: every group's gp store is visible
    if (t < kGroups) sh[t] = __builtin_nontemporal_load(gp + t);
    __syncthreads();
    for (int w = kGroups / 2; w > 0; w >>= 1) {
        if (t < w) sh[t] = sh[t] + sh[t + w];
        __syncthreads();
    }
    if (t == 0) {
        *out = sh[0];
        *ticket = 0u;
    }
}

// ---------------------------------------------------------------------------
// Keyed ordered scatter.
// ---------------------------------------------------------------------------
constexpr int kScatterChunks = 256;    // reference hawk/_lane_bind.py:108
constexpr int kWalkThreads = 512;
constexpr int kWalkWaves = kWalkThreads / 64;
constexpr int kWalkItems = 8;                      // keys per thread per tile (striped)
constexpr int kTile = kWalkThreads * kWalkItems;   // 4096 raw lanes per tile
constexpr int kStage = 2048;                       // staged entries per batch
constexpr int kSortItems = kStage / kWalkThreads;  // 4 per thread in the sort
constexpr int kIdxBits = 11;                       // 2^11 == kStage
constexpr int kBinCap = 8192;                      // f64 bins a workgroup holds in LDS (64 KiB)
constexpr int kDigitBits = 4;
constexpr int kDigits = 1 << kDigitBits;

__device__ __forceinline__ unsigned wave_inclusive_scan(unsigned v) {
    const int lane = threadIdx.x & 63;
    unsigned x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        unsigned y = __shfl_up(x, d, 64);
        if (lane >= d) x += y;
    }
    return x;
}

// Exclusive scan of one value per thread over the block (all threads call it).
__device__ __forceinline__ unsigned block_exclusive_scan(unsigned v, unsigned* scratch, unsigned* total) {
    const unsigned incl = wave_inclusive_scan(v);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 63) scratch[wave] = incl;
    __syncthreads();
    unsigned before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kWalkWaves; ++w) {
        const unsigned s = scratch[w];
        if (w < wave) before += s;
        all += s;
    }
    __syncthreads();
    *total = all;
    return incl - v + before;
}

struct WalkShared {
    double bins[kBinCap];                          // 64 KiB: this partition's partial sums
    unsigned comp[2][kStage];                      // 16 KiB: (local key << 11) | staged index
    double vals[kStage];                           // 16 KiB: staged values, arrival order
    double sorted_vals[kStage];                    // 16 KiB: values in sorted order
    unsigned counts[kDigits * kWalkWaves * kSortItems];   // 2 KiB: per (digit, wave, slot)
    unsigned scan[kWalkWaves];
    unsigned slab[kWalkItems][kWalkWaves];         // per (slab, wave) counts of a tile
    int longs[kStage / 64 + 1];                    // heads of runs of 64 or more
    int nlong;
};

static_assert(kDigits * kWalkWaves * kSortItems == kWalkThreads, "one radix counter per thread");

// Stable LSD radix sort of the kStage composite keys over bits [lo, hi), 4 bits
// a pass, ping-ponging comp[0] <-> comp[1]; returns the buffer holding the
// result.  Element e = wave*256 + slot*64 + lane (the input order); within a
// (wave, slot) group the lanes with one digit are ranked by ballots, and the
// exclusive scan over (digit, wave, slot) in that order places every group's
// members after all earlier ones: each pass is stable.
__device__ int radix_sort(WalkShared& sh, int lo, int hi) {
    const int t = threadIdx.x;
    const int wave = t >> 6;
    const int lane = t & 63;
    const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int src = 0;
    for (int shift = lo; shift < hi; shift += kDigitBits) {
        const unsigned* in = sh.comp[src];
        unsigned* out = sh.comp[src ^ 1];
        unsigned item[kSortItems], digit[kSortItems], rank[kSortItems];
#pragma unroll
        for (int j = 0; j < kSortItems; ++j) {
            item[j] = in[wave * (kSortItems * 64) + j * 64 + lane];
            digit[j] = (item[j] >> shift) & (kDigits - 1);
            unsigned long long bits[kDigitBits];
#pragma unroll
            for (int b = 0; b < kDigitBits; ++b) bits[b] = __ballot((digit[j] >> b) & 1u);
            unsigned long long peers = ~0ull;          // lanes whose digit equals mine
#pragma unroll
            for (int b = 0; b < kDigitBits; ++b) peers &= ((digit[j] >> b) & 1u) ? bits[b] : ~bits[b];
            rank[j] = static_cast<unsigned>(__popcll(peers & below));
            // lane d < 16 counts the group's members with digit d
            unsigned long long with_d = ~0ull;
#pragma unroll
            for (int b = 0; b < kDigitBits; ++b) with_d &= ((lane >> b) & 1) ? bits[b] : ~bits[b];
            if (lane < kDigits)
                sh.counts[(lane * kWalkWaves + wave) * kSortItems + j] = static_cast<unsigned>(__popcll(with_d));
        }
        __syncthreads();
        unsigned total;
        const unsigned off = block_exclusive_scan(sh.counts[t], sh.scan, &total);
        sh.counts[t] = off;                          // every thread read its count before the scan's barrier
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kSortItems; ++j)
            out[sh.counts[(digit[j] * kWalkWaves + wave) * kSortItems + j] + rank[j]] = item[j];
        __syncthreads();
        src ^= 1;
    }
    return src;
}

// Sort the `m` staged entries by local key (stable, so arrival order holds
// within a key) and add each key's run, in order, onto its bin: a run shorter
// than 64 by one lane, a longer one by a whole wave (64 values per LDS load,
// folded in order through uniform readlanes).
__device__ void flush_batch(WalkShared& sh, int m, int key_bits) {
    const int t = threadIdx.x;
    const int wave = t >> 6;
    const int lane = t & 63;
    for (int j = m + t; j < kStage; j += kWalkThreads) sh.comp[0][j] = 0xffffffffu;
    if (t == 0) sh.nlong = 0;
    __syncthreads();
    const int buf = radix_sort(sh, kIdxBits, kIdxBits + key_bits);
    unsigned* comp = sh.comp[buf];
    for (int j = t; j < m; j += kWalkThreads) sh.sorted_vals[j] = sh.vals[comp[j] & (kStage - 1)];
    __syncthreads();
    for (int j = t; j < m; j += kWalkThreads) {
        const unsigned key = comp[j] >> kIdxBits;
        if (j > 0 && (comp[j - 1] >> kIdxBits) == key) continue;   // not the head of its run
        if (j + 63 < m && (comp[j + 63] >> kIdxBits) == key) {     // sorted: a run of 64 or more
            sh.longs[atomicAdd(&sh.nlong, 1)] = j;
            continue;
        }
        double acc = sh.bins[key];
        for (int jj = j; jj < m && (comp[jj] >> kIdxBits) == key; ++jj) acc = acc + sh.sorted_vals[jj];
        sh.bins[key] = acc;
    }
    __syncthreads();
    for (int r = wave; r < sh.nlong; r += kWalkWaves) {
        const int j = sh.longs[r];
        const unsigned key = comp[j] >> kIdxBits;
        double acc = sh.bins[key];
        for (int base = j; base < m; base += 64) {
            const int e = base + lane;
            const bool in = e < m && (comp[e] >> kIdxBits) == key;
            const double x = in ? sh.sorted_vals[e] : 0.0;
            const int cnt = __popcll(__ballot(in));     // a prefix of the lanes: the run is contiguous
            const int xlo = __double2loint(x);
            const int xhi = __double2hiint(x);
            for (int k = 0; k < cnt; ++k)
                acc = acc + __hiloint2double(__builtin_amdgcn_readlane(xhi, k), __builtin_amdgcn_readlane(xlo, k));
            if (cnt < 64) break;
        }
        if (lane == 0) sh.bins[key] = acc;
    }
    __syncthreads();
}

// Load the striped tile at `tile`: element j*512 + t of the tile goes to
// thread t's slot j, so every load instruction of a wave is one contiguous run.
__device__ __forceinline__ void load_tile(const int* __restrict__ key, const double* __restrict__ v, long long tile,
                                          long long hi, int (&kk)[kWalkItems], double (&vv)[kWalkItems]) {
#pragma unroll
    for (int j = 0; j < kWalkItems; ++j) {
        const long long i = tile + static_cast<long long>(j) * kWalkThreads + threadIdx.x;
        const bool in = i < hi;
        kk[j] = in ? __builtin_nontemporal_load(key + i) : -1;
        vv[j] = in ? __builtin_nontemporal_load(v + i) : 0.0;
    }
}

// One workgroup per (chunk b, key partition q): keys k with k % Q == q, local
// key k / Q, live in LDS bins.  The workgroup walks its chunk's lanes in
// order (the next tile's keys and values in flight while the current one is
// staged), stages its partition's (key, value) pairs in lane order, and adds
// every batch into the bins; the bins of every key of the partition (zeros
// included) go to partsT[b*cells + k] at the end, so no zeroing stage is
// needed.  The Q workgroups of one chunk take consecutive dispatch slots of
// one XCD, so the chunk's keys are fetched from HBM once and re-read from L2.
__global__ __launch_bounds__(kWalkThreads) void hawk_scatter_walk(
        const int* __restrict__ key, const double* __restrict__ v, long long n, long long cells,
        int chunks, long long span, int parts, int key_bits, double* __restrict__ partsT,
        int* __restrict__ status) {
    __shared__ WalkShared sh;
    const int t = threadIdx.x;
    const int wave = t >> 6;
    const int lane = t & 63;
    const long long total = static_cast<long long>(chunks) * parts;
    long long w = blockIdx.x;
    if (total % 8 == 0) w = (blockIdx.x % 8) * (total / 8) + blockIdx.x / 8;
    const int b = static_cast<int>(w / parts);
    const int q = static_cast<int>(w % parts);
    const long long lo = static_cast<long long>(b) * span;
    const long long hi = lo + span < n ? lo + span : n;
    const long long nb = (cells - q + parts - 1) / parts;   // keys q, q+Q, ... below cells

    for (long long k = t; k < nb; k += kWalkThreads) sh.bins[k] = 0.0;
    int staged = 0;
    bool bad = false;
    int nk[kWalkItems];
    double nv[kWalkItems];
    if (lo < hi) load_tile(key, v, lo, hi, nk, nv);
    __syncthreads();
    for (long long tile = lo; tile < hi; tile += kTile) {
        int kk[kWalkItems];
        double vv[kWalkItems];
#pragma unroll
        for (int j = 0; j < kWalkItems; ++j) { kk[j] = nk[j]; vv[j] = nv[j]; }
        if (tile + kTile < hi) load_tile(key, v, tile + kTile, hi, nk, nv);
        // Per slab j (512 consecutive lanes), this wave's members in lane order.
        unsigned long long mask[kWalkItems];
#pragma unroll
        for (int j = 0; j < kWalkItems; ++j) {
            const bool valid = kk[j] >= 0 && kk[j] < cells;
            bad = bad || (kk[j] != -1 && !valid);
            const bool mine = valid && (kk[j] % parts == q);
            mask[j] = __ballot(mine);
            if (lane == 0) sh.slab[j][wave] = static_cast<unsigned>(__popcll(mask[j]));
        }
        __syncthreads();
        // Offsets: all of slab j' < j first, then the waves before this one in slab j.
        unsigned before[kWalkItems];
        unsigned m = 0;
#pragma unroll
        for (int j = 0; j < kWalkItems; ++j) {
            unsigned inslab = 0, mine_before = 0;
#pragma unroll
            for (int x = 0; x < kWalkWaves; ++x) {
                const unsigned c = sh.slab[j][x];
                if (x < wave) mine_before += c;
                inslab += c;
            }
            before[j] = m + mine_before;
            m += inslab;
        }
        if (staged + static_cast<int>(m) > kStage) {
            flush_batch(sh, staged, key_bits);      // ends with a barrier
            staged = 0;
        }
        const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
        for (int j = 0; j < kWalkItems; ++j) {
            if (!((mask[j] >> lane) & 1ull)) continue;
            const unsigned idx = static_cast<unsigned>(staged) + before[j] +
                                 static_cast<unsigned>(__popcll(mask[j] & below));
            sh.comp[0][idx] = (static_cast<unsigned>(kk[j] / parts) << kIdxBits) | idx;
            sh.vals[idx] = vv[j];
        }
        staged += static_cast<int>(m);
        __syncthreads();
    }
    if (staged > 0) flush_batch(sh, staged, key_bits);
    double* row = partsT + static_cast<long long>(b) * cells;
    for (long long k = t; k < nb; k += kWalkThreads) row[k * parts + q] = sh.bins[k];
    if (bad) status[1 + b] = 1;
}

// Cell c adds its chunk partials in chunk order from +0.0, then onto the
// target: target[c] += sum (reference hawk/emit/team.py:437-460).
__global__ __launch_bounds__(256) void hawk_scatter_cells(const double* __restrict__ partsT, long long cells,
                                                          int chunks, double* __restrict__ target) {
    const long long c = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    if (c >= cells) return;
    double s = 0.0;
    for (int b = 0; b < chunks; ++b) s = s + partsT[static_cast<long long>(b) * cells + c];
    target[c] = target[c] + s;
}

__global__ void hawk_scatter_status(int* status, long long cells) {
    const int t = threadIdx.x;
    if (t == 0) status[0] = static_cast<int>(cells);
    if (t < kScatterChunks) status[1 + t] = 0;
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

extern "C" {

size_t hk_ordered_sum_scratch_bytes(void) { return kSumScratch; }

int hk_ordered_fold_f64(const double* lanes, double* out, void* scratch, void* stream) {
    if (!lanes || !out || !scratch)
        return hawk_internal::set_error(HK_EVALUE, "hk_ordered_fold_f64: lanes, out and scratch are required");
    auto* base = static_cast<unsigned char*>(scratch);
    auto* gp = reinterpret_cast<double*>(base + kLanesBytes);
    auto* ticket = reinterpret_cast<unsigned*>(base + kLanesBytes + kGpBytes);
    hipLaunchKernelGGL(hawk_sum_fold, dim3(kGroups), dim3(256), 0, static_cast<hipStream_t>(stream),
                       lanes, gp, ticket, out);
    return launch_error("hawk_sum_fold launch");
}

int hk_ordered_sum_f64(const double* u, int64_t n, double* out, void* scratch, void* stream) {
    if (n < 0) return hawk_internal::set_error(HK_EVALUE, "hk_ordered_sum_f64: n must be >= 0");
    if ((n > 0 && !u) || !out || !scratch)
        return hawk_internal::set_error(HK_EVALUE, "hk_ordered_sum_f64: u, out and scratch are required");
    auto* lanes = static_cast<double*>(scratch);
    hipLaunchKernelGGL(hawk_sum_lanes, dim3(kVirtualLanes / kLaneBlock), dim3(kLaneBlock), 0,
                       static_cast<hipStream_t>(stream), u, static_cast<long long>(n), lanes);
    int rc = launch_error("hawk_sum_lanes launch");
    if (rc != HK_OK) return rc;
    return hk_ordered_fold_f64(lanes, out, scratch, stream);
}

int hk_scatter_chunks(int64_t n, int64_t cells) {
    if (n <= 0) return 1;
    const int64_t fit = n / (cells < 1 ? 1 : cells);
    return static_cast<int>(fit < 1 ? 1 : (fit > kScatterChunks ? kScatterChunks : fit));
}

size_t hk_ordered_scatter_scratch_bytes(int64_t n, int64_t cells) {
    if (cells <= 0) return 0;
    return sizeof(double) * static_cast<size_t>(hk_scatter_chunks(n, cells)) * static_cast<size_t>(cells);
}

int hk_ordered_scatter_f64(const int32_t* key, const double* v, int64_t n, double* target, int64_t cells,
                           void* scratch, int32_t* status, void* stream) {
    if (n < 0 || cells < 0)
        return hawk_internal::set_error(HK_EVALUE, "hk_ordered_scatter_f64: n and cells must be >= 0");
    if (cells == 0) return HK_OK;   // a scatter into no cells adds nothing (reference hawk/runtime.py:727)
    if ((n > 0 && (!key || !v)) || !target || !scratch || !status)
        return hawk_internal::set_error(HK_EVALUE,
                                        "hk_ordered_scatter_f64: key, v, target, scratch and status are required");
    if (cells > 0x7fffffffLL)
        return hawk_internal::set_error(HK_EVALUE, "hk_ordered_scatter_f64: more than 2^31-1 cells");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int chunks = hk_scatter_chunks(n, cells);
    const long long span = (n + chunks - 1) / chunks;
    const long long parts = (cells + kBinCap - 1) / kBinCap;
    const long long nb = (cells + parts - 1) / parts;
    const int key_bits = bits_for(nb - 1);
    if (key_bits + kIdxBits > 31)
        return hawk_internal::set_error(HK_EVALUE, "hk_ordered_scatter_f64: too many cells for one partition");
    hipLaunchKernelGGL(hawk_scatter_status, dim3(1), dim3(kScatterChunks + 64), 0, s, status,
                       static_cast<long long>(cells));
    int rc = launch_error("hawk_scatter_status launch");
    if (rc != HK_OK) return rc;
    const long long blocks = static_cast<long long>(chunks) * parts;
    if (blocks > 0x7fffffffLL) return hawk_internal::set_error(HK_EVALUE, "hk_ordered_scatter_f64: grid too large");
    auto* partsT = static_cast<double*>(scratch);
    hipLaunchKernelGGL(hawk_scatter_walk, dim3(static_cast<unsigned>(blocks)), dim3(kWalkThreads), 0, s, key, v,
                       static_cast<long long>(n), static_cast<long long>(cells), chunks, span,
                       static_cast<int>(parts), key_bits, partsT, status);
    rc = launch_error("hawk_scatter_walk launch");
    if (rc != HK_OK) return rc;
    const long long grid = (cells + 255) / 256;
    hipLaunchKernelGGL(hawk_scatter_cells, dim3(static_cast<unsigned>(grid)), dim3(256), 0, s, partsT,
                       static_cast<long long>(cells), chunks, target);
    return launch_error("hawk_scatter_cells launch");
}

}  // extern "C"
