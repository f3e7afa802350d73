// hawk_linalg.hip — per-sample 16x16 fp32 matrix products on gfx950 MFMA.
//
// A hawk kernel whose every sink is a product of two 16x16 fp32 planes (each
// possibly transposed) — the per-sample `mm` of reference
// hawk/emit/policy.py:283-299 and hawk/emit/writer_aether.py:663-671, and its
// VJP bar_A = bar_C B^T, bar_B = A^T bar_C — runs here as one team stage
// instead of a thread-per-sample loop.  Planes keep hawk's layout: element
// (r, c) of sample s at (r*16 + c)*N + s.
//
// A workgroup takes a tile of consecutive samples: 64 on 1024 threads for one
// product (each element row of the tile is a 256-byte run in HBM), 32 on 512
// threads for two (128-byte runs; the VJP's second set of accumulators would
// otherwise cost occupancy).  Workgroup i runs on XCD i % 8, so tiles are
// handed out XCD by XCD in contiguous eighths: the tiles one XCD's L2 serves
// are neighbours, which share the lines a run straddles when N*4 is not a
// multiple of 128.  The product's K = 16 runs as four MFMA K-slices
// (v_mfma_f32_16x16x4f32): for each slice the workgroup stages in LDS only
// the 64 operand elements of each side of each product (33-34 KB of LDS); the
// accumulators stay in registers across slices, and the results go back
// through LDS and out as contiguous element rows.

#include "hawk_core.h"
#include "hawk_internal.h"

#include <hip/hip_runtime.h>
#include <cstdint>
#include <string>

namespace {

constexpr int kDim = 16;
constexpr int kElems = kDim * kDim;          // 256 elements per sample
constexpr int kMaxIn = 3;
constexpr int kMaxOut = 2;
constexpr int kSlices = 4;                   // K = 16 as four MFMA K-slices of 4
constexpr int kSlotRows = 64;                // operand elements of one side of one product per slice

typedef float float4_t __attribute__((ext_vector_type(4)));

struct Product {
    int lhs, lhs_t, rhs, rhs_t, out;
};

struct MmArgs {
    const float* in[kMaxIn];
    float* out[kMaxOut];
    Product prod[kMaxOut];
    int n_in, n_out;
    int shared;              // two products reading one plane: its index (else -1)
    int shared_side[kMaxOut];  // the side (0 = lhs, 1 = rhs) product o reads it on
};

// The MFMA's operand fragments for K slice q: lane l holds A[i][k] with
// i = l % 16, k = 4q + l / 16 and B[k][j] with j = l % 16, k = 4q + l / 16;
// the 4 accumulator registers of lane l hold D[4*(l/16) + v][l % 16], v = 0..3.
__device__ __forceinline__ int lhs_elem(int lane, int q, int t) {
    const int i = lane & 15, k = 4 * q + (lane >> 4);
    return t ? k * kDim + i : i * kDim + k;
}
__device__ __forceinline__ int rhs_elem(int lane, int q, int t) {
    const int j = lane & 15, k = 4 * q + (lane >> 4);
    return t ? j * kDim + k : k * kDim + j;
}

// The launch shape per number of products: TILE samples on THREADS threads.
template <int NOUT> struct Shape;
template <> struct Shape<1> { static constexpr int kTile = 64, kThreads = 1024; };
template <> struct Shape<2> { static constexpr int kTile = 32, kThreads = 512; };

// LDS (NOUT products): during the products, slot (o*2 + side)*64 + l holds,
// for the tile's samples, the element that lane l of the MFMA reads for
// product o's side (0 = lhs, 1 = rhs) in the current K slice; afterwards the
// same memory holds half of one output (128 element rows) at a time.  A row
// is TILE + 1 floats: odd, so rows fall in different banks.
constexpr int kHalfRows = kElems / 2;
template <int NOUT>
constexpr int lds_floats() {
    return (NOUT * 2 * kSlotRows > kHalfRows ? NOUT * 2 * kSlotRows : kHalfRows) * (Shape<NOUT>::kTile + 1);
}

// Load slice q of the tile into registers: thread t takes sample s0 + t % TILE
// of slots t/TILE + (THREADS/TILE)*r, so every load instruction of a wave
// reads whole runs of TILE consecutive samples of an element row.
template <int NOUT>
__device__ __forceinline__ void slice_load(const MmArgs& args, long long n, long long s0, int count, int q,
                                           float (&staged)[NOUT * 2 * kSlotRows * Shape<NOUT>::kTile /
                                                           Shape<NOUT>::kThreads]) {
    constexpr int kTile = Shape<NOUT>::kTile;
    constexpr int kRowStep = Shape<NOUT>::kThreads / kTile;
    const int s_own = threadIdx.x % kTile;
    const int e_own = threadIdx.x / kTile;
    const bool live = s_own < count;
    constexpr int rows = NOUT * 2 * kSlotRows / kRowStep;
    // Slots 8r .. 8r+7 lie in one 64-slot group, so product and side depend on
    // r alone: the plane pointer and transposition are uniform per load.
    constexpr int kRowsPerGroup = kSlotRows / kRowStep;
#pragma unroll
    for (int r = 0; r < rows; ++r) {
        const int group = r / kRowsPerGroup;
        const int o = group >> 1, side = group & 1;
        const int l = e_own + (r % kRowsPerGroup) * kRowStep;
        const Product& pr = args.prod[o];
        const float* plane = args.in[side ? pr.rhs : pr.lhs];
        const int e = side ? rhs_elem(l, q, pr.rhs_t) : lhs_elem(l, q, pr.lhs_t);
        staged[r] = live ? __builtin_nontemporal_load(plane + static_cast<long long>(e) * n + s0 + s_own) : 0.0f;
    }
}

// One workgroup per tile: four K slices (the next slice's loads in flight
// during the current slice's MFMAs), then each output through LDS, half at a
// time, and out as contiguous element rows.  The grid is 8 * ceil(tiles / 8)
// workgroups; workgroup i takes tile (i % 8) * ceil(tiles / 8) + i / 8, and
// one past the last tile returns.
template <int NOUT>
__global__ __launch_bounds__(Shape<NOUT>::kThreads)
void hawk_mm16_f32(MmArgs args, long long n, long long tiles) {
    constexpr int kTile = Shape<NOUT>::kTile;
    constexpr int kStride = kTile + 1;
    constexpr int kWaves = Shape<NOUT>::kThreads / 64;
    constexpr int kRowStep = Shape<NOUT>::kThreads / kTile;
    __shared__ float lds[lds_floats<NOUT>()];
    constexpr int rows = NOUT * 2 * kSlotRows / kRowStep;
    const int t = threadIdx.x;
    const int wave = t >> 6;
    const int lane = t & 63;
    const int s_own = t % kTile;
    const int e_own = t / kTile;
    const long long per_xcd = (tiles + 7) / 8;
    const long long tile = static_cast<long long>(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (tile >= tiles) return;
    const long long s0 = tile * kTile;
    const int count = n - s0 < kTile ? static_cast<int>(n - s0) : kTile;

    float4_t acc[NOUT][kTile / kWaves];
#pragma unroll
    for (int o = 0; o < NOUT; ++o)
#pragma unroll
        for (int m = 0; m < kTile / kWaves; ++m) acc[o][m] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};

    float staged[rows];
    slice_load<NOUT>(args, n, s0, count, 0, staged);
#pragma unroll
    for (int q = 0; q < kSlices; ++q) {
        if (q > 0) __syncthreads();                     // the previous slice's operands are read
#pragma unroll
        for (int r = 0; r < rows; ++r) lds[(e_own + r * kRowStep) * kStride + s_own] = staged[r];
        __syncthreads();
        if (q + 1 < kSlices) slice_load<NOUT>(args, n, s0, count, q + 1, staged);
#pragma unroll
        for (int o = 0; o < NOUT; ++o) {
            const float* L = lds + (o * 2) * kSlotRows * kStride;
            const float* R = L + kSlotRows * kStride;
#pragma unroll
            for (int m = 0; m < kTile / kWaves; ++m) {
                const int s = wave + m * kWaves;
                acc[o][m] = __builtin_amdgcn_mfma_f32_16x16x4f32(L[lane * kStride + s], R[lane * kStride + s],
                                                                 acc[o][m], 0, 0, 0);
            }
        }
    }

    // Lane l holds rows 4*(l/16) .. +3 of column l % 16: rows 0..7 (the first
    // 128 elements) live in lanes 0..31, rows 8..15 in lanes 32..63.
#pragma unroll
    for (int o = 0; o < NOUT; ++o) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            __syncthreads();                            // the LDS is free for this half
            if ((lane >> 5) == h) {
#pragma unroll
                for (int m = 0; m < kTile / kWaves; ++m) {
                    const int s = wave + m * kWaves;
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int e = (4 * (lane >> 4) + v) * kDim + (lane & 15) - h * kHalfRows;
                        lds[e * kStride + s] = acc[o][m][v];
                    }
                }
            }
            __syncthreads();
            if (s_own < count) {
                float* dst = args.out[o] + s0 + s_own;
#pragma unroll
                for (int r = 0; r < kHalfRows / kRowStep; ++r) {
                    const int e = e_own + r * kRowStep;
                    __builtin_nontemporal_store(lds[e * kStride + s_own],
                                                dst + static_cast<long long>(e + h * kHalfRows) * n);
                }
            }
        }
    }
}

// Two products that read one plane between them (the VJP: bar_A = bar_C B^T
// and bar_B = A^T bar_C both read bar_C) on 32-sample tiles of 512 threads:
// the shared plane's whole tile (256 element rows) is staged in LDS once, and
// each K slice stages only the other operand of each product, so every input
// element is read from HBM once.  LDS: the shared tile (33 KB, later the
// output halves) and one slice of the two other operands (17 KB).
constexpr int kShTile = 32, kShThreads = 512, kShStride = kShTile + 1, kShRowStep = kShThreads / kShTile;
constexpr int kShWaves = kShThreads / 64;
constexpr int kShFullRows = kElems / kShRowStep;          // 16 shared-tile rows per thread
constexpr int kShSliceRows = 2 * kSlotRows / kShRowStep;  // 8 slice rows per thread

// Slice q of the non-shared operands: slot row o*64 + l holds the element lane
// l of the MFMA reads from product o's other side.
__device__ __forceinline__ void shared_slice_load(const MmArgs& args, long long n, long long s0, int count, int q,
                                                  float (&staged)[kShSliceRows]) {
    const int s_own = threadIdx.x % kShTile;
    const int e_own = threadIdx.x / kShTile;
    const bool live = s_own < count;
    constexpr int kRowsPerGroup = kSlotRows / kShRowStep;
#pragma unroll
    for (int r = 0; r < kShSliceRows; ++r) {
        const int o = r / kRowsPerGroup;
        const int l = e_own + (r % kRowsPerGroup) * kShRowStep;
        const Product& pr = args.prod[o];
        const bool other_rhs = args.shared_side[o] == 0;
        const float* plane = args.in[other_rhs ? pr.rhs : pr.lhs];
        const int e = other_rhs ? rhs_elem(l, q, pr.rhs_t) : lhs_elem(l, q, pr.lhs_t);
        staged[r] = live ? __builtin_nontemporal_load(plane + static_cast<long long>(e) * n + s0 + s_own) : 0.0f;
    }
}

__global__ __launch_bounds__(kShThreads)
void hawk_mm16_f32_shared(MmArgs args, long long n, long long tiles) {
    __shared__ float full[kElems * kShStride];
    __shared__ float slot[2 * kSlotRows * kShStride];
    const int t = threadIdx.x;
    const int wave = t >> 6;
    const int lane = t & 63;
    const int s_own = t % kShTile;
    const int e_own = t / kShTile;
    const long long per_xcd = (tiles + 7) / 8;
    const long long tile = static_cast<long long>(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (tile >= tiles) return;
    const long long s0 = tile * kShTile;
    const int count = n - s0 < kShTile ? static_cast<int>(n - s0) : kShTile;
    const bool live = s_own < count;

    const float* S = args.in[args.shared];
    float whole[kShFullRows];
#pragma unroll
    for (int r = 0; r < kShFullRows; ++r)
        whole[r] = live ? __builtin_nontemporal_load(S + static_cast<long long>(e_own + r * kShRowStep) * n + s0 + s_own)
                        : 0.0f;
    float staged[kShSliceRows];
    shared_slice_load(args, n, s0, count, 0, staged);
#pragma unroll
    for (int r = 0; r < kShFullRows; ++r) full[(e_own + r * kShRowStep) * kShStride + s_own] = whole[r];

    float4_t acc[2][kShTile / kShWaves];
#pragma unroll
    for (int o = 0; o < 2; ++o)
#pragma unroll
        for (int m = 0; m < kShTile / kShWaves; ++m) acc[o][m] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int q = 0; q < kSlices; ++q) {
        if (q > 0) __syncthreads();                     // the previous slice's operands are read
#pragma unroll
        for (int r = 0; r < kShSliceRows; ++r) slot[(e_own + r * kShRowStep) * kShStride + s_own] = staged[r];
        __syncthreads();
        if (q + 1 < kSlices) shared_slice_load(args, n, s0, count, q + 1, staged);
#pragma unroll
        for (int o = 0; o < 2; ++o) {
            const Product& pr = args.prod[o];
            const bool lhs_shared = args.shared_side[o] == 0;
            const int e = lhs_shared ? lhs_elem(lane, q, pr.lhs_t) : rhs_elem(lane, q, pr.rhs_t);
            const float* F = full + e * kShStride;
            const float* O = slot + (o * kSlotRows + lane) * kShStride;
#pragma unroll
            for (int m = 0; m < kShTile / kShWaves; ++m) {
                const int sm = wave + m * kShWaves;
                const float fv = F[sm], ov = O[sm];
                acc[o][m] = __builtin_amdgcn_mfma_f32_16x16x4f32(lhs_shared ? fv : ov, lhs_shared ? ov : fv,
                                                                 acc[o][m], 0, 0, 0);
            }
        }
    }

    // As hawk_mm16_f32: each output through LDS (the shared tile's memory),
    // half at a time, and out as contiguous element rows.
#pragma unroll
    for (int o = 0; o < 2; ++o) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            __syncthreads();
            if ((lane >> 5) == h) {
#pragma unroll
                for (int m = 0; m < kShTile / kShWaves; ++m) {
                    const int sm = wave + m * kShWaves;
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int e = (4 * (lane >> 4) + v) * kDim + (lane & 15) - h * kHalfRows;
                        full[e * kShStride + sm] = acc[o][m][v];
                    }
                }
            }
            __syncthreads();
            if (live) {
                float* dst = args.out[o] + s0 + s_own;
#pragma unroll
                for (int r = 0; r < kHalfRows / kShRowStep; ++r) {
                    const int e = e_own + r * kShRowStep;
                    __builtin_nontemporal_store(full[e * kShStride + s_own],
                                                dst + static_cast<long long>(e + h * kHalfRows) * n);
                }
            }
        }
    }
}

int launch_error(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hawk_internal::set_hip_error(what, e);
    return HK_OK;
}

}  // namespace

extern "C" {

int hk_mm16_f32(const float* const* in, int n_in, float* const* out, int n_out, const int32_t* products,
                int64_t n, void* stream) {
    if (n_in < 1 || n_in > kMaxIn || n_out < 1 || n_out > kMaxOut || n_out > n_in)
        return hawk_internal::set_error(HK_EVALUE,
                                        "hk_mm16_f32: 1..3 input planes and 1..2 products, no more products than inputs");
    if (n < 0) return hawk_internal::set_error(HK_EVALUE, "hk_mm16_f32: n must be >= 0");
    if (!in || !out || !products)
        return hawk_internal::set_error(HK_EVALUE, "hk_mm16_f32: in, out and products are required");
    MmArgs args{};
    args.n_in = n_in;
    args.n_out = n_out;
    for (int p = 0; p < n_in; ++p) {
        if (!in[p]) return hawk_internal::set_error(HK_EVALUE, "hk_mm16_f32: input plane " + std::to_string(p) + " is null");
        args.in[p] = in[p];
    }
    for (int o = 0; o < n_out; ++o) {
        const int32_t* d = products + 3 * o;
        const Product pr{d[0], d[2] & 1, d[1], (d[2] >> 1) & 1, o};
        if (pr.lhs < 0 || pr.lhs >= n_in || pr.rhs < 0 || pr.rhs >= n_in)
            return hawk_internal::set_error(HK_EINDEX, "hk_mm16_f32: product " + std::to_string(o) +
                                                           " names an input plane outside [0, n_in)");
        if (!out[o]) return hawk_internal::set_error(HK_EVALUE, "hk_mm16_f32: output plane " + std::to_string(o) + " is null");
        args.prod[o] = pr;
        args.out[o] = out[o];
    }
    // Two products that share exactly one plane, each reading it on one side,
    // take the kernel that stages it once.
    args.shared = -1;
    if (n_out == 2 && args.prod[0].lhs != args.prod[0].rhs && args.prod[1].lhs != args.prod[1].rhs) {
        for (int side = 0; side < 2 && args.shared < 0; ++side) {
            const int cand = side == 0 ? args.prod[0].lhs : args.prod[0].rhs;
            if (cand == args.prod[1].lhs || cand == args.prod[1].rhs) {
                args.shared = cand;
                args.shared_side[0] = side;
                args.shared_side[1] = cand == args.prod[1].lhs ? 0 : 1;
            }
        }
    }
    if (n == 0) return HK_OK;
    if (args.shared >= 0) {
        const long long tiles = (n + kShTile - 1) / kShTile;
        const long long grid = 8 * ((tiles + 7) / 8);
        if (grid > 0x7fffffffLL) return hawk_internal::set_error(HK_EVALUE, "hk_mm16_f32: too many samples");
        hipLaunchKernelGGL(hawk_mm16_f32_shared, dim3(static_cast<unsigned>(grid)), dim3(kShThreads), 0,
                           static_cast<hipStream_t>(stream), args, static_cast<long long>(n), tiles);
        return launch_error("hawk_mm16_f32_shared launch");
    }
    const int tile = n_out == 1 ? Shape<1>::kTile : Shape<2>::kTile;
    const long long tiles = (n + tile - 1) / tile;
    const long long grid = 8 * ((tiles + 7) / 8);     // every tile gets a workgroup on its XCD
    if (grid > 0x7fffffffLL) return hawk_internal::set_error(HK_EVALUE, "hk_mm16_f32: too many samples");
    if (n_out == 1)
        hipLaunchKernelGGL(hawk_mm16_f32<1>, dim3(static_cast<unsigned>(grid)), dim3(Shape<1>::kThreads), 0,
                           static_cast<hipStream_t>(stream), args, static_cast<long long>(n), tiles);
    else
        hipLaunchKernelGGL(hawk_mm16_f32<2>, dim3(static_cast<unsigned>(grid)), dim3(Shape<2>::kThreads), 0,
                           static_cast<hipStream_t>(stream), args, static_cast<long long>(n), tiles);
    return launch_error("hawk_mm16_f32 launch");
}

}  // extern "C"
