// hawk_linalg.hip — per-sample 16x16 matrix products on gfx950 MFMA, fp32 and fp64.
//
// A hawk kernel whose every sink is a product of two 16x16 planes (each
// possibly transposed) — the per-sample `mm` of reference
// hawk/emit/policy.py:283-299 and hawk/emit/writer_aether.py:663-671, and its
// VJP bar_A = bar_C B^T, bar_B = A^T bar_C — runs here as one team stage
// instead of a thread-per-sample loop.  Planes keep hawk's layout: element
// (r, c) of sample s at (r*16 + c)*N + s.
//
// A workgroup takes a tile of consecutive samples whose element rows are
// 256-byte runs in HBM for one product (fp32: 64 samples on 1024 threads;
// fp64: 32 on 1024) and 128-byte runs for two (fp32: 32 on 512; fp64: 16 on
// 512, or on 256 when the two share a plane; the VJP's second set of
// accumulators would otherwise cost occupancy).
// Workgroup i runs on XCD i % 8, so tiles are handed out XCD by XCD in
// contiguous eighths: the tiles one XCD's L2 serves are neighbours, which
// share the lines a run straddles when N*sizeof(T) is not a multiple of 128.
// The product's K = 16 runs as four MFMA K-slices (v_mfma_f32_16x16x4f32 or
// v_mfma_f64_16x16x4f64, whose operand and accumulator layouts are the same):
// for each slice the workgroup stages in LDS only the 64 operand elements of
// each side of each product (33-34 KB of LDS either way); the accumulators
// stay in registers across slices, and the results go back through LDS and
// out as contiguous element rows.

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
typedef double double4_t __attribute__((ext_vector_type(4)));

// One MFMA K-slice step per element type, D += A(16x4) B(4x16), and the row
// of D that accumulator register v of a lane holds (its column is lane % 16):
// 4*(lane/16) + v for v_mfma_f32_16x16x4f32, lane/16 + 4v for
// v_mfma_f64_16x16x4f64 (read off the device with known operands).
template <class T> struct Mfma;
template <> struct Mfma<float> {
    typedef float4_t acc;
    __device__ static __forceinline__ acc step(float a, float b, acc c) {
        return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
    }
    __device__ static __forceinline__ int row(int lane, int v) { return 4 * (lane >> 4) + v; }
};
template <> struct Mfma<double> {
    typedef double4_t acc;
    __device__ static __forceinline__ acc step(double a, double b, acc c) {
        return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
    }
    __device__ static __forceinline__ int row(int lane, int v) { return (lane >> 4) + 4 * v; }
};

struct Product {
    int lhs, lhs_t, rhs, rhs_t, out;
};

template <class T>
struct MmArgs {
    const T* in[kMaxIn];
    T* out[kMaxOut];
    Product prod[kMaxOut];
    int n_in, n_out;
    int shared;              // two products reading one plane: its index (else -1)
    int shared_side[kMaxOut];  // the side (0 = lhs, 1 = rhs) product o reads it on
};

// The MFMA's operand fragments for K slice q (both types): lane l holds
// A[i][k] with i = l % 16, k = 4q + l / 16 and B[k][j] with j = l % 16,
// k = 4q + l / 16; the accumulators' rows are Mfma<T>::row.
__device__ __forceinline__ int lhs_elem(int lane, int q, int t) {
    const int i = lane & 15, k = 4 * q + (lane >> 4);
    return t ? k * kDim + i : i * kDim + k;
}
__device__ __forceinline__ int rhs_elem(int lane, int q, int t) {
    const int j = lane & 15, k = 4 * q + (lane >> 4);
    return t ? j * kDim + k : k * kDim + j;
}

// The launch shape per element type and number of products: TILE samples,
// TILE * sizeof(T) = 256 bytes for one product and 128 for two, on 16 threads
// a sample for fp32 and 32 for fp64.  With 32, a thread stages half an fp64
// slice's rows and a CU has twice as many rows in flight (the fp64 forward at
// 2^20 samples: 1.30 ms on 512 threads, 1.25 ms on 1024).
template <class T, int NOUT> struct Shape {
    static constexpr int kTile = 256 / static_cast<int>(sizeof(T)) / NOUT;
    static constexpr int kThreads = (sizeof(T) == 8 ? 32 : 16) * kTile;
};

// LDS (NOUT products): during the products, slot (o*2 + side)*64 + l holds,
// for the tile's samples, the element that lane l of the MFMA reads for
// product o's side (0 = lhs, 1 = rhs) in the current K slice; afterwards the
// same memory holds half of one output (128 element rows) at a time.  A row
// is TILE + 1 elements: odd, so rows fall in different banks.
constexpr int kHalfRows = kElems / 2;
template <class T, int NOUT>
constexpr int lds_elems() {
    return (NOUT * 2 * kSlotRows > kHalfRows ? NOUT * 2 * kSlotRows : kHalfRows) * (Shape<T, NOUT>::kTile + 1);
}

// Load slice q of the tile into registers: thread t takes sample s0 + t % TILE
// of slots t/TILE + (THREADS/TILE)*r, so every load instruction of a wave
// reads whole runs of TILE consecutive samples of an element row.
template <class T, int NOUT>
__device__ __forceinline__ void slice_load(const MmArgs<T>& args, long long n, long long s0, int count, int q,
                                           T (&staged)[NOUT * 2 * kSlotRows * Shape<T, NOUT>::kTile /
                                                       Shape<T, NOUT>::kThreads]) {
    constexpr int kTile = Shape<T, NOUT>::kTile;
    constexpr int kRowStep = Shape<T, NOUT>::kThreads / kTile;
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
        const T* plane = args.in[side ? pr.rhs : pr.lhs];
        const int e = side ? rhs_elem(l, q, pr.rhs_t) : lhs_elem(l, q, pr.lhs_t);
        staged[r] = live ? __builtin_nontemporal_load(plane + static_cast<long long>(e) * n + s0 + s_own) : T(0);
    }
}

// One workgroup per tile: four K slices (the next slice's loads in flight
// during the current slice's MFMAs), then each output through LDS, half at a
// time, and out as contiguous element rows.  The grid is 8 * ceil(tiles / 8)
// workgroups; workgroup i takes tile (i % 8) * ceil(tiles / 8) + i / 8, and
// one past the last tile returns.
template <class T, int NOUT>
__device__ __forceinline__ void mm16_tiles(const MmArgs<T>& args, long long n, long long tiles) {
    constexpr int kTile = Shape<T, NOUT>::kTile;
    constexpr int kStride = kTile + 1;
    constexpr int kWaves = Shape<T, NOUT>::kThreads / 64;
    constexpr int kRowStep = Shape<T, NOUT>::kThreads / kTile;
    typedef typename Mfma<T>::acc Acc;
    __shared__ T lds[lds_elems<T, NOUT>()];
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

    Acc acc[NOUT][kTile / kWaves];
#pragma unroll
    for (int o = 0; o < NOUT; ++o)
#pragma unroll
        for (int m = 0; m < kTile / kWaves; ++m) acc[o][m] = Acc{T(0), T(0), T(0), T(0)};

    T staged[rows];
    slice_load<T, NOUT>(args, n, s0, count, 0, staged);
#pragma unroll
    for (int q = 0; q < kSlices; ++q) {
        if (q > 0) __syncthreads();                     // the previous slice's operands are read
#pragma unroll
        for (int r = 0; r < rows; ++r) lds[(e_own + r * kRowStep) * kStride + s_own] = staged[r];
        __syncthreads();
        if (q + 1 < kSlices) slice_load<T, NOUT>(args, n, s0, count, q + 1, staged);
#pragma unroll
        for (int o = 0; o < NOUT; ++o) {
            const T* L = lds + (o * 2) * kSlotRows * kStride;
            const T* R = L + kSlotRows * kStride;
#pragma unroll
            for (int m = 0; m < kTile / kWaves; ++m) {
                const int s = wave + m * kWaves;
                acc[o][m] = Mfma<T>::step(L[lane * kStride + s], R[lane * kStride + s], acc[o][m]);
            }
        }
    }

    // Half h of an output is its rows 8h .. 8h+7 (128 elements): fp32 keeps
    // them in lanes 32h .. 32h+31, fp64 in registers 2h and 2h+1 of every lane.
#pragma unroll
    for (int o = 0; o < NOUT; ++o) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            __syncthreads();                            // the LDS is free for this half
#pragma unroll
            for (int m = 0; m < kTile / kWaves; ++m) {
                const int s = wave + m * kWaves;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int row = Mfma<T>::row(lane, v);
                    if ((row >> 3) == h) lds[((row - 8 * h) * kDim + (lane & 15)) * kStride + s] = acc[o][m][v];
                }
            }
            __syncthreads();
            if (s_own < count) {
                T* dst = args.out[o] + s0 + s_own;
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

template <int NOUT>
__global__ __launch_bounds__((Shape<float, NOUT>::kThreads))
void hawk_mm16_f32(MmArgs<float> args, long long n, long long tiles) {
    mm16_tiles<float, NOUT>(args, n, tiles);
}

template <int NOUT>
__global__ __launch_bounds__((Shape<double, NOUT>::kThreads))
void hawk_mm16_f64(MmArgs<double> args, long long n, long long tiles) {
    mm16_tiles<double, NOUT>(args, n, tiles);
}

// Two products that read one plane between them (the VJP: bar_A = bar_C B^T
// and bar_B = A^T bar_C both read bar_C) on 128-byte tiles (fp32: 32 samples
// on 512 threads; fp64: 16 on 256): the shared plane's whole tile (256
// element rows) is staged in LDS once, and each K slice stages only the other
// operand of each product, so every input element is read from HBM once.
// LDS: the shared tile (33-35 KB, later the output halves) and one slice of
// the two other operands (17 KB).
template <class T> struct ShShape {
    static constexpr int kTile = 128 / static_cast<int>(sizeof(T));
    static constexpr int kThreads = 16 * kTile, kStride = kTile + 1, kRowStep = 16, kWaves = kThreads / 64;
};
constexpr int kShFullRows = kElems / 16;          // 16 shared-tile rows per thread
constexpr int kShSliceRows = 2 * kSlotRows / 16;  // 8 slice rows per thread

// Slice q of the non-shared operands: slot row o*64 + l holds the element lane
// l of the MFMA reads from product o's other side.
template <class T>
__device__ __forceinline__ void shared_slice_load(const MmArgs<T>& args, long long n, long long s0, int count, int q,
                                                  T (&staged)[kShSliceRows]) {
    typedef ShShape<T> Sh;
    const int s_own = threadIdx.x % Sh::kTile;
    const int e_own = threadIdx.x / Sh::kTile;
    const bool live = s_own < count;
    constexpr int kRowsPerGroup = kSlotRows / Sh::kRowStep;
#pragma unroll
    for (int r = 0; r < kShSliceRows; ++r) {
        const int o = r / kRowsPerGroup;
        const int l = e_own + (r % kRowsPerGroup) * Sh::kRowStep;
        const Product& pr = args.prod[o];
        const bool other_rhs = args.shared_side[o] == 0;
        const T* plane = args.in[other_rhs ? pr.rhs : pr.lhs];
        const int e = other_rhs ? rhs_elem(l, q, pr.rhs_t) : lhs_elem(l, q, pr.lhs_t);
        staged[r] = live ? __builtin_nontemporal_load(plane + static_cast<long long>(e) * n + s0 + s_own) : T(0);
    }
}

template <class T>
__device__ __forceinline__ void mm16_shared_tiles(const MmArgs<T>& args, long long n, long long tiles) {
    typedef ShShape<T> Sh;
    typedef typename Mfma<T>::acc Acc;
    __shared__ T full[kElems * Sh::kStride];
    __shared__ T slot[2 * kSlotRows * Sh::kStride];
    const int t = threadIdx.x;
    const int wave = t >> 6;
    const int lane = t & 63;
    const int s_own = t % Sh::kTile;
    const int e_own = t / Sh::kTile;
    const long long per_xcd = (tiles + 7) / 8;
    const long long tile = static_cast<long long>(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (tile >= tiles) return;
    const long long s0 = tile * Sh::kTile;
    const int count = n - s0 < Sh::kTile ? static_cast<int>(n - s0) : Sh::kTile;
    const bool live = s_own < count;

    const T* S = args.in[args.shared];
    T whole[kShFullRows];
#pragma unroll
    for (int r = 0; r < kShFullRows; ++r)
        whole[r] = live ? __builtin_nontemporal_load(S + static_cast<long long>(e_own + r * Sh::kRowStep) * n + s0 + s_own)
                        : T(0);
    T staged[kShSliceRows];
    shared_slice_load<T>(args, n, s0, count, 0, staged);
#pragma unroll
    for (int r = 0; r < kShFullRows; ++r) full[(e_own + r * Sh::kRowStep) * Sh::kStride + s_own] = whole[r];

    Acc acc[2][Sh::kTile / Sh::kWaves];
#pragma unroll
    for (int o = 0; o < 2; ++o)
#pragma unroll
        for (int m = 0; m < Sh::kTile / Sh::kWaves; ++m) acc[o][m] = Acc{T(0), T(0), T(0), T(0)};
#pragma unroll
    for (int q = 0; q < kSlices; ++q) {
        if (q > 0) __syncthreads();                     // the previous slice's operands are read
#pragma unroll
        for (int r = 0; r < kShSliceRows; ++r) slot[(e_own + r * Sh::kRowStep) * Sh::kStride + s_own] = staged[r];
        __syncthreads();
        if (q + 1 < kSlices) shared_slice_load<T>(args, n, s0, count, q + 1, staged);
#pragma unroll
        for (int o = 0; o < 2; ++o) {
            const Product& pr = args.prod[o];
            const bool lhs_shared = args.shared_side[o] == 0;
            const int e = lhs_shared ? lhs_elem(lane, q, pr.lhs_t) : rhs_elem(lane, q, pr.rhs_t);
            const T* F = full + e * Sh::kStride;
            const T* O = slot + (o * kSlotRows + lane) * Sh::kStride;
#pragma unroll
            for (int m = 0; m < Sh::kTile / Sh::kWaves; ++m) {
                const int sm = wave + m * Sh::kWaves;
                const T fv = F[sm], ov = O[sm];
                acc[o][m] = Mfma<T>::step(lhs_shared ? fv : ov, lhs_shared ? ov : fv, acc[o][m]);
            }
        }
    }

    // As mm16_tiles: each output through LDS (the shared tile's memory), half
    // at a time, and out as contiguous element rows.
#pragma unroll
    for (int o = 0; o < 2; ++o) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            __syncthreads();
#pragma unroll
            for (int m = 0; m < Sh::kTile / Sh::kWaves; ++m) {
                const int sm = wave + m * Sh::kWaves;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int row = Mfma<T>::row(lane, v);
                    if ((row >> 3) == h) full[((row - 8 * h) * kDim + (lane & 15)) * Sh::kStride + sm] = acc[o][m][v];
                }
            }
            __syncthreads();
            if (live) {
                T* dst = args.out[o] + s0 + s_own;
#pragma unroll
                for (int r = 0; r < kHalfRows / Sh::kRowStep; ++r) {
                    const int e = e_own + r * Sh::kRowStep;
                    __builtin_nontemporal_store(full[e * Sh::kStride + s_own],
                                                dst + static_cast<long long>(e + h * kHalfRows) * n);
                }
            }
        }
    }
}

__global__ __launch_bounds__(ShShape<float>::kThreads)
void hawk_mm16_f32_shared(MmArgs<float> args, long long n, long long tiles) {
    mm16_shared_tiles<float>(args, n, tiles);
}

__global__ __launch_bounds__(ShShape<double>::kThreads)
void hawk_mm16_f64_shared(MmArgs<double> args, long long n, long long tiles) {
    mm16_shared_tiles<double>(args, n, tiles);
}

int launch_error(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hawk_internal::set_hip_error(what, e);
    return HK_OK;
}

// The products' launch for either element type; NAME prefixes every error.
template <class T>
int mm16_launch(const char* name, const T* const* in, int n_in, T* const* out, int n_out, const int32_t* products,
                int64_t n, hipStream_t stream) {
    const std::string who(name);
    if (n_in < 1 || n_in > kMaxIn || n_out < 1 || n_out > kMaxOut || n_out > n_in)
        return hawk_internal::set_error(HK_EVALUE,
                                        who + ": 1..3 input planes and 1..2 products, no more products than inputs");
    if (n < 0) return hawk_internal::set_error(HK_EVALUE, who + ": n must be >= 0");
    if (!in || !out || !products)
        return hawk_internal::set_error(HK_EVALUE, who + ": in, out and products are required");
    MmArgs<T> args{};
    args.n_in = n_in;
    args.n_out = n_out;
    for (int p = 0; p < n_in; ++p) {
        if (!in[p]) return hawk_internal::set_error(HK_EVALUE, who + ": input plane " + std::to_string(p) + " is null");
        args.in[p] = in[p];
    }
    for (int o = 0; o < n_out; ++o) {
        const int32_t* d = products + 3 * o;
        const Product pr{d[0], d[2] & 1, d[1], (d[2] >> 1) & 1, o};
        if (pr.lhs < 0 || pr.lhs >= n_in || pr.rhs < 0 || pr.rhs >= n_in)
            return hawk_internal::set_error(HK_EINDEX, who + ": product " + std::to_string(o) +
                                                           " names an input plane outside [0, n_in)");
        if (!out[o]) return hawk_internal::set_error(HK_EVALUE, who + ": output plane " + std::to_string(o) + " is null");
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
    constexpr bool f64 = sizeof(T) == 8;
    if (args.shared >= 0) {
        const long long tiles = (n + ShShape<T>::kTile - 1) / ShShape<T>::kTile;
        const long long grid = 8 * ((tiles + 7) / 8);
        if (grid > 0x7fffffffLL) return hawk_internal::set_error(HK_EVALUE, who + ": too many samples");
        const dim3 g(static_cast<unsigned>(grid)), b(ShShape<T>::kThreads);
        if constexpr (f64)
            hipLaunchKernelGGL(hawk_mm16_f64_shared, g, b, 0, stream, args, static_cast<long long>(n), tiles);
        else
            hipLaunchKernelGGL(hawk_mm16_f32_shared, g, b, 0, stream, args, static_cast<long long>(n), tiles);
        return launch_error(f64 ? "hawk_mm16_f64_shared launch" : "hawk_mm16_f32_shared launch");
    }
    const int tile = n_out == 1 ? Shape<T, 1>::kTile : Shape<T, 2>::kTile;
    const long long tiles = (n + tile - 1) / tile;
    const long long grid = 8 * ((tiles + 7) / 8);     // every tile gets a workgroup on its XCD
    if (grid > 0x7fffffffLL) return hawk_internal::set_error(HK_EVALUE, who + ": too many samples");
    const dim3 g(static_cast<unsigned>(grid));
    if constexpr (f64) {
        if (n_out == 1)
            hipLaunchKernelGGL(hawk_mm16_f64<1>, g, dim3(Shape<T, 1>::kThreads), 0, stream, args,
                               static_cast<long long>(n), tiles);
        else
            hipLaunchKernelGGL(hawk_mm16_f64<2>, g, dim3(Shape<T, 2>::kThreads), 0, stream, args,
                               static_cast<long long>(n), tiles);
    } else {
        if (n_out == 1)
            hipLaunchKernelGGL(hawk_mm16_f32<1>, g, dim3(Shape<T, 1>::kThreads), 0, stream, args,
                               static_cast<long long>(n), tiles);
        else
            hipLaunchKernelGGL(hawk_mm16_f32<2>, g, dim3(Shape<T, 2>::kThreads), 0, stream, args,
                               static_cast<long long>(n), tiles);
    }
    return launch_error(f64 ? "hawk_mm16_f64 launch" : "hawk_mm16_f32 launch");
}

}  // namespace

extern "C" {

int hk_mm16_f32(const float* const* in, int n_in, float* const* out, int n_out, const int32_t* products,
                int64_t n, void* stream) {
    return mm16_launch<float>("hk_mm16_f32", in, n_in, out, n_out, products, n, static_cast<hipStream_t>(stream));
}

int hk_mm16_f64(const double* const* in, int n_in, double* const* out, int n_out, const int32_t* products,
                int64_t n, void* stream) {
    return mm16_launch<double>("hk_mm16_f64", in, n_in, out, n_out, products, n, static_cast<hipStream_t>(stream));
}

}  // extern "C"
