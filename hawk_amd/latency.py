"""gfx950 latencies the team stages are designed around, measured on one CU.

``python -m hawk_amd.latency`` builds one probe kernel through the package's
hipRTC path (:func:`hawk_amd.compile.compile_source`), launches it as a single
workgroup through ``hk_launch_grid`` and prints one JSON object: shader-clock
cycles (``clock64``) per operation for

* ``add_chain_registers``: a dependent fp64 add whose operand is a register;
* ``add_chain_lds_alone``: the same chain with its operands read from LDS,
  eight reads ahead, by one wave on an otherwise idle CU;
* ``add_chain_lds_loaded``: that chain while fifteen other waves of the
  workgroup read LDS without pause;
* ``add_chain_lds_deep_alone`` / ``_loaded``: the same two with 24 values
  read ahead (four rotating blocks of eight);
* ``add_chain_readlane`` / ``add_chain_dpp``: operands taken from the other
  lanes of one register by ``readlane`` or by a DPP ``wave_shl`` rotation;
* ``lds_round_trip`` / ``lds_round_trip_loaded``: dependent LDS reads (each
  address the previous read's value) by one wave, alone or while fifteen
  other waves read LDS;
* ``ds_or_same_address``: a 64-bit ``ds_or`` by all 64 lanes into one slot,
  per instruction.

These bound the ordered scatter's split walk: a key's additions are one
dependent chain per chunk, fed from LDS while the rest of the workgroup uses
it.  Only the probe kernel's own buffers are touched (4096 doubles in, two
doubles a wave out).
"""

from __future__ import annotations

import json

_SOURCE = r"""
struct GRefMirror { void* data_; unsigned long long samples_, compStride_, sampleStride_; int deviceType_, deviceId_; };
extern "C" __attribute__((used)) __device__ char eagle_abi_tag[] = "aether-abi/2";
extern "C" __attribute__((used)) __device__ unsigned long long eagle_layout_sizes[5] = {40, 32, 32, 8, 24};

__device__ __forceinline__ double lane_shl(double x) {
    const long long b = __double_as_longlong(x);
    const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(b), 0x130, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(b >> 32), 0x130, 0xf, 0xf, false);
    return __longlong_as_double((static_cast<long long>(hi) << 32) | static_cast<unsigned>(lo));
}

// src: 4096 doubles; out: two doubles a wave (cycles, a value that keeps the
// work alive).  Wave 0 runs the probe; in mode 2 the other waves read LDS.
extern "C" __global__ void __launch_bounds__(1024) hawk_latency(
        GRefMirror src_m, GRefMirror out_m, long long mode, long long reps,
        long long base, long long count, long long nSamples) {
    (void)count; (void)nSamples;
    const double* src = static_cast<const double*>(src_m.data_);
    double* out = static_cast<double*>(out_m.data_);
    __shared__ double buf[4096 + 64];               // 64 zeros past the end for the deep feed's last loads
    __shared__ int next[4096];
    __shared__ unsigned long long tab[64];
    __shared__ volatile int done;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    for (int i = t; i < 4096; i += blockDim.x) {
        buf[i] = src[i];
        next[i] = (i * 1021 + 7) & 4095;          // 1021 is odd: a permutation of [0, 4096)
    }
    if (t < 64) buf[4096 + t] = 0.0;
    if (t < 64) tab[t] = 0;
    if (t == 0) done = 0;
    __syncthreads();
    double a = 0.0;
    long long c0 = clock64();
    if (wave != 0) {
        if (mode == 2 || mode == 7 || mode == 9) {  // loaders: LDS reads until wave 0's probe ends
            // (bounded as well: at most 4096 * reps rounds, more than the chain takes)
            for (long long r = 0; r < reps * 4096 && !done; ++r)
#pragma unroll
                for (int q = 0; q < 8; ++q) a += buf[(static_cast<int>(r) * 512 + q * 64 + lane) & 4095];
        }
    } else if (mode == 0) {
        const double x = buf[lane];
        for (long long r = 0; r < reps; ++r)
#pragma unroll
            for (int q = 0; q < 64; ++q) a = a + x;
    } else if (mode == 1 || mode == 2) {
        for (long long r = 0; r < reps; ++r) {
            double cur[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) cur[q] = buf[q];
            for (int m = 8; m < 4096; m += 8) {
                double nxt[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) nxt[q] = buf[m + q];
#pragma unroll
                for (int q = 0; q < 8; ++q) a = a + cur[q];
#pragma unroll
                for (int q = 0; q < 8; ++q) cur[q] = nxt[q];
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) a = a + cur[q];
        }
    } else if (mode == 8 || mode == 9) {
        // four rotating blocks of 8: three blocks (24 values) in flight while one is added
        for (long long r = 0; r < reps; ++r) {
            double b0[8], b1[8], b2[8], b3[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) { b0[q] = buf[q]; b1[q] = buf[8 + q]; b2[q] = buf[16 + q]; }
            for (int m = 24; m < 4096 + 24; m += 32) {
#pragma unroll
                for (int q = 0; q < 8; ++q) b3[q] = buf[m + q];
#pragma unroll
                for (int q = 0; q < 8; ++q) a = a + b0[q];
#pragma unroll
                for (int q = 0; q < 8; ++q) b0[q] = buf[m + 8 + q];
#pragma unroll
                for (int q = 0; q < 8; ++q) a = a + b1[q];
#pragma unroll
                for (int q = 0; q < 8; ++q) b1[q] = buf[m + 16 + q];
#pragma unroll
                for (int q = 0; q < 8; ++q) a = a + b2[q];
#pragma unroll
                for (int q = 0; q < 8; ++q) b2[q] = buf[m + 24 + q];
#pragma unroll
                for (int q = 0; q < 8; ++q) a = a + b3[q];
            }
        }
    } else if (mode == 3) {
        for (long long r = 0; r < reps; ++r) {
            const double x = buf[(static_cast<int>(r) * 64 + lane) & 4095];
            const long long b = __double_as_longlong(x);
#pragma unroll
            for (int q = 0; q < 64; ++q) {
                const int lo = __builtin_amdgcn_readlane(static_cast<int>(b), q);
                const int hi = __builtin_amdgcn_readlane(static_cast<int>(b >> 32), q);
                a = a + __longlong_as_double((static_cast<long long>(hi) << 32) | static_cast<unsigned>(lo));
            }
        }
    } else if (mode == 4) {
        for (long long r = 0; r < reps; ++r) {
            double x = buf[(static_cast<int>(r) * 64 + lane) & 4095];
#pragma unroll
            for (int q = 0; q < 64; ++q) { a = a + x; x = lane_shl(x); }
        }
    } else if (mode == 5 || mode == 7) {
        int j = lane & 0;
        for (long long r = 0; r < reps * 64; ++r) j = next[j];
        a = j;
    } else if (mode == 6) {
        // every lane's slot is lane * base = 0 (base is 0 at run time, which
        // the compiler cannot see, so it keeps one ds_or per lane)
        unsigned long long* slot = &tab[(lane * static_cast<int>(base)) & 63];
        for (long long r = 0; r < reps; ++r) {
            atomicOr(slot, 1ull << lane);
            __builtin_amdgcn_wave_barrier();
        }
        a = static_cast<double>(tab[0]);
    }
    const long long c1 = clock64();
    if (wave == 0 && lane == 0) done = 1;
    if (lane == 0) {
        out[2 * wave] = static_cast<double>(c1 - c0);
        out[2 * wave + 1] = a;
    }
}
"""

#: mode -> (name, waves, operations per repetition)
PROBES = {
    0: ("add_chain_registers", 1, 64),
    1: ("add_chain_lds_alone", 1, 4096),
    2: ("add_chain_lds_loaded", 16, 4096),
    3: ("add_chain_readlane", 1, 64),
    4: ("add_chain_dpp", 1, 64),
    5: ("lds_round_trip", 1, 64),
    6: ("ds_or_same_address", 1, 1),
    7: ("lds_round_trip_loaded", 16, 64),
    8: ("add_chain_lds_deep_alone", 1, 4096),
    9: ("add_chain_lds_deep_loaded", 16, 4096),
}


def measure(device=None, reps: int = 64) -> dict:
    """Cycles per operation of every probe (median of five launches each)."""
    import statistics

    import torch

    from . import _core
    from .compile import compile_source

    device = torch.device("cuda:0") if device is None else device
    code, _key, _hit = compile_source(_SOURCE, "hawk_latency")
    entry = _core.DeviceLibrary(code).entry("hawk_latency")
    src = torch.arange(4096, dtype=torch.float64, device=device) * 1e-3
    out = torch.zeros(32, dtype=torch.float64, device=device)
    stream = torch.cuda.current_stream()
    result = {}
    for mode, (name, waves, per_rep) in PROBES.items():
        ab = _core.ArgBlock(["gref", "gref", "int", "int"])
        ab.bind(0, src.data_ptr(), 4096)
        ab.bind(1, out.data_ptr(), 32)
        ab.bind_value(2, mode)
        ab.bind_value(3, reps)
        cycles = []
        for _ in range(6):
            entry.run_grid(ab, 0, 1, 1, 1, 64 * waves, stream.cuda_stream)
            stream.synchronize()
            cycles.append(float(out[0].item()))
        result[name] = round(statistics.median(cycles[1:]) / (reps * per_rep), 2)
    return result


def main() -> int:
    import torch
    print(json.dumps({"device": torch.cuda.get_device_name(0), "cycles_per_op": measure()}), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
