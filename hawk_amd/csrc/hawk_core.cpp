// hawk_core.cpp — the C-ABI launcher of hawk's gfx950 device target.
//
// What the reference keeps in its nanobind module `hawk._core`
// (reference src/hawk_core.cpp) — the load-time ABI self-check, the
// contiguous block of by-value mirror PODs, the bulk rebind and the one
// launch crossing — lives here as plain `extern "C"` functions that
// hawk_amd/_core.py binds with ctypes.  Three things differ by design:
//
//  * an artifact is a gfx950 code object loaded with hipModuleLoadData, not
//    a dlopen'ed host .so, and the self-check reads its exported
//    `eagle_abi_tag` / `eagle_layout_sizes` device globals;
//  * a launch is hipModuleLaunchKernel over a grid this library chooses
//    (block x per-thread samples), on the caller's HIP stream, with the
//    argument block's cells as the kernel parameters — the cell addresses
//    ARE the `void**` kernelParams array, so binding costs nothing per launch;
//  * the compiler is hipRTC pinned to gfx950 (hk_rtc_compile).
//
// The team-stage kernels (ordered sum, ordered scatter) are in hawk_team.hip.

#include "hawk_core.h"
#include "hawk_internal.h"

#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <atomic>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#ifndef HAWK_BUILD_DIGEST
#define HAWK_BUILD_DIGEST "unstamped"
#endif
#ifndef HAWK_BUILD_INFO
#define HAWK_BUILD_INFO "compiler=unknown"
#endif

namespace {

std::atomic<std::uint64_t> g_crossings{0};
thread_local std::string g_error;

inline void cross() { g_crossings.fetch_add(1, std::memory_order_relaxed); }

// The by-value mirror PODs an emitted entry takes, one per arg_spec slot.
// Layouts follow reference tests/stale_stack_harness.cpp:14-15 and the sizes
// pinned at reference hawk/_contracts.py:66-92.
struct GRefMirror {
    double* data_;
    std::uint64_t samples_, compStride_, sampleStride_;
    std::int32_t deviceType_, deviceId_;
};
struct ScalarHandle {
    void* data;
    std::uint64_t samples, stride;
    std::int32_t deviceType, deviceId;
};
using IntHandle = ScalarHandle;
struct PartitionTriple {
    std::int64_t base, count, nSamples;
};
using index_t = std::uint64_t;   // the nsamples role: 64-bit on a 288 GB device

static_assert(sizeof(GRefMirror) == 40, "GRefMirror is 40 bytes");
static_assert(sizeof(ScalarHandle) == 32, "ScalarHandle is 32 bytes");
static_assert(sizeof(PartitionTriple) == 24, "PartitionTriple is 24 bytes");

const std::uint64_t kLayout[HK_LAYOUT_FIELDS] = {
    sizeof(GRefMirror), sizeof(ScalarHandle), sizeof(IntHandle),
    sizeof(index_t), sizeof(PartitionTriple)};
const char* const kLayoutNames[HK_LAYOUT_FIELDS] = {
    "GRefMirror", "ScalarHandle", "IntHandle", "index_t", "PartitionTriple"};

enum class Kind { GRef, Handle, IntHandle, F64, F32, Int, NSamples };

bool kind_from_name(const char* name, Kind* out) {
    static const struct { const char* n; Kind k; } table[] = {
        {"gref", Kind::GRef},     {"handle", Kind::Handle},
        {"int_handle", Kind::IntHandle}, {"f64", Kind::F64},
        {"f32", Kind::F32},       {"int", Kind::Int},
        {"nsamples", Kind::NSamples}};
    for (const auto& row : table)
        if (name && std::strcmp(name, row.n) == 0) { *out = row.k; return true; }
    return false;
}

const char* kind_name(Kind k) {
    switch (k) {
        case Kind::GRef: return "gref";
        case Kind::Handle: return "handle";
        case Kind::IntHandle: return "int_handle";
        case Kind::F64: return "f64";
        case Kind::F32: return "f32";
        case Kind::Int: return "int";
        case Kind::NSamples: return "nsamples";
    }
    return "<unknown>";
}

int fail(int code, std::string text) {
    g_error = std::move(text);
    return code;
}

int hip_fail(const char* what, hipError_t err) {
    return fail(HK_EHIP, std::string("hawk_core: ") + what + " failed: " +
                             hipGetErrorName(err) + " (" + hipGetErrorString(err) + ")");
}

}  // namespace

// The argument block: one 40-byte, 8-aligned cell per slot, allocated once and
// never resized, plus three trailing cells for the partition triple, so
// `params` is directly the kernelParams array of a launch.
struct hk_argblock {
    struct Cell {
        alignas(8) unsigned char bytes[sizeof(GRefMirror)];
        Kind kind;
    };
    std::vector<Cell> cells;
    std::vector<void*> params;   // cells..., &base, &count, &nSamples
    std::int64_t triple[3] = {0, 0, 0};
};

struct hk_library {
    hipModule_t module = nullptr;
};

struct hk_entry {
    hipFunction_t fn = nullptr;
    std::string name;
};

// Error helpers shared with hawk_team.hip.
namespace hawk_internal {
int set_error(int code, const std::string& text) { return fail(code, text); }
int set_hip_error(const char* what, hipError_t err) { return hip_fail(what, err); }
}  // namespace hawk_internal

extern "C" {

const char* hk_last_error(void) { return g_error.c_str(); }

int hk_layout_sizes(uint64_t out[HK_LAYOUT_FIELDS]) {
    cross();
    if (!out) return fail(HK_EVALUE, "hk_layout_sizes: out is NULL");
    for (int i = 0; i < HK_LAYOUT_FIELDS; ++i) out[i] = kLayout[i];
    return HK_OK;
}

const char* hk_layout_field_name(int i) {
    cross();
    return (i >= 0 && i < HK_LAYOUT_FIELDS) ? kLayoutNames[i] : "<absent>";
}

const char* hk_build_digest(void) {
    cross();
    return HAWK_BUILD_DIGEST;
}

const char* hk_build_info(void) {
    cross();
    static const std::string info =
        std::string(HAWK_BUILD_INFO) + "\nabi_tag=" HK_ABI_TAG +
        "\nindex_type_bytes=" + std::to_string(sizeof(index_t)) +
        "\nbuild_digest=" HAWK_BUILD_DIGEST;
    return info.c_str();
}

uint64_t hk_crossings(void) {
    cross();
    return g_crossings.load(std::memory_order_relaxed);
}

void hk_free(void* p) { std::free(p); }

int hk_rtc_version(void) {
    cross();
    int major = 0, minor = 0;
    if (hiprtcVersion(&major, &minor) != HIPRTC_SUCCESS) return -1;
    return major * 100 + minor;
}

int hk_rtc_compile(const char* source, const char* name,
                   const char* const* options, int n_options,
                   void** code, size_t* code_size, char** log) {
    cross();
    if (code) *code = nullptr;
    if (code_size) *code_size = 0;
    if (log) *log = nullptr;
    if (!source || !name || !code || !code_size)
        return fail(HK_EVALUE, "hk_rtc_compile: source, name, code and code_size are required");
    if (n_options < 0 || (n_options > 0 && !options))
        return fail(HK_EVALUE, "hk_rtc_compile: options is NULL with n_options > 0");
    std::vector<const char*> opts;
    opts.push_back("--offload-arch=gfx950");
    for (int i = 0; i < n_options; ++i) {
        if (!options[i]) return fail(HK_EVALUE, "hk_rtc_compile: option " + std::to_string(i) + " is NULL");
        if (std::strncmp(options[i], "--offload-arch", 14) == 0 ||
            std::strncmp(options[i], "--gpu-architecture", 18) == 0)
            return fail(HK_EVALUE, std::string("hk_rtc_compile: the target is pinned to gfx950; "
                                               "refusing option '") + options[i] + "'");
        opts.push_back(options[i]);
    }
    hiprtcProgram prog = nullptr;
    hiprtcResult r = hiprtcCreateProgram(&prog, source, name, 0, nullptr, nullptr);
    if (r != HIPRTC_SUCCESS)
        return fail(HK_EHIP, std::string("hiprtcCreateProgram: ") + hiprtcGetErrorString(r));
    const hiprtcResult compiled = hiprtcCompileProgram(prog, static_cast<int>(opts.size()), opts.data());
    size_t log_size = 0;
    std::string text;
    if (hiprtcGetProgramLogSize(prog, &log_size) == HIPRTC_SUCCESS && log_size > 1) {
        text.resize(log_size);
        hiprtcGetProgramLog(prog, &text[0]);
        text.resize(std::strlen(text.c_str()));
    }
    if (log) {
        *log = static_cast<char*>(std::malloc(text.size() + 1));
        if (*log) std::memcpy(*log, text.c_str(), text.size() + 1);
    }
    if (compiled != HIPRTC_SUCCESS) {
        hiprtcDestroyProgram(&prog);
        return fail(HK_EHIP, std::string("hipRTC could not compile '") + name + "' for gfx950: " +
                                 hiprtcGetErrorString(compiled) + "\n" + text);
    }
    size_t size = 0;
    r = hiprtcGetCodeSize(prog, &size);
    if (r != HIPRTC_SUCCESS || size == 0) {
        hiprtcDestroyProgram(&prog);
        return fail(HK_EHIP, std::string("hiprtcGetCodeSize: ") + hiprtcGetErrorString(r));
    }
    void* buf = std::malloc(size);
    if (!buf) {
        hiprtcDestroyProgram(&prog);
        return fail(HK_EVALUE, "hk_rtc_compile: out of host memory");
    }
    r = hiprtcGetCode(prog, static_cast<char*>(buf));
    hiprtcDestroyProgram(&prog);
    if (r != HIPRTC_SUCCESS) {
        std::free(buf);
        return fail(HK_EHIP, std::string("hiprtcGetCode: ") + hiprtcGetErrorString(r));
    }
    *code = buf;
    *code_size = size;
    return HK_OK;
}

int hk_load(const void* code, size_t code_size, hk_library** out) {
    cross();
    if (out) *out = nullptr;
    if (!code || code_size == 0 || !out)
        return fail(HK_EVALUE, "hk_load: an empty code object cannot be loaded");
    auto* lib = new (std::nothrow) hk_library();
    if (!lib) return fail(HK_EVALUE, "hk_load: out of host memory");
    hipError_t e = hipModuleLoadData(&lib->module, code);
    if (e != hipSuccess) {
        delete lib;
        return hip_fail("hipModuleLoadData", e);
    }
    // The tag first, then the layout: the order reference
    // src/hawk_core.cpp:366-390 checks them in.
    hipDeviceptr_t dptr = nullptr;
    size_t bytes = 0;
    e = hipModuleGetGlobal(&dptr, &bytes, lib->module, "eagle_abi_tag");
    if (e != hipSuccess) {
        hipModuleUnload(lib->module);
        delete lib;
        return fail(HK_EVALUE, "hawk_core: the code object exports no 'eagle_abi_tag'; "
                               "it was not emitted by hawk's hip target");
    }
    std::vector<char> tag(bytes + 1, 0);
    e = hipMemcpyDtoH(tag.data(), dptr, bytes);
    if (e != hipSuccess) {
        hipModuleUnload(lib->module);
        delete lib;
        return hip_fail("hipMemcpyDtoH(eagle_abi_tag)", e);
    }
    if (std::strcmp(tag.data(), HK_ABI_TAG) != 0) {
        hipModuleUnload(lib->module);
        delete lib;
        return fail(HK_EVALUE, std::string("hawk_core: exported eagle_abi_tag is '") + tag.data() +
                                   "', this build speaks '" HK_ABI_TAG "'");
    }
    e = hipModuleGetGlobal(&dptr, &bytes, lib->module, "eagle_layout_sizes");
    std::uint64_t sizes[HK_LAYOUT_FIELDS] = {0};
    if (e == hipSuccess && bytes == sizeof(sizes)) e = hipMemcpyDtoH(sizes, dptr, bytes);
    if (e != hipSuccess || bytes != sizeof(sizes)) {
        hipModuleUnload(lib->module);
        delete lib;
        return fail(HK_EVALUE, "hawk_core: the code object exports no 5-field 'eagle_layout_sizes'");
    }
    for (int i = 0; i < HK_LAYOUT_FIELDS; ++i) {
        if (sizes[i] != kLayout[i]) {
            hipModuleUnload(lib->module);
            delete lib;
            return fail(HK_EVALUE, std::string("hawk_core: the code object's layout disagrees in sizeof(") +
                                       kLayoutNames[i] + "): it was built with " + std::to_string(sizes[i]) +
                                       " bytes, this library marshals " + std::to_string(kLayout[i]));
        }
    }
    *out = lib;
    return HK_OK;
}

void hk_unload(hk_library* lib) {
    cross();
    if (!lib) return;
    if (lib->module) hipModuleUnload(lib->module);
    delete lib;
}

int hk_entry_get(hk_library* lib, const char* name, hk_entry** out) {
    cross();
    if (out) *out = nullptr;
    if (!lib || !name || !out) return fail(HK_EVALUE, "hk_entry_get: library, name and out are required");
    hipFunction_t fn = nullptr;
    hipError_t e = hipModuleGetFunction(&fn, lib->module, name);
    if (e != hipSuccess)
        return fail(HK_EVALUE, std::string("hawk_core: the code object exports no entry '") + name + "'");
    auto* entry = new (std::nothrow) hk_entry();
    if (!entry) return fail(HK_EVALUE, "hk_entry_get: out of host memory");
    entry->fn = fn;
    entry->name = name;
    *out = entry;
    return HK_OK;
}

int hk_argblock_new(const char* const* kinds, int n_slots, hk_argblock** out) {
    cross();
    if (out) *out = nullptr;
    if (!out || n_slots < 0 || (n_slots > 0 && !kinds))
        return fail(HK_EVALUE, "hk_argblock_new: kinds and out are required");
    auto* ab = new (std::nothrow) hk_argblock();
    if (!ab) return fail(HK_EVALUE, "hk_argblock_new: out of host memory");
    ab->cells.resize(static_cast<size_t>(n_slots));
    for (int k = 0; k < n_slots; ++k) {
        auto& cell = ab->cells[static_cast<size_t>(k)];
        if (!kind_from_name(kinds[k], &cell.kind)) {
            delete ab;
            return fail(HK_EVALUE, std::string("hawk_core.ArgBlock: unknown slot kind '") +
                                       (kinds[k] ? kinds[k] : "(null)") +
                                       "'; the descriptor vocabulary is 'gref' (40 B GRefMirror), "
                                       "'handle' / 'int_handle' (32 B), 'f64' / 'f32' / 'int' / "
                                       "'nsamples' (by value)");
        }
        std::memset(cell.bytes, 0, sizeof(cell.bytes));
        // A fresh mirror holds the POD's own defaults: a unit sample stride
        // and the ROCm device type, never a zero stride.
        if (cell.kind == Kind::GRef) {
            auto* m = reinterpret_cast<GRefMirror*>(cell.bytes);
            m->sampleStride_ = 1;
            m->deviceType_ = HK_DEVICE_ROCM;
        } else if (cell.kind == Kind::Handle || cell.kind == Kind::IntHandle) {
            auto* m = reinterpret_cast<ScalarHandle*>(cell.bytes);
            m->stride = 1;
            m->deviceType = HK_DEVICE_ROCM;
        }
    }
    ab->params.resize(static_cast<size_t>(n_slots) + 3);
    for (int k = 0; k < n_slots; ++k) ab->params[static_cast<size_t>(k)] = ab->cells[static_cast<size_t>(k)].bytes;
    for (int t = 0; t < 3; ++t) ab->params[static_cast<size_t>(n_slots + t)] = &ab->triple[t];
    *out = ab;
    return HK_OK;
}

void hk_argblock_free(hk_argblock* ab) {
    cross();
    delete ab;
}

int hk_argblock_size(const hk_argblock* ab) {
    cross();
    return ab ? static_cast<int>(ab->cells.size()) : 0;
}

int hk_bind(hk_argblock* ab, int slot, uint64_t ptr, uint64_t samples,
            uint64_t stride, int32_t device_type, int32_t device_id) {
    cross();
    if (!ab) return fail(HK_EVALUE, "hk_bind: argblock is NULL");
    if (slot < 0 || static_cast<size_t>(slot) >= ab->cells.size())
        return fail(HK_EINDEX, "hawk_core.ArgBlock: slot " + std::to_string(slot) +
                                   " is outside this block's " + std::to_string(ab->cells.size()) + " slots");
    auto& cell = ab->cells[static_cast<size_t>(slot)];
    switch (cell.kind) {
        case Kind::GRef: {
            if (stride != 1)
                return fail(HK_EVALUE, "hawk_core.ArgBlock.bind: slot " + std::to_string(slot) +
                                           " has sample stride " + std::to_string(stride) +
                                           "; the gfx950 entries read contiguous component-major planes "
                                           "(stride 1)");
            auto* m = reinterpret_cast<GRefMirror*>(cell.bytes);
            m->data_ = reinterpret_cast<double*>(static_cast<uintptr_t>(ptr));
            m->samples_ = samples;
            m->compStride_ = samples * stride;
            m->sampleStride_ = stride;
            m->deviceType_ = device_type;
            m->deviceId_ = device_id;
            return HK_OK;
        }
        case Kind::Handle:
        case Kind::IntHandle: {
            if (stride != 1)
                return fail(HK_EVALUE, "hawk_core.ArgBlock.bind: slot " + std::to_string(slot) +
                                           " has sample stride " + std::to_string(stride) +
                                           "; the gfx950 entries read contiguous planes (stride 1)");
            auto* m = reinterpret_cast<ScalarHandle*>(cell.bytes);
            m->data = reinterpret_cast<void*>(static_cast<uintptr_t>(ptr));
            m->samples = samples;
            m->stride = stride;
            m->deviceType = device_type;
            m->deviceId = device_id;
            return HK_OK;
        }
        default: {
            if (ptr == 0)
                return fail(HK_EVALUE, "hawk_core.ArgBlock.bind: slot " + std::to_string(slot) +
                                           " is a by-value slot and needs the ADDRESS of the value to "
                                           "copy, got a null pointer");
            const void* src = reinterpret_cast<const void*>(static_cast<uintptr_t>(ptr));
            size_t width = cell.kind == Kind::F32 ? sizeof(float)
                         : cell.kind == Kind::NSamples ? sizeof(index_t) : sizeof(double);
            std::memset(cell.bytes, 0, sizeof(cell.bytes));
            std::memcpy(cell.bytes, src, width);
            return HK_OK;
        }
    }
}

int hk_rebind(hk_argblock* ab, const int64_t* slots, const int64_t* ptrs, size_t n) {
    cross();
    if (!ab || (n > 0 && (!slots || !ptrs))) return fail(HK_EVALUE, "hk_rebind: argblock, slots and ptrs are required");
    for (size_t i = 0; i < n; ++i) {
        const int64_t s = slots[i];
        if (s < 0 || static_cast<size_t>(s) >= ab->cells.size())
            return fail(HK_EINDEX, "hawk_core.ArgBlock.rebind: slot " + std::to_string(s) +
                                       " is outside this block's " + std::to_string(ab->cells.size()) + " slots");
        auto& cell = ab->cells[static_cast<size_t>(s)];
        const auto ptr = static_cast<uintptr_t>(ptrs[i]);
        switch (cell.kind) {
            case Kind::GRef:
                reinterpret_cast<GRefMirror*>(cell.bytes)->data_ = reinterpret_cast<double*>(ptr);
                break;
            case Kind::Handle:
            case Kind::IntHandle:
                reinterpret_cast<ScalarHandle*>(cell.bytes)->data = reinterpret_cast<void*>(ptr);
                break;
            default:
                return fail(HK_EVALUE, "hawk_core.ArgBlock.rebind: slot " + std::to_string(s) +
                                           " is a by-value '" + kind_name(cell.kind) +
                                           "' slot and carries no pointer to rebind; set it with bind() "
                                           "(rebind is the bulk POINTER path)");
        }
    }
    return HK_OK;
}

// A launch writes the block's triple cells before handing the cells to HIP;
// one block is never launched from two threads at once (the caller's lock).
static int launch_impl(const hk_entry* entry, const hk_argblock* ab, int64_t base, int64_t count,
                       int64_t n_samples, uint32_t grid, uint32_t block, void* stream) {
    auto* block_args = const_cast<hk_argblock*>(ab);
    block_args->triple[0] = base;
    block_args->triple[1] = count;
    block_args->triple[2] = n_samples;
    hipError_t e = hipModuleLaunchKernel(entry->fn, grid, 1, 1, block, 1, 1, 0,
                                         static_cast<hipStream_t>(stream),
                                         block_args->params.data(), nullptr);
    if (e != hipSuccess) return hip_fail(("hipModuleLaunchKernel(" + entry->name + ")").c_str(), e);
    return HK_OK;
}

int hk_launch(const hk_entry* entry, const hk_argblock* ab, int64_t base,
              int64_t count, int64_t n_samples, uint32_t block,
              uint32_t per_thread, void* stream) {
    cross();
    if (!entry || !ab) return fail(HK_EVALUE, "hk_launch: entry and argblock are required");
    if (count <= 0) return HK_OK;   // an empty range launches nothing (reference src/hawk_core.cpp:439)
    if (base < 0 || n_samples < 0 || base + count > n_samples)
        return fail(HK_EVALUE, "hk_launch: the range [" + std::to_string(base) + ", " +
                                   std::to_string(base + count) + ") is not inside [0, " +
                                   std::to_string(n_samples) + ")");
    if (block == 0 || block > 1024 || block % 64 != 0)
        return fail(HK_EVALUE, "hk_launch: block must be a multiple of 64 in [64, 1024], got " +
                                   std::to_string(block));
    if (per_thread == 0 || per_thread > 64)
        return fail(HK_EVALUE, "hk_launch: per_thread must be in [1, 64], got " + std::to_string(per_thread));
    const int64_t per_block = static_cast<int64_t>(block) * per_thread;
    // a multiple of 8 workgroups, so the emitted stage can hand each XCD a
    // contiguous eighth of the blocks (a workgroup past `count` finds no samples)
    const int64_t grid = ((count + per_block - 1) / per_block + 7) / 8 * 8;
    if (grid > 0x7fffffffLL) return fail(HK_EVALUE, "hk_launch: " + std::to_string(grid) + " workgroups exceed the grid limit");
    return launch_impl(entry, ab, base, count, n_samples, static_cast<uint32_t>(grid), block, stream);
}

int hk_launch_grid(const hk_entry* entry, const hk_argblock* ab, int64_t base,
                   int64_t count, int64_t n_samples, uint32_t grid,
                   uint32_t block, void* stream) {
    cross();
    if (!entry || !ab) return fail(HK_EVALUE, "hk_launch_grid: entry and argblock are required");
    if (base < 0 || count < 0 || n_samples < 0 || base + count > n_samples)
        return fail(HK_EVALUE, "hk_launch_grid: the range [" + std::to_string(base) + ", " +
                                   std::to_string(base + count) + ") is not inside [0, " +
                                   std::to_string(n_samples) + ")");
    if (grid == 0 || block == 0 || block > 1024 || block % 64 != 0)
        return fail(HK_EVALUE, "hk_launch_grid: grid must be positive and block a multiple of 64 in [64, 1024]");
    return launch_impl(entry, ab, base, count, n_samples, grid, block, stream);
}

}  // extern "C"
