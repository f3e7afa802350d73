/* hawk_core.h — the C-ABI of hawk's MI355X (gfx950) device target.
 *
 * This library replaces the reference's nanobind module `hawk._core`
 * (reference `src/hawk_core.cpp:518-679`) with a plain C ABI that any FFI
 * (Python ctypes here) can bind: every argument is a pointer, a size or a
 * scalar, and no PyTorch or Python type crosses it.  Device planes are passed
 * as raw HIP device pointers (`torch.Tensor.data_ptr()` on the Python side).
 *
 * Every call returns HK_OK (0) or a non-zero HK_E* code; on failure the
 * thread-local text returned by hk_last_error() names the field, slot or
 * argument at fault, with the same wording the reference raises as
 * ValueError / IndexError (reference `src/hawk_core.cpp:152-156`, `:274-302`,
 * `:360-389`).  Every exported call counts one boundary crossing
 * (hk_crossings), like the reference's `crossings()` instrument
 * (reference `src/hawk_core.cpp:97-118`).
 *
 * Threading: distinct objects may be used from distinct threads.  One
 * ArgBlock shared by threads must be serialised by the caller (the Python
 * runtime holds a per-kernel lock, as reference `hawk/runtime.py:46-53`).
 */
#ifndef HAWK_CORE_H
#define HAWK_CORE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes -------------------------------------------------------- */
#define HK_OK 0
#define HK_EVALUE 1   /* a ValueError in the reference's binding           */
#define HK_EINDEX 2   /* an IndexError (slot out of range)                  */
#define HK_EHIP 3     /* a HIP runtime / hipRTC call failed                 */
#define HK_ESTATUS 4  /* a team stage reported a bad key (status plane)     */

/* The ABI generation every artifact must export as `eagle_abi_tag`
 * (reference `hawk/_contracts.py:40-92`, `src/hawk_core.cpp:366-374`). */
#define HK_ABI_TAG "aether-abi/2"

/* Field order of the exported `eagle_layout_sizes[5]` table:
 * GRefMirror (40), ScalarHandle (32), IntHandle (32), index_t (8),
 * PartitionTriple (24) (reference `hawk/artifact/layout.py:35-61`). */
#define HK_LAYOUT_FIELDS 5

/* DLPack device codes a mirror carries: CPU = 1, ROCm = 10. */
#define HK_DEVICE_CPU 1
#define HK_DEVICE_ROCM 10

typedef struct hk_library hk_library;   /* a loaded gfx950 code object */
typedef struct hk_entry hk_entry;       /* one __global__ entry of it  */
typedef struct hk_argblock hk_argblock; /* the by-value mirror block   */

/* ---- diagnostics / self-check ------------------------------------------- */

/* Thread-local text of the last failure on this thread ("" if none). */
const char* hk_last_error(void);

/* Replaces `_core.layout_sizes()` (reference `src/hawk_core.cpp:536-541`):
 * this library's own sizes, in the field order above. */
int hk_layout_sizes(uint64_t out[HK_LAYOUT_FIELDS]);

/* Replaces `_core.layout_field_name(i)` (reference `src/hawk_core.cpp:543`). */
const char* hk_layout_field_name(int i);

/* Replaces `_core.build_digest()` (reference `src/hawk_core.cpp:522-529`):
 * the sha256 of this library's sources, stamped at build. */
const char* hk_build_digest(void);

/* Replaces `_core.build_info()` (reference `src/hawk_core.cpp:544-559`):
 * "key=value" lines (compiler, flags, offload arch, abi tag, index width). */
const char* hk_build_info(void);

/* Replaces `_core.crossings()` (reference `src/hawk_core.cpp:561-567`). */
uint64_t hk_crossings(void);

/* ---- build: hipRTC pinned to gfx950 -------------------------------------- */

/* Compile `source` (HIP C++) with hipRTC for --offload-arch=gfx950 plus the
 * given extra options.  On success *code / *code_size hold a malloc'ed code
 * object (free with hk_free).  *log (may be NULL) receives the compiler log,
 * malloc'ed, on success and failure.  Replaces the NVRTC route of reference
 * `hawk/compile/nvrtc.py:479-582`. */
int hk_rtc_compile(const char* source, const char* name,
                   const char* const* options, int n_options,
                   void** code, size_t* code_size, char** log);

/* The hipRTC version as major*100+minor (part of the compile-cache key). */
int hk_rtc_version(void);

void hk_free(void* p);

/* ---- load: module + ABI self-check -------------------------------------- */

/* Load a gfx950 code object and check its exported `eagle_abi_tag` and
 * `eagle_layout_sizes` against this library, refusing a mismatch by naming
 * the field.  Replaces `_core.HostLibrary(path)` (reference
 * `src/hawk_core.cpp:354-390`). */
int hk_load(const void* code, size_t code_size, hk_library** out);
void hk_unload(hk_library* lib);

/* Resolve one __global__ entry.  Replaces `HostLibrary.entry(name)`
 * (reference `src/hawk_core.cpp:395-401`). */
int hk_entry_get(hk_library* lib, const char* name, hk_entry** out);

/* ---- bind: the by-value mirror block ------------------------------------ */

/* One kind name per slot, in arg_spec order: "gref" (40 B GRefMirror),
 * "handle" / "int_handle" (32 B), "f64" / "f32" / "int" / "nsamples"
 * (by value).  Replaces `_core.ArgBlock(descriptor)` (reference
 * `src/hawk_core.cpp:185-215`). */
int hk_argblock_new(const char* const* kinds, int n_slots, hk_argblock** out);
void hk_argblock_free(hk_argblock* ab);
int hk_argblock_size(const hk_argblock* ab);

/* Write ONE slot's mirror.  For a by-value slot `ptr` is the ADDRESS of the
 * value, which is copied.  A GRef plane's component pitch is
 * samples*stride.  Replaces `ArgBlock.bind` (reference
 * `src/hawk_core.cpp:228-267`). */
int hk_bind(hk_argblock* ab, int slot, uint64_t ptr, uint64_t samples,
            uint64_t stride, int32_t device_type, int32_t device_id);

/* The bulk pointer swap: `n` (slot, ptr) pairs in one crossing.  A by-value
 * slot is refused.  Replaces `ArgBlock.rebind` (reference
 * `src/hawk_core.cpp:270-305`). */
int hk_rebind(hk_argblock* ab, const int64_t* slots, const int64_t* ptrs,
              size_t n);

/* ---- launch ------------------------------------------------------------ */

/* Launch `entry` over samples [base, base+count) of n_samples on `stream`
 * (a hipStream_t, NULL = default stream): ceil(count/(block*per_thread))
 * workgroups of `block` threads, each thread taking `per_thread` samples,
 * rounded up to a multiple of 8 workgroups (one per XCD in turn; a workgroup
 * past `count` finds no samples).
 * Replaces `HostEntry.run(argblock, base, count, n_samples)` (reference
 * `src/hawk_core.cpp:438-442`); the device entry signature is
 * `(mirrors..., long long base, long long count, long long nSamples)` as
 * reference `hawk/emit/cuda.py:46-54`. */
int hk_launch(const hk_entry* entry, const hk_argblock* ab, int64_t base,
              int64_t count, int64_t n_samples, uint32_t block,
              uint32_t per_thread, void* stream);

/* Launch `entry` on exactly `grid` workgroups of `block` threads with the
 * triple (base, count, n_samples) — the virtual-lane form of a fused
 * ordered-sum stage, whose grid is fixed by the sum, not by count. */
int hk_launch_grid(const hk_entry* entry, const hk_argblock* ab, int64_t base,
                   int64_t count, int64_t n_samples, uint32_t grid,
                   uint32_t block, void* stream);

/* ---- team stages: hand-written gfx950 kernels --------------------------- */

/* The fixed-tree ordered sum of reference `hawk/emit/team.py:208-278`
 * (`_block_part`) and `:173-192` (`_block`, gp form): 65536 virtual lanes,
 * lane l adds u[l], u[l+65536], ... in order from 0; each group of 1024 lanes
 * is folded by the halving tree s[i] += s[i+w], w = 512..1; the 64 group
 * values by the same tree, w = 32..1; the result is STORED to *out.
 * Scratch: hk_ordered_sum_scratch_bytes() bytes, zero before the first call
 * (each call leaves its counters at zero again). */
size_t hk_ordered_sum_scratch_bytes(void);
int hk_ordered_sum_f64(const double* u, int64_t n, double* out, void* scratch,
                       void* stream);
/* The same sum in the float32 mode: the lanes, the trees and *out are float
 * (the reference's team stages add `Real`s, `hawk/emit/team.py:248-261`).
 * Same scratch (size and zero-before-first-call rule) as the fp64 sum. */
int hk_ordered_sum_f32(const float* u, int64_t n, float* out, void* scratch,
                       void* stream);

/* hk_ordered_sum_f64 for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  It has no counterpart in the reference.  It allocates nothing:
 * its scratch is a static device array of hk_ordered_sum_noalloc_scratch_bytes()
 * bytes (512 KiB + 768 B, whatever n is), one copy per GPU, held until the
 * process ends; the caller passes only the input and the output.  Same
 * kernels, same bits as hk_ordered_sum_f64.  Every call on one GPU shares
 * that GPU's array, so calls that overlap on one GPU (on different streams,
 * or from different threads without ordering) race; calls in order on one
 * stream do not.  n < 0 is refused (HK_EVALUE). */
size_t hk_ordered_sum_noalloc_scratch_bytes(void);
int hk_ordered_sum_f64_noalloc(const double* u, int64_t n, double* out, void* stream);

/* The same fold over 65536 lane partials already computed in `lanes`
 * (the second half of a fused ordered-sum stage). */
int hk_ordered_fold_f64(const double* lanes, double* out, void* scratch,
                        void* stream);

/* Keyed fixed-tree sum: out[k] for k < n / group is key k's rows
 * u[k*group .. (k+1)*group) added by the ordered sum's tree, the same bits
 * hk_ordered_sum_f64 gives for those rows alone — hawk.sum(x, over=<trailing
 * lane axes>, policy="ordered") of a Grid's leading-axis coordinates.
 * Replaces the block-sum team stage of reference hawk/emit/team.py:115-205
 * (`_block` with its `gp` stage) and hawk/emit/team.py:208-278
 * (`_block_part`).  n must be a multiple of group (HK_EVALUE otherwise);
 * group == n is the one-key case and runs hk_ordered_sum_f64.
 * Scratch: hk_keyed_ordered_sum_scratch_bytes(n, group) bytes, no contents
 * needed (for group == n, the ordered sum's scratch, zero before its first call). */
size_t hk_keyed_ordered_sum_scratch_bytes(int64_t n, int64_t group);
int hk_keyed_ordered_sum_f64(const double* u, int64_t n, int64_t group, double* out,
                             void* scratch, void* stream);
/* The keyed ordered sum in the float32 mode (float rows, trees and cells),
 * same scratch and refusals. */
int hk_keyed_ordered_sum_f32(const float* u, int64_t n, int64_t group, float* out,
                             void* scratch, void* stream);

/* `hawk.sum(x, over=<trailing lane axes>)` under the default policy: for
 * k < n / group, out[k] = the default-policy sample sum of u[k*group ..
 * (k+1)*group) on its own (compensated rows of 32 from the key's first value,
 * the canonical ordered finish below, hi + comp).  The reference commits
 * each key with atomic adds of per-warp partials (`hawk/emit/wrapper.py:
 * 380-415`, the compensated accumulate), whose order varies between launches
 * once a key spans three warps; here every key takes one fixed order.  A key
 * of more than 2^25 samples is refused (HK_EVALUE).  No scratch. */
int hk_keyed_sample_sum_f64(const double* u, int64_t n, int64_t group, double* out, void* stream);
/* The same in the float32 mode: float rows, float compensation, a float
 * cell (the reference finishes a float32 build's rows in their dtype). */
int hk_keyed_sample_sum_f32(const float* u, int64_t n, int64_t group, float* out, void* stream);

/* The finish of a default-policy sample sum (`hawk.sum(x)`): `rows`
 * compensated (hi, comp) row pairs (one per 32 samples, written by the
 * per-sample stage as reference `hawk/emit/wrapper.py:542-665` does) folded
 * in the canonical ordered tree of reference `hawk/_cells.py:71-119` (leaves
 * of 256 slots x 16 rows with Neumaier adds, the in-leaf halving tree,
 * pairwise levels over the leaves) and STORED to *out as hi + comp.  The
 * reference finishes on the host; here it stays on the device.
 * Scratch: hk_rows_finish_scratch_bytes(rows) bytes. */
size_t hk_rows_finish_scratch_bytes(int64_t rows);
int hk_rows_finish_f64(const double* hi, const double* comp, int64_t rows,
                       double* out, void* scratch, void* stream);
/* The same finish of float32 rows in float32 arithmetic: the float32 scalar
 * mode's default-policy sum (reference `hawk/_cells.py:44-119` runs the
 * finish in the rows' dtype, float32 in that mode; the rows are the
 * per-sample stage's in `Real`, reference `hawk/emit/wrapper.py:542-665`).
 * Scratch: hk_rows_finish_scratch_bytes(rows) bytes. */
int hk_rows_finish_f32(const float* hi, const float* comp, int64_t rows,
                       float* out, void* scratch, void* stream);

/* The finish of `hawk.max(x)` (op 1) / `hawk.min(x)` (op 2): `rows` row
 * extremes (one per 32 samples; a row's NaN-ignoring extreme, -inf / +inf
 * past the last sample, reference `hawk/emit/wrapper.py:543-600`) folded in
 * the same canonical tree as the sum (reference `hawk/_cells.py:66-71` and
 * `finish`), every add the extreme a > b ? a : b (max) or a < b ? a : b
 * (min) of the earlier partial and the later, and stored to *out.  Exact;
 * the cell is the reference host finish's bit for bit.  Scratch:
 * hk_rows_finish_scratch_bytes(rows) bytes.  HK_EVALUE for rows < 1 or
 * another op. */
int hk_rows_extreme_f64(const double* hi, int64_t rows, int32_t op, double* out,
                        void* scratch, void* stream);
int hk_rows_extreme_f32(const float* hi, int64_t rows, int32_t op, float* out,
                        void* scratch, void* stream);

/* Banded reductions: the sample sums of the banded scalar mode (reference
 * `hawk/emit/wrapper.py:140` BANDED and its row sum `:542-665`,
 * `hawk/emit/team.py:26-49` and `:225-245`: band partials folded in the
 * float64 stages' fixed order, one value stored at the end).  A band is a
 * normalised double-double (h, l), |l| <= ulp(h)/2, added with the QD
 * library's TwoSum-based adds; the stored cell is the final band's h.
 *
 * hk_band_rows_finish_f64: `rows` band rows (hi, lo) (one per 32 samples,
 * written by a banded per-sample stage) folded in the default sum's
 * canonical tree (leaves of 256 slots x 16 rows, the halving tree, pairwise
 * levels), every add a band add.  Scratch: hk_band_rows_finish_scratch_bytes(rows).
 *
 * hk_band_ordered_sum_f64: the fixed-tree ordered sum with band
 * accumulators (65536 virtual lanes add their rows as terms, the group and
 * final trees add bands).  Scratch: hk_band_ordered_sum_scratch_bytes(), no
 * initial contents needed. */
size_t hk_band_rows_finish_scratch_bytes(int64_t rows);
int hk_band_rows_finish_f64(const double* hi, const double* lo, int64_t rows,
                            double* out, void* scratch, void* stream);
size_t hk_band_ordered_sum_scratch_bytes(void);
int hk_band_ordered_sum_f64(const double* u, int64_t n, double* out, void* scratch,
                            void* stream);

/* The keyed ordered scatter of reference `hawk/emit/team.py:322-460`
 * (`_scatter_zero`, `_scatter_chunks`, `_scatter_cells`) with the chunk rule
 * of `hawk/_lane_bind.py:111-114`: chunks = clamp(n / max(cells, 1), 1, 256),
 * span = ceil(n / chunks); part[key][b] = the in-order sum from 0 of chunk
 * b's values with that key; target[c] += (sum from 0 over b, in order, of
 * part[c][b]).  Key -1 adds nothing; any other key outside [0, cells) adds
 * nothing and sets status[1+b] (status[0] = cells).  Returns HK_OK even when
 * a bad key was met: the caller reads status[1..256] (the reference's
 * `check_scatter_status`, `hawk/_lane_bind.py:148-154`).
 * Scratch: hk_ordered_scatter_scratch_bytes(n, cells) bytes, no initial
 * contents needed: the per-(chunk, cell) partials, then (for 12288 < cells
 * <= 65536) the bins that carry each tile's lanes of keys past the first
 * 12288 from the first walk to the second. */
int hk_scatter_chunks(int64_t n, int64_t cells);
size_t hk_ordered_scatter_scratch_bytes(int64_t n, int64_t cells);
int hk_ordered_scatter_f64(const int32_t* key, const double* v, int64_t n,
                           double* target, int64_t cells, void* scratch,
                           int32_t* status, void* stream);
/* The ordered scatter in the float32 mode: v, the partials, the cells' sums
 * and target are float, every addition a float addition (the reference's
 * `_scatter_chunks` / `_scatter_cells` over `Real`).  Same scratch (the fp64
 * size is an upper bound), status and refusals. */
int hk_ordered_scatter_f32(const int32_t* key, const float* v, int64_t n,
                           float* target, int64_t cells, void* scratch,
                           int32_t* status, void* stream);

/* The ordered gradient's log fold: reference `hawk/diff/ordered.py` (the VJP
 * of a kernel holding an ordered keyed sum logs each table read's
 * contribution per lane and slot, and the cell it adds to per key and slot),
 * `hawk/ir/team.py:684-693` (`fold_spec`) and `hawk/emit/team.py:281-312`
 * (`_fold`).  For key k < keys and slot e < width: out[cells_log[e*keys + k]]
 * = the sum from +0.0, in lane order r = 0 .. rows-1, of
 * values[e*stride + k*rows + r] (STORED, not added to out).  A cell outside
 * [0, cells) is skipped and sets status[0] bit 0; a cell named by more than
 * one (key, slot) sets bit 1 and status[1] = the least such cell (those
 * stores race, as in the reference).  Returns HK_OK even then: the caller
 * reads status[0..1] after the stream completes.  Scratch:
 * hk_keyed_log_fold_scratch_bytes(cells) bytes (the claim counts, cleared by
 * the call). */
size_t hk_keyed_log_fold_scratch_bytes(int64_t cells);
int hk_keyed_log_fold_f64(const double* values, int64_t stride, const int32_t* cells_log,
                          int64_t keys, int64_t rows, int32_t width, double* out,
                          int64_t cells, void* scratch, int32_t* status, void* stream);
/* The same fold in the float32 mode (float contributions, sums and gradient
 * plane), with the same scratch, status words and refusals. */
int hk_keyed_log_fold_f32(const float* values, int64_t stride, const int32_t* cells_log, int64_t keys,
                          int64_t rows, int32_t width, float* out, int64_t cells, void* scratch,
                          int32_t* status, void* stream);

/* Per-sample 16x16 fp32 matrix products on MFMA: for every sample s < n and
 * product o < n_out, out[o] = op(in[lhs]) @ op(in[rhs]) with
 * products[3*o .. 3*o+2] = {lhs, rhs, flags}, flags bit 0 = transpose lhs,
 * bit 1 = transpose rhs.  Planes are [16, 16, n] fp32 (element (r, c) of
 * sample s at (r*16 + c)*n + s); outputs are overwritten.  1..3 inputs,
 * 1..2 products, no more products than inputs.  This is the per-sample `mm`
 * of reference `hawk/emit/policy.py:283-299` / `hawk/emit/writer_aether.py:663-671`
 * (forward C = A @ B) and its VJP (bar_A = bar_C @ B^T, bar_B = A^T @ bar_C,
 * reference `hawk/diff/rules.py`), as one team stage. */
int hk_mm16_f32(const float* const* in, int n_in, float* const* out, int n_out,
                const int32_t* products, int64_t n, void* stream);

/* hk_mm16_f32 for fp64 planes ([16, 16, n] doubles), on v_mfma_f64_16x16x4f64:
 * the per-sample `mm` of reference `hawk/emit/policy.py:283-299` in the
 * float64 mode (reference `hawk/targets/__init__.py:48-49` builds both scalar
 * modes), same arguments and refusals. */
int hk_mm16_f64(const double* const* in, int n_in, double* const* out, int n_out,
                const int32_t* products, int64_t n, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* HAWK_CORE_H */
