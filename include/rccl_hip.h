/*
 * rccl_hip: MI355X (gfx950) ordering primitives behind a plain C ABI.
 *
 * This is the drop-in boundary for the ordering hot path of StarGazerM/rccl
 * (a Rust CUB/Thrust reimplementation). Each entry point replaces one family
 * of the reference's public functions; the comment above it cites the
 * reference interface (paths relative to that tree). A Rust binding would
 * declare these in an `extern "C"` block and keep the reference's public
 * surface (Program, Launch/Execution, views, typed workspaces) on top.
 *
 * Conventions (rccl-cub/src/error.rs:3-25, rccl-thrust/src/cuda.rs):
 *  - All pointers are device pointers unless stated otherwise; sizes are in
 *    elements. The caller owns inputs, outputs and the workspace; no entry
 *    point allocates device memory (the one-time device probes of
 *    rccl_hip_program_load write a static device array of the library).
 *  - The first call on a device probes it (lane order of LDS atomics, block
 *    placement, CU count) with launches on the null stream and a synchronous
 *    copy, unless rccl_hip_program_load already did. On a stream under HIP
 *    graph capture such a first call returns RCCL_HIP_ERROR_INVALID_ARGUMENT
 *    before any launch: load the program on the device before capturing.
 *  - Work is enqueued on `stream` and is asynchronous (CUB semantics). The
 *    Thrust-style synchronous behaviour is the host layer's job.
 *  - Every call validates all arguments before the first launch and returns a
 *    status that maps onto DeviceAlgorithmError, one code per variant (1-8);
 *    9 is an invalid-argument guard with no variant, and
 *    InvalidHistogramShape (error.rs:19, DeviceHistogram) has no code, as
 *    histograms are outside this library. Details of the last failure on
 *    the calling thread are available from rccl_hip_last_error().
 *  - Empty inputs (and empty radix bit windows) return success without
 *    launching anything.
 */
#ifndef RCCL_HIP_H
#define RCCL_HIP_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RCCL_HIP_ABI_VERSION 1

#if defined(__GNUC__) || defined(__clang__)
#define RCCL_HIP_API __attribute__((visibility("default")))
#else
#define RCCL_HIP_API
#endif

/* Status codes: DeviceAlgorithmError variants (rccl-cub/src/error.rs:3-17). */
typedef enum rccl_hip_status {
  RCCL_HIP_SUCCESS = 0,
  RCCL_HIP_ERROR_LENGTH_MISMATCH = 1,     /* LengthMismatch{role,expected,actual} */
  RCCL_HIP_ERROR_WORKSPACE_TOO_SMALL = 2, /* WorkspaceTooSmall{role,required,actual} */
  RCCL_HIP_ERROR_INVALID_BIT_RANGE = 3,   /* InvalidBitRange{begin,end,key_bits} */
  RCCL_HIP_ERROR_UNSUPPORTED_TARGET = 4,  /* UnsupportedTarget(msg) */
  RCCL_HIP_ERROR_SIZE_OVERFLOW = 5,       /* SizeOverflow */
  RCCL_HIP_ERROR_MEMORY = 6,              /* Memory(MemoryError) */
  RCCL_HIP_ERROR_DRIVER = 7,              /* Driver(DriverError): a HIP call failed */
  RCCL_HIP_ERROR_LAUNCH = 8,              /* Launch(LaunchContractError) */
  RCCL_HIP_ERROR_INVALID_ARGUMENT = 9     /* a null pointer or unknown enum value */
} rccl_hip_status;

/* Key types. 0..5 are the radix-sortable RadixKey set
 * (rccl-cub/src/radix.rs:114-173); merge, merge sort and set operations also
 * accept the 8/16-bit integers, which the reference reaches through generic
 * DeviceCopy keys with a natural-order closure. */
typedef enum rccl_hip_key_kind {
  RCCL_HIP_KEY_U32 = 0,
  RCCL_HIP_KEY_I32 = 1,
  RCCL_HIP_KEY_F32 = 2,
  RCCL_HIP_KEY_U64 = 3,
  RCCL_HIP_KEY_I64 = 4,
  RCCL_HIP_KEY_F64 = 5,
  RCCL_HIP_KEY_U8 = 6,
  RCCL_HIP_KEY_I8 = 7,
  RCCL_HIP_KEY_U16 = 8,
  RCCL_HIP_KEY_I16 = 9
} rccl_hip_key_kind;

/* Comparator variants. A reference closure `|a, b| a.cmp(b)` (or the
 * closure-free natural order, rccl-thrust/src/merge.rs:169-178) lowers to
 * ASCENDING and `|a, b| b.cmp(a)` to DESCENDING. For floats the order is IEEE
 * `<` (-0.0 and +0.0 are equivalent). */
typedef enum rccl_hip_order {
  RCCL_HIP_ORDER_ASCENDING = 0,
  RCCL_HIP_ORDER_DESCENDING = 1
} rccl_hip_order;

/* Set operations (rccl-cub/src/ordering_backend/set.rs:564-827). */
typedef enum rccl_hip_set_operation {
  RCCL_HIP_SET_UNION = 0,
  RCCL_HIP_SET_INTERSECTION = 1,
  RCCL_HIP_SET_DIFFERENCE = 2,
  RCCL_HIP_SET_SYMMETRIC_DIFFERENCE = 3
} rccl_hip_set_operation;

/* Per-run operators of the adjacent-run compactions: UNIQUE keeps a run's
 * first key; the others also fold the run's values left to right with the
 * reference's sealed provenance operators
 * (rccl-cub/src/grouped_reduction.rs:17-75): NATURAL_BAG_ADD on u64 (wrapping
 * add), BOOLEAN_OR on one-byte BooleanProvenance (nonzero is true, the result
 * is 0 or 1), INDEPENDENT_PROBABILITY_OR on f64 ((l + r) - l * r, each step
 * rounded, clamped to [0, 1]). */
typedef enum rccl_hip_group_op {
  RCCL_HIP_GROUP_UNIQUE = 0,
  RCCL_HIP_GROUP_NATURAL_BAG_ADD = 1,
  RCCL_HIP_GROUP_BOOLEAN_OR = 2,
  RCCL_HIP_GROUP_INDEPENDENT_PROBABILITY_OR = 3
} rccl_hip_group_op;

/* Details of the most recent failing call on this thread. `role` names the
 * offending range, as the reference's `role: &'static str` does. */
typedef struct rccl_hip_error_info {
  rccl_hip_status status;
  const char *role;     /* static string; never NULL */
  uint64_t expected;    /* LengthMismatch.expected / WorkspaceTooSmall.required */
  uint64_t actual;
  uint32_t begin_bit;   /* InvalidBitRange */
  uint32_t end_bit;
  uint32_t key_bits;
  int hip_error;        /* hipError_t for DRIVER/LAUNCH, else 0 */
} rccl_hip_error_info;

/* Copy the last error of the calling thread into *info. */
RCCL_HIP_API void rccl_hip_last_error(rccl_hip_error_info *info);
/* Static description of a status code. */
RCCL_HIP_API const char *rccl_hip_status_string(rccl_hip_status status);
/* RCCL_HIP_ABI_VERSION of the loaded library. */
RCCL_HIP_API int rccl_hip_abi_version(void);

/* Check that `device` is a gfx950 GPU the kernels were built for. Replaces
 * Program::load (rccl-cub/src/cuda.rs:749-756, rccl-thrust/src/cuda.rs:85-91)
 * and the target gate ensure_radix_target (rccl-cub/src/radix.rs:14-22).
 * Returns UNSUPPORTED_TARGET on any other architecture. On first use of a
 * device it also checks, on every CU at once, that the LDS serves the lanes
 * of one atomic hitting the same address in lane order (the default radix
 * ranking relies on it); where it does not, the radix sorts rank by wave
 * match-any instead, with the same results (forcing the lane-ordered ranking
 * with rccl_hip_radix_configure then fails with UNSUPPORTED_TARGET). */
RCCL_HIP_API rccl_hip_status rccl_hip_program_load(int device);

/* ------------------------------------------------------------------------
 * Kernel timing (observability). The reference has no tracing in code; its
 * benchmarks bracket calls with CUDA events
 * (rccl-cub/examples/device_ordering_benchmark.rs:29-69). When enabled, the
 * library records a hipEvent pair around every kernel it launches, on the
 * launch's stream; rccl_hip_timing_read synchronizes those events, returns
 * one record per launch in issue order and clears the log.
 * ------------------------------------------------------------------------ */
typedef struct rccl_hip_kernel_timing {
  const char *kernel; /* static name, e.g. "radix_onesweep" */
  float ms;           /* hipEventElapsedTime of the launch */
  uint64_t items;     /* items the launch processed */
} rccl_hip_kernel_timing;

/* Turn per-launch timing on (nonzero) or off (0). Off by default. */
RCCL_HIP_API rccl_hip_status rccl_hip_timing_enable(int enable);
/* Copy up to `capacity` records into `out` (may be NULL to query the count),
 * store the number of records in *count and clear the log. */
RCCL_HIP_API rccl_hip_status rccl_hip_timing_read(rccl_hip_kernel_timing *out,
                                                  size_t capacity, size_t *count);

/* ------------------------------------------------------------------------
 * DeviceRadixSort
 * ------------------------------------------------------------------------ */

/* Bytes of control workspace (bins, look-back descriptors, tile counters) a
 * radix sort of n items needs. value_bytes is 0 for keys-only, else one of
 * 1, 2, 4, 8, 16. Replaces device_radix_sort_{keys,pairs}_buffer_workspace
 * and the control part of device_radix_sort_{,pairs_}workspace
 * (rccl-cub/src/workspace.rs:108-177). The workspace needs no initialisation
 * and may be reused by later calls on the same stream. */
RCCL_HIP_API rccl_hip_status rccl_hip_radix_sort_workspace_bytes(rccl_hip_key_kind key,
                                                    size_t value_bytes, size_t n,
                                                    size_t *bytes);

/* Double-buffer radix sort over bits [begin_bit, end_bit) of the key's
 * order-preserving bit image. Input is the buffer selected by
 * *current_is_first (1: keys_first/values_first); the result lands in the
 * buffer *current_is_first selects on return, the other buffer is clobbered.
 * values_first/values_second are NULL iff value_bytes == 0.
 * Replaces device_radix_sort_{keys,pairs}_buffer{,_descending}
 * (rccl-cub/src/dispatch.rs:2091-2943; pass control rccl-cub/src/radix.rs:427-554,
 * :627-759; DoubleBuffer rccl-cub/src/double_buffer.rs:6-130). Stable; no
 * length cap below 2^32 items. The four buffers must not share a byte
 * (RCCL_HIP_ERROR_INVALID_ARGUMENT before any launch): every pass reads one of
 * each pair and writes the other. */
RCCL_HIP_API rccl_hip_status rccl_hip_radix_sort_buffer(rccl_hip_key_kind key, size_t value_bytes,
                                           rccl_hip_order order, void *keys_first,
                                           void *keys_second, void *values_first,
                                           void *values_second, size_t n,
                                           int *current_is_first, uint32_t begin_bit,
                                           uint32_t end_bit, void *workspace,
                                           size_t workspace_bytes, hipStream_t stream);

/* Onesweep ranking modes (rccl_hip_radix_configure). */
enum {
  RCCL_HIP_RANKING_AUTO = 0,        /* lane-ordered atomics where the device check passes,
                                       else match-any */
  RCCL_HIP_RANKING_LANE_ATOMIC = 1, /* returning LDS atomics served in lane order */
  RCCL_HIP_RANKING_MATCH_ANY = 2    /* wave64 ballot/mbcnt match-any multisplit */
};

/* Onesweep tile orders (rccl_hip_radix_configure). */
enum {
  RCCL_HIP_TILE_ORDER_AUTO = 0,  /* XCD-ordered tiles where the device check sees blocks land
                                    on the 8 XCDs round-robin, else tickets */
  RCCL_HIP_TILE_ORDER_TICKET = 1 /* every block claims its tile from an atomic ticket */
};

/* Selects how the radix sort ranks keys within a tile (every radix path:
 * radix sort, the merge-sort lowering and the record sort) and how blocks find
 * their tiles (those paths, and the set operations and compactions, whose
 * look-backs order tiles the same way), for every later call in the process.
 * No counterpart in the
 * reference, whose onesweep always ranks with match-any and claims tiles
 * from a ticket (rccl-cub/src/ordering_backend/radix.rs:918-938, :1078-1087).
 * The output is identical in every mode; the defaults are the fastest ones
 * the device supports. RCCL_HIP_RANKING_LANE_ATOMIC makes sorts return
 * RCCL_HIP_ERROR_UNSUPPORTED_TARGET on a device whose LDS does not serve
 * same-address atomic lanes in lane order (checked once per device by
 * rccl_hip_program_load). */
RCCL_HIP_API rccl_hip_status rccl_hip_radix_configure(int ranking, int tile_order);

/* Size of the device-resident control workspace of rccl_hip_radix_sort_static
 * (per device, held until the process ends): 48 MiB, enough for 2^28 u32 keys
 * or 2^28 u64-key/u32-value pairs. */
#define RCCL_HIP_STATIC_RADIX_WORKSPACE_BYTES (48u << 20)

/* rccl_hip_radix_sort without a workspace argument: no counterpart in the
 * reference. For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc): the
 * bins and look-back buffers live in a library-owned static device array of
 * RCCL_HIP_STATIC_RADIX_WORKSPACE_BYTES per device, and nothing is
 * allocated. The caller still passes keys, values and the n-item scratch
 * buffers. A sort whose workspace (rccl_hip_radix_sort_workspace_bytes)
 * exceeds that size returns RCCL_HIP_ERROR_WORKSPACE_TOO_SMALL before any
 * launch. Every call on one device shares that device's array (each call
 * clears what it uses), so calls that overlap on one device (different
 * streams, or threads) race: serialize them. Under graph capture, load the
 * program on the device first (rccl_hip_program_load): the device probe of a
 * first call cannot run on a capturing stream (RCCL_HIP_ERROR_INVALID_ARGUMENT). */
RCCL_HIP_API rccl_hip_status rccl_hip_radix_sort_static(rccl_hip_key_kind key,
                                                        size_t value_bytes, rccl_hip_order order,
                                                        void *keys, void *values,
                                                        void *scratch_keys, void *scratch_values,
                                                        size_t n, hipStream_t stream);

/* In-place radix sort of all key bits with caller-owned scratch of n keys
 * (and n values). Replaces device_radix_sort_{keys,pairs}{,_descending}
 * (rccl-cub/src/radix.rs:558-623, :763-876): the result is copied back when
 * it lands in the scratch buffer. keys, values and the scratch buffers must
 * not share a byte (RCCL_HIP_ERROR_INVALID_ARGUMENT). */
RCCL_HIP_API rccl_hip_status rccl_hip_radix_sort(rccl_hip_key_kind key, size_t value_bytes,
                                    rccl_hip_order order, void *keys, void *values,
                                    void *scratch_keys, void *scratch_values, size_t n,
                                    void *workspace, size_t workspace_bytes,
                                    hipStream_t stream);

/* ------------------------------------------------------------------------
 * DeviceMerge
 * ------------------------------------------------------------------------ */

/* Workspace bytes for merging na + nb items. Replaces
 * device_merge_{keys,pairs}_workspace (rccl-cub/src/workspace.rs:215-243). */
RCCL_HIP_API rccl_hip_status rccl_hip_merge_workspace_bytes(rccl_hip_key_kind key, size_t value_bytes,
                                               size_t na, size_t nb, size_t *bytes);

/* Stable merge of two sorted ranges into out (na + nb items); on equivalent
 * keys every item of A precedes those of B. Values (value_bytes > 0) follow
 * their keys. Replaces device_merge_keys/device_merge_pairs
 * (rccl-cub/src/dispatch.rs:1572,1915; rccl-cub/src/merge.rs:194-368) and the
 * Thrust merge(..).write_into forms (rccl-thrust/src/merge.rs:83-247). An
 * output that shares a byte with an input, or out_keys with out_values, is
 * rejected with RCCL_HIP_ERROR_INVALID_ARGUMENT. */
RCCL_HIP_API rccl_hip_status rccl_hip_merge(rccl_hip_key_kind key, size_t value_bytes,
                               rccl_hip_order order, const void *a_keys,
                               const void *a_values, size_t na, const void *b_keys,
                               const void *b_values, size_t nb, void *out_keys,
                               void *out_values, void *workspace, size_t workspace_bytes,
                               hipStream_t stream);

/* ------------------------------------------------------------------------
 * DeviceMergeSort
 * ------------------------------------------------------------------------ */

/* Workspace bytes (scratch keys/values and partitions) for a merge sort of n
 * items. Replaces device_merge_sort_{keys,pairs}_workspace
 * (rccl-cub/src/workspace.rs:251-285). */
RCCL_HIP_API rccl_hip_status rccl_hip_merge_sort_workspace_bytes(rccl_hip_key_kind key,
                                                    size_t value_bytes, size_t n,
                                                    size_t *bytes);

/* Stable merge sort. in_keys == out_keys (and in_values == out_values) sorts
 * in place; otherwise the inputs are left untouched (the _copy forms), and an
 * output that partly overlaps its input (or out_keys that overlaps
 * out_values) is rejected with RCCL_HIP_ERROR_INVALID_ARGUMENT. Float
 * keys compare with IEEE `<` (-0.0 and +0.0 are equal and keep their input
 * order); inputs holding NaN, which `<` cannot order, have no defined order.
 * Replaces device_merge_sort_{keys,pairs}{,_copy}
 * (rccl-cub/src/dispatch.rs:170-322,1116-1400; rccl-cub/src/merge_sort.rs:156-690)
 * and Thrust sort_by / sort_unstable_by (rccl-thrust/src/backend.rs:39-150). */
RCCL_HIP_API rccl_hip_status rccl_hip_merge_sort(rccl_hip_key_kind key, size_t value_bytes,
                                    rccl_hip_order order, const void *in_keys,
                                    const void *in_values, void *out_keys,
                                    void *out_values, size_t n, void *workspace,
                                    size_t workspace_bytes, hipStream_t stream);

/* ------------------------------------------------------------------------
 * Record sort (SRDatalog/HISA relation rows)
 * ------------------------------------------------------------------------ */

/* Workspace bytes for a record sort of n rows of `arity` u32 columns with a
 * payload of payload_bytes (0, 1 or 8) per row. Replaces the internal
 * DeviceMergeSort{Keys,Pairs}Workspace of the record sorts
 * (rccl-thrust/src/record_sort.rs:159-160,253-254). UNSUPPORTED_TARGET for an
 * arity outside 2..6 (record_sort.rs:117-126). */
RCCL_HIP_API rccl_hip_status rccl_hip_record_sort_workspace_bytes(uint32_t arity,
                                                     size_t payload_bytes, size_t n,
                                                     size_t *bytes);

/* Stable ascending lexicographic sort of n padding-free rows of `arity` u32
 * columns (row-major, 4 * arity bytes per row); equal rows keep their input
 * order, and each row's payload (payload_bytes = 0, 1 for BooleanProvenance or
 * 8 for u64/f64, NULL pointers when 0) moves with it. in_rows == out_rows
 * (and in_payloads == out_payloads) sorts in place; otherwise the inputs are
 * left untouched; inputs and outputs must otherwise not overlap. From 65,536
 * rows the sort is a multi-word LSD radix sort whose ranking relies on the
 * check rccl_hip_program_load runs, so load the device first. Replaces
 * sort_rows_lexicographic{,_into} and sort_rows_with_payload_lexicographic{,_into}
 * (rccl-thrust/src/record_sort.rs:144-366). Outputs that partly overlap their inputs,
 * or out_rows that overlaps out_payloads, are rejected with
 * RCCL_HIP_ERROR_INVALID_ARGUMENT. */
RCCL_HIP_API rccl_hip_status rccl_hip_record_sort(uint32_t arity, size_t payload_bytes,
                                     const void *in_rows, const void *in_payloads,
                                     void *out_rows, void *out_payloads, size_t n,
                                     void *workspace, size_t workspace_bytes,
                                     hipStream_t stream);

/* ------------------------------------------------------------------------
 * Set operations
 * ------------------------------------------------------------------------ */

/* Workspace bytes for a set operation over na + nb items. Replaces
 * set_workspace_counts and the TemporaryWorkspace5 layout of
 * rccl-thrust/src/set.rs:27-125 (rccl-cub/src/workspace.rs:287-357). */
RCCL_HIP_API rccl_hip_status rccl_hip_set_op_workspace_bytes(rccl_hip_set_operation op, rccl_hip_key_kind key,
                                                size_t value_bytes, size_t na, size_t nb,
                                                size_t *bytes);

/* Sorted multiset operation. Writes the result length to *d_out_count
 * (device memory, one uint64_t; may be NULL when out_keys is given).
 * out_keys == NULL counts without writing keys (the `.count()` form; then
 * d_out_count is required); out_values is read only when value_bytes != 0
 * and out_keys != NULL. INTERSECTION and DIFFERENCE emit values from A only
 * and do not read b_values. Empty inputs write a count of 0. out_capacity is
 * the number of items out_keys (and out_values) can hold: the full result
 * length is always counted, but items at or past out_capacity are not
 * written (the reference leaves the destination's size to the caller).
 * Outputs (out_capacity items) that share a byte with an input it reads are
 * rejected with RCCL_HIP_ERROR_INVALID_ARGUMENT.
 * Replaces Launch::set_keys / set_pairs (rccl-cub/src/dispatch.rs:413-550;
 * rccl-cub/src/set_operation.rs:265-589) and the Thrust union/intersection/
 * difference/symmetric_difference expressions (rccl-thrust/src/set.rs:357-898). */
RCCL_HIP_API rccl_hip_status rccl_hip_set_op(rccl_hip_set_operation op, rccl_hip_key_kind key,
                                size_t value_bytes, rccl_hip_order order,
                                const void *a_keys, const void *a_values, size_t na,
                                const void *b_keys, const void *b_values, size_t nb,
                                void *out_keys, void *out_values, size_t out_capacity,
                                uint64_t *d_out_count, void *workspace,
                                size_t workspace_bytes, hipStream_t stream);

/* Set operation over two finite arithmetic ranges, keys only: item i of A is
 * a_start + a_step * i (and likewise B), in the key type's wrapping integer
 * arithmetic; neither input is materialised. a_start/a_step/b_start/b_step
 * point to one host value of the key type each. Integer key kinds only; each
 * index must fit the key type (the reference traps on the device when it does
 * not; here the call fails before any launch). Output, count, capacity and
 * workspace (rccl_hip_set_op_workspace_bytes with value_bytes 0) as for
 * rccl_hip_set_op. Replaces Launch::set_arithmetic
 * (rccl-cub/src/dispatch.rs:552-740, set_operation.rs:417-480) and the Thrust
 * arithmetic-range expressions (rccl-thrust/src/set.rs:127-244,477-530). */
RCCL_HIP_API rccl_hip_status rccl_hip_set_op_arithmetic(
    rccl_hip_set_operation op, rccl_hip_key_kind key, rccl_hip_order order,
    const void *a_start, const void *a_step, size_t na, const void *b_start,
    const void *b_step, size_t nb, void *out_keys, size_t out_capacity, uint64_t *d_out_count,
    void *workspace, size_t workspace_bytes, hipStream_t stream);

/* ------------------------------------------------------------------------
 * Adjacent-run compaction (unique, reduce-by-key)
 * ------------------------------------------------------------------------ */

/* Keys are `key` scalars when arity == 1, or padding-free rows of `arity`
 * (2..6) u32 columns when key == RCCL_HIP_KEY_U32. Adjacent keys are in one
 * run when they compare equal (scalars with ==, so NaN keys never join a run;
 * rows column by column). A key may carry a payload of payload_bytes per item
 * (UNIQUE: 0, 1, 2, 4 or 8; the reductions: 0, 4 or 8) that takes no part in
 * the comparison; each output gets the payload of its run's first item (the
 * reference's key/value ranges compared by key). Workspace bytes for n keys. */
RCCL_HIP_API rccl_hip_status rccl_hip_group_workspace_bytes(rccl_hip_key_kind key, uint32_t arity,
                                                           rccl_hip_group_op op,
                                                           size_t payload_bytes, size_t n,
                                                           size_t *bytes);

/* Stable adjacent unique: out_keys[0, count) (and out_payloads) = the first
 * item of every run of in_keys[0, n); count is written to *d_count (device
 * memory, one uint64_t). Outputs must hold n items and not overlap the
 * inputs or each other (RCCL_HIP_ERROR_INVALID_ARGUMENT). Replaces unique_copy_by (rccl-thrust/src/compaction.rs:224-301)
 * with the natural equivalence; the in-place unique_by (:303-378) is a copy
 * to the scratch range followed by this call from the scratch back into the
 * values. */
RCCL_HIP_API rccl_hip_status rccl_hip_unique_copy(rccl_hip_key_kind key, uint32_t arity,
                                                  size_t payload_bytes, const void *in_keys,
                                                  const void *in_payloads, void *out_keys,
                                                  void *out_payloads, size_t n, uint64_t *d_count,
                                                  void *workspace, size_t workspace_bytes,
                                                  hipStream_t stream);

/* Reduce by key over sorted adjacent runs: for every run of equal adjacent
 * keys, out_keys (and out_key_payloads) get its first item and out_values the
 * left fold ((v0 op v1) op v2) ... of its values, in run order; the number of
 * runs is written to *d_group_count. op is NATURAL_BAG_ADD (u64 values),
 * BOOLEAN_OR (1-byte values) or INDEPENDENT_PROBABILITY_OR (f64 values).
 * Outputs must hold n items and not overlap the inputs or each other
 * (RCCL_HIP_ERROR_INVALID_ARGUMENT). Replaces reduce_by_key (rccl-thrust/src/grouped_reduction.rs:102-216,
 * rccl-cub/src/grouped_reduction.rs:83-143) with the natural equivalence. */
RCCL_HIP_API rccl_hip_status rccl_hip_reduce_by_key(
    rccl_hip_key_kind key, uint32_t arity, rccl_hip_group_op op, size_t payload_bytes,
    const void *keys, const void *key_payloads, const void *values, void *out_keys,
    void *out_key_payloads, void *out_values, size_t n, uint64_t *d_group_count,
    void *workspace, size_t workspace_bytes, hipStream_t stream);

/* ------------------------------------------------------------------------
 * Vectorized binary search
 * ------------------------------------------------------------------------ */

/* For each of the m needles, the index in the sorted haystack[0, n) of the
 * first item not before it (upper == 0: lower_bound, the first i with
 * !(h[i] < x)) or of the first item after it (upper != 0: upper_bound, the
 * first i with x < h[i]); n when there is none. Indices are written to
 * out_indices[0, m) as uint64_t. `<` is the natural order of `key` (or its
 * reverse when order is DESCENDING); with arity 2..6 and key == U32 the
 * items are [u32; arity] rows in ascending lexicographic order. The haystack
 * must be sorted under that order (results are unspecified otherwise, as
 * with NaN keys). out_indices must not overlap the haystack or the needles
 * (RCCL_HIP_ERROR_INVALID_ARGUMENT). thrust::lower_bound / upper_bound over a range of values
 * has no counterpart in the reference (CCCL_RUST_CAPABILITY_CHECKLIST.md:107
 * lists it as missing); its datalog callers search sorted columns.
 * The workspace (rccl_hip_bound_search_workspace_bytes) holds a per-call
 * index of the haystack's cache-line chunks, built when there are enough
 * needles to repay it; WORKSPACE_TOO_SMALL when such a call's is short. */
RCCL_HIP_API rccl_hip_status rccl_hip_bound_search(rccl_hip_key_kind key, uint32_t arity,
                                                   rccl_hip_order order, int upper,
                                                   const void *haystack, size_t n,
                                                   const void *needles, size_t m,
                                                   uint64_t *out_indices, void *workspace,
                                                   size_t workspace_bytes, hipStream_t stream);

/* Workspace bytes for bound searches in a haystack of n items of `key` (or
 * [u32; arity] rows): the chunk index, one item per 128 bytes of haystack,
 * or 0 when the haystack is small enough to need none. No counterpart in
 * the reference (see rccl_hip_bound_search). */
RCCL_HIP_API rccl_hip_status rccl_hip_bound_search_workspace_bytes(rccl_hip_key_kind key,
                                                                   uint32_t arity, size_t n,
                                                                   size_t *bytes);

#ifdef __cplusplus
}
#endif

#endif /* RCCL_HIP_H */
