/*
 * CPU restatement of the reference's ordering semantics.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (rccl_amd/, include/)
 * links, loads or calls this code. It is the checker used by tests/,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (paths are relative to the StarGazerM/rccl tree).
 *
 * Pinning (how each function is checked independently of its own formula):
 *   oracle_radix_*      reference literal vectors (tests/golden): signed keys,
 *                       f32/f64 ±0/±inf keys and pairs, the f32/f64 NaN bit
 *                       order ascending and descending, and the descending
 *                       [-0.0, +0.0] -> [0x80000000, 0] known answer; the
 *                       reference's unit rule that ±0 share every digit
 *                       window in both orders (a stable two-zero sort is
 *                       unchanged in every 1..8-bit window); Python's stable
 *                       sorted() under a comparator written from IEEE 754
 *                       totalOrder with ±0 tied (float compares for numbers,
 *                       payload rules for NaNs of either sign); stable
 *                       argsort and sorted() on integer keys and windows.
 *                       A planted removal of the ±0 collapse fails all of
 *                       the ±0 checks.
 *   oracle_merge        reference literal vectors, heapq.merge (stable,
 *                       first-iterable-first on ties).
 *   oracle_merge_sort   reference literal vectors, Python sorted() (stable).
 *   oracle_set_op       reference literal vectors (incl. by-key value
 *                       selection), collections.Counter multiset algebra.
 *   oracle_record_sort  reference literal vectors, numpy's stable lexsort.
 *   oracle_unique,
 *   oracle_reduce_by_key reference literal vectors (examples/compaction.rs,
 *                       examples/grouped_reduction.rs), the reference's
 *                       operator known answers (grouped_reduction.rs:209-224),
 *                       an itertools.groupby restatement in the tests.
 *   oracle_splitmix64   published splitmix64 test value.
 */
#ifndef RCCL_ORACLE_H
#define RCCL_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Key kinds; numbering equals rccl_hip_key_kind in include/rccl_hip.h. */
enum {
  ORACLE_KEY_U32 = 0,
  ORACLE_KEY_I32 = 1,
  ORACLE_KEY_F32 = 2,
  ORACLE_KEY_U64 = 3,
  ORACLE_KEY_I64 = 4,
  ORACLE_KEY_F64 = 5,
  ORACLE_KEY_U8 = 6,
  ORACLE_KEY_I8 = 7,
  ORACLE_KEY_U16 = 8,
  ORACLE_KEY_I16 = 9
};

enum {
  ORACLE_SET_UNION = 0,
  ORACLE_SET_INTERSECTION = 1,
  ORACLE_SET_DIFFERENCE = 2,
  ORACLE_SET_SYMMETRIC_DIFFERENCE = 3
};

uint64_t oracle_splitmix64(uint64_t x);

/* Order-preserving key -> bits transform (ascending or descending). */
uint64_t oracle_radix_ordered(int kind, int descending, uint64_t raw);
/* Ordered bits with the float ±0 collapse applied (what digits come from). */
uint64_t oracle_radix_digit_source(int kind, int descending, uint64_t raw);

/* Stable LSD radix sort over bits [begin_bit, end_bit) with 8-bit passes.
 * keys/values are sorted in place. Returns 0, or -1 for an invalid kind or
 * bit range. */
int oracle_radix_sort(int kind, int descending, void *keys, void *values,
                      size_t value_bytes, size_t n, unsigned begin_bit,
                      unsigned end_bit);

/* Stable two-way merge; on equal keys the first input comes first. */
int oracle_merge(int kind, int descending, const void *a_keys,
                 const void *a_values, size_t na, const void *b_keys,
                 const void *b_values, size_t nb, void *out_keys,
                 void *out_values, size_t value_bytes);

/* Stable comparison sort under natural order (or its reverse). */
int oracle_merge_sort(int kind, int descending, void *keys, void *values,
                      size_t value_bytes, size_t n);

/* Sorted multiset operation. out_keys == NULL counts only. Returns the
 * output length, or -1 on invalid arguments. */
long long oracle_set_op(int op, int kind, int descending, const void *a_keys,
                        const void *a_values, size_t na, const void *b_keys,
                        const void *b_values, size_t nb, void *out_keys,
                        void *out_values, size_t value_bytes);

/* Stable ascending lexicographic sort of n rows of `arity` u32 columns
 * (row-major), each row's payload (payload_bytes, may be 0) moving with it.
 * Returns 0, or -1 for an arity outside 2..6. */
int oracle_record_sort(unsigned arity, uint32_t *rows, void *payloads,
                       size_t payload_bytes, size_t n);

/* Reduce-by-key operators; numbering equals rccl_hip_group_op. */
enum {
  ORACLE_GROUP_NATURAL_BAG_ADD = 1,
  ORACLE_GROUP_BOOLEAN_OR = 2,
  ORACLE_GROUP_INDEPENDENT_PROBABILITY_OR = 3
};

/* Stable adjacent unique of n keys (`kind` scalars when arity == 1, rows of
 * `arity` u32 columns otherwise). Returns the number of runs, or -1. */
long long oracle_unique(int kind, unsigned arity, const void *in, void *out, size_t n);

/* Reduce by key: first key and left fold of the values of every run of equal
 * adjacent keys. Values are u64 (NATURAL_BAG_ADD), u8 (BOOLEAN_OR) or f64
 * (INDEPENDENT_PROBABILITY_OR). Returns the number of runs, or -1. */
long long oracle_reduce_by_key(int kind, unsigned arity, int op, const void *keys,
                               const void *values, void *out_keys, void *out_values, size_t n);

/* One INDEPENDENT_PROBABILITY_OR step. */
double oracle_prob_or(double l, double r);

#ifdef __cplusplus
}
#endif

#endif
