/*
 * CPU restatement of the reference's ordering semantics.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg. The product never links or calls it.
 * Reference paths below are relative to the StarGazerM/rccl tree.
 *
 * Pinning (tests/test_oracle.py): every function is checked against the
 * reference's literal probe/test vectors (tests/golden/reference_vectors.json)
 * and against an independent restatement (numpy key transform + stable
 * argsort, heapq.merge, sorted, multiset algebra with a per-run value rule).
 * Parity unpinned: NaN keys in oracle_merge, oracle_merge_sort and
 * oracle_set_op (IEEE '<' makes NaN equivalent to every key, so the result
 * depends on the merge and balanced paths; no reference vector covers it).
 * Radix order of NaN bit patterns is pinned.
 */
#include "oracle.h"

#include <stdlib.h>
#include <string.h>

/* splitmix64 (Steele, Lea, Flood 2014), as used by the reference's set-op
 * benchmark input generator: benchmarks/set-operations-reference.cu:116-122. */
uint64_t oracle_splitmix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ull;
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}

static int kind_bytes(int kind) {
  switch (kind) {
  case ORACLE_KEY_U32: case ORACLE_KEY_I32: case ORACLE_KEY_F32: return 4;
  case ORACLE_KEY_U64: case ORACLE_KEY_I64: case ORACLE_KEY_F64: return 8;
  case ORACLE_KEY_U8: case ORACLE_KEY_I8: return 1;
  case ORACLE_KEY_U16: case ORACLE_KEY_I16: return 2;
  default: return 0;
  }
}

static int is_radix_kind(int kind) { return kind >= ORACLE_KEY_U32 && kind <= ORACLE_KEY_F64; }

/* Key transforms: rccl-cub/src/ordering_backend/radix.rs:75-235.
 *   unsigned: identity; signed: flip the sign bit;
 *   float: negative -> all bits inverted, otherwise sign bit flipped;
 *   descending: bitwise complement of the ascending bits. */
uint64_t oracle_radix_ordered(int kind, int descending, uint64_t raw) {
  uint64_t asc;
  uint64_t mask;
  switch (kind) {
  case ORACLE_KEY_U32: asc = raw & 0xffffffffull; mask = 0xffffffffull; break;
  case ORACLE_KEY_I32: asc = (raw ^ 0x80000000ull) & 0xffffffffull; mask = 0xffffffffull; break;
  case ORACLE_KEY_F32:
    raw &= 0xffffffffull;
    asc = (raw & 0x80000000ull) ? (~raw & 0xffffffffull) : (raw ^ 0x80000000ull);
    mask = 0xffffffffull;
    break;
  case ORACLE_KEY_U64: asc = raw; mask = ~0ull; break;
  case ORACLE_KEY_I64: asc = raw ^ 0x8000000000000000ull; mask = ~0ull; break;
  case ORACLE_KEY_F64:
    asc = (raw & 0x8000000000000000ull) ? ~raw : (raw ^ 0x8000000000000000ull);
    mask = ~0ull;
    break;
  default: return 0;
  }
  return descending ? (~asc & mask) : asc;
}

/* Digit source with the ±0 collapse: rccl-cub/src/ordering_backend/radix.rs:257-337
 * (radix_float_digit_masked_u32/u64). The ordered value 0x7fff..ff (-0.0
 * ascending, +0.0 descending) is replaced by 0x8000..00 (the other zero), so
 * the two zeros share every digit and keep input order. */
uint64_t oracle_radix_digit_source(int kind, int descending, uint64_t raw) {
  uint64_t ordered = oracle_radix_ordered(kind, descending, raw);
  if (kind == ORACLE_KEY_F32 && ordered == 0x7fffffffull) return 0x80000000ull;
  if (kind == ORACLE_KEY_F64 && ordered == 0x7fffffffffffffffull) return 0x8000000000000000ull;
  return ordered;
}

static uint64_t load_raw(const void *base, size_t i, int bytes) {
  const unsigned char *p = (const unsigned char *)base + i * (size_t)bytes;
  switch (bytes) {
  case 1: return *(const uint8_t *)p;
  case 2: { uint16_t v; memcpy(&v, p, 2); return v; }
  case 4: { uint32_t v; memcpy(&v, p, 4); return v; }
  default: { uint64_t v; memcpy(&v, p, 8); return v; }
  }
}

static void gather(void *base, size_t elem, const size_t *perm, size_t n) {
  if (!base || elem == 0 || n == 0) return;
  unsigned char *tmp = (unsigned char *)malloc(n * elem);
  const unsigned char *src = (const unsigned char *)base;
  for (size_t i = 0; i < n; ++i) memcpy(tmp + i * elem, src + perm[i] * elem, elem);
  memcpy(base, tmp, n * elem);
  free(tmp);
}

/* Stable LSD radix sort. Pass structure from rccl-cub/src/radix.rs:364-386
 * (passes = ceil((end-begin)/8)) and :518-552 (pass p sorts the digit at
 * bit begin+8p, width min(8, end-bit)); each pass is a stable counting sort,
 * which is what the onesweep pass computes
 * (rccl-cub/src/ordering_backend/radix.rs:1029-1312). */
int oracle_radix_sort(int kind, int descending, void *keys, void *values,
                      size_t value_bytes, size_t n, unsigned begin_bit,
                      unsigned end_bit) {
  if (!is_radix_kind(kind)) return -1;
  int kb = kind_bytes(kind);
  unsigned key_bits = (unsigned)kb * 8u;
  if (begin_bit > end_bit || end_bit > key_bits) return -1;
  unsigned passes = (end_bit - begin_bit + 7u) / 8u;
  if (n == 0 || passes == 0) return 0;

  uint64_t *src = (uint64_t *)malloc(n * sizeof(uint64_t));
  uint64_t *src2 = (uint64_t *)malloc(n * sizeof(uint64_t));
  size_t *perm = (size_t *)malloc(n * sizeof(size_t));
  size_t *perm2 = (size_t *)malloc(n * sizeof(size_t));
  for (size_t i = 0; i < n; ++i) {
    src[i] = oracle_radix_digit_source(kind, descending, load_raw(keys, i, kb));
    perm[i] = i;
  }
  for (unsigned p = 0; p < passes; ++p) {
    unsigned bit = begin_bit + 8u * p;
    unsigned width = end_bit - bit < 8u ? end_bit - bit : 8u;
    uint64_t mask = (1ull << width) - 1ull;
    size_t count[257];
    memset(count, 0, sizeof(count));
    for (size_t i = 0; i < n; ++i) count[((src[i] >> bit) & mask) + 1]++;
    for (int d = 0; d < 256; ++d) count[d + 1] += count[d];
    for (size_t i = 0; i < n; ++i) {
      size_t dst = count[(src[i] >> bit) & mask]++;
      src2[dst] = src[i];
      perm2[dst] = perm[i];
    }
    uint64_t *ts = src; src = src2; src2 = ts;
    size_t *tp = perm; perm = perm2; perm2 = tp;
  }
  gather(keys, (size_t)kb, perm, n);
  gather(values, value_bytes, perm, n);
  free(src); free(src2); free(perm); free(perm2);
  return 0;
}

/* Natural order per key kind, the comparator Thrust passes for the
 * closure-free calls: rccl-thrust/src/merge.rs:169-178 and set.rs:16-25
 * (Less iff left < right, Greater iff right < left, else Equal). Floats use
 * IEEE `<`, so -0.0 and +0.0 are equivalent. Descending is the reversed
 * comparator `|a, b| b.cmp(a)`. */
#define DEFINE_LESS(NAME, T)                                                    \
  static int NAME(const void *x, size_t i, const void *y, size_t j, int desc) { \
    T a = ((const T *)x)[i];                                                    \
    T b = ((const T *)y)[j];                                                    \
    return desc ? (b < a) : (a < b);                                            \
  }
DEFINE_LESS(less_u32, uint32_t)
DEFINE_LESS(less_i32, int32_t)
DEFINE_LESS(less_f32, float)
DEFINE_LESS(less_u64, uint64_t)
DEFINE_LESS(less_i64, int64_t)
DEFINE_LESS(less_f64, double)
DEFINE_LESS(less_u8, uint8_t)
DEFINE_LESS(less_i8, int8_t)
DEFINE_LESS(less_u16, uint16_t)
DEFINE_LESS(less_i16, int16_t)

typedef int (*less_fn)(const void *, size_t, const void *, size_t, int);

static less_fn less_for(int kind) {
  switch (kind) {
  case ORACLE_KEY_U32: return less_u32;
  case ORACLE_KEY_I32: return less_i32;
  case ORACLE_KEY_F32: return less_f32;
  case ORACLE_KEY_U64: return less_u64;
  case ORACLE_KEY_I64: return less_i64;
  case ORACLE_KEY_F64: return less_f64;
  case ORACLE_KEY_U8: return less_u8;
  case ORACLE_KEY_I8: return less_i8;
  case ORACLE_KEY_U16: return less_u16;
  case ORACLE_KEY_I16: return less_i16;
  default: return 0;
  }
}

/* Two-pointer merge: rccl-cub/examples/device_ordering_probe.rs:89-102 (take
 * the first input unless the second is strictly before it), which is the
 * merge-path tie rule of rccl-memory/src/device.rs:59-63 and
 * rccl-cub/src/ordering_backend/merge.rs:240-246. */
int oracle_merge(int kind, int descending, const void *a_keys,
                 const void *a_values, size_t na, const void *b_keys,
                 const void *b_values, size_t nb, void *out_keys,
                 void *out_values, size_t value_bytes) {
  less_fn less = less_for(kind);
  int kb = kind_bytes(kind);
  if (!less) return -1;
  size_t i = 0, j = 0, o = 0;
  unsigned char *ok = (unsigned char *)out_keys;
  unsigned char *ov = (unsigned char *)out_values;
  while (i < na || j < nb) {
    int take_b = (i == na) || (j < nb && less(b_keys, j, a_keys, i, descending));
    const void *sk = take_b ? b_keys : a_keys;
    const void *sv = take_b ? b_values : a_values;
    size_t si = take_b ? j++ : i++;
    memcpy(ok + o * kb, (const unsigned char *)sk + si * kb, kb);
    if (value_bytes && ov)
      memcpy(ov + o * value_bytes, (const unsigned char *)sv + si * value_bytes, value_bytes);
    ++o;
  }
  return 0;
}

/* Stable comparison sort: DeviceMergeSort is a stable merge sort
 * (rccl-cub/src/ordering_backend/merge.rs:1128-1262, stable odd-even block
 * sort then merge rounds that prefer the left run on ties). Restated as a
 * bottom-up merge sort of an index permutation. */
int oracle_merge_sort(int kind, int descending, void *keys, void *values,
                      size_t value_bytes, size_t n) {
  less_fn less = less_for(kind);
  int kb = kind_bytes(kind);
  if (!less) return -1;
  if (n < 2) return 0;
  size_t *perm = (size_t *)malloc(n * sizeof(size_t));
  size_t *tmp = (size_t *)malloc(n * sizeof(size_t));
  for (size_t i = 0; i < n; ++i) perm[i] = i;
  for (size_t width = 1; width < n; width *= 2) {
    for (size_t lo = 0; lo < n; lo += 2 * width) {
      size_t mid = lo + width < n ? lo + width : n;
      size_t hi = lo + 2 * width < n ? lo + 2 * width : n;
      size_t i = lo, j = mid, o = lo;
      while (i < mid || j < hi) {
        int take_right = (i == mid) || (j < hi && less(keys, perm[j], keys, perm[i], descending));
        tmp[o++] = take_right ? perm[j++] : perm[i++];
      }
    }
    size_t *t = perm; perm = tmp; tmp = t;
  }
  gather(keys, (size_t)kb, perm, n);
  gather(values, value_bytes, perm, n);
  free(perm);
  free(tmp);
  return 0;
}

/* Relation-row sort: the reference's record sort
 * (rccl-thrust/src/record_sort.rs:88-126,144-366) orders [u32; N] rows by the
 * unrolled unsigned lexicographic comparator (:88-115) with a stable merge
 * sort, arity 2..6; a payload row moves with its key row. Restated as a
 * bottom-up stable merge sort of row indices, then a gather. */
static int row_less(const uint32_t *rows, unsigned arity, size_t x, size_t y) {
  const uint32_t *a = rows + x * arity, *b = rows + y * arity;
  for (unsigned c = 0; c < arity; ++c)
    if (a[c] != b[c]) return a[c] < b[c];
  return 0;
}

int oracle_record_sort(unsigned arity, uint32_t *rows, void *payloads, size_t payload_bytes,
                       size_t n) {
  if (arity < 2 || arity > 6) return -1;
  if (n < 2) return 0;
  size_t *perm = (size_t *)malloc(n * sizeof(size_t));
  size_t *tmp = (size_t *)malloc(n * sizeof(size_t));
  for (size_t i = 0; i < n; ++i) perm[i] = i;
  for (size_t width = 1; width < n; width *= 2) {
    for (size_t lo = 0; lo < n; lo += 2 * width) {
      size_t mid = lo + width < n ? lo + width : n;
      size_t hi = lo + 2 * width < n ? lo + 2 * width : n;
      size_t i = lo, j = mid, o = lo;
      while (i < mid || j < hi) {
        int take_right = (i == mid) || (j < hi && row_less(rows, arity, perm[j], perm[i]));
        tmp[o++] = take_right ? perm[j++] : perm[i++];
      }
    }
    size_t *t = perm; perm = tmp; tmp = t;
  }
  gather(rows, (size_t)arity * sizeof(uint32_t), perm, n);
  gather(payloads, payload_bytes, perm, n);
  free(perm);
  free(tmp);
  return 0;
}

/* Sorted multiset operations: the reference's own host oracle
 * rccl-thrust/examples/set_operations_tests.rs:40-107 (host_set_by), whose
 * selections match the serial device operations of
 * rccl-cub/src/ordering_backend/set.rs:564-827: union emits A on ties and B
 * only when B is strictly first; intersection emits A; difference emits
 * unmatched A; symmetric difference emits unmatched elements of either side.
 * Values always come from the side whose key is emitted. */
long long oracle_set_op(int op, int kind, int descending, const void *a_keys,
                        const void *a_values, size_t na, const void *b_keys,
                        const void *b_values, size_t nb, void *out_keys,
                        void *out_values, size_t value_bytes) {
  less_fn less = less_for(kind);
  int kb = kind_bytes(kind);
  if (!less || op < 0 || op > 3) return -1;
  size_t a = 0, b = 0;
  long long o = 0;
  unsigned char *ok = (unsigned char *)out_keys;
  unsigned char *ov = (unsigned char *)out_values;
#define EMIT(KEYS, VALS, IDX)                                                        \
  do {                                                                               \
    if (ok) memcpy(ok + (size_t)o * kb, (const unsigned char *)(KEYS) + (IDX) * kb, kb); \
    if (ok && ov && value_bytes && (VALS))                                           \
      memcpy(ov + (size_t)o * value_bytes,                                           \
             (const unsigned char *)(VALS) + (IDX) * value_bytes, value_bytes);      \
    ++o;                                                                             \
  } while (0)
  while (a < na && b < nb) {
    int first_before = less(a_keys, a, b_keys, b, descending);
    int second_before = less(b_keys, b, a_keys, a, descending);
    switch (op) {
    case ORACLE_SET_UNION:
      if (second_before) { EMIT(b_keys, b_values, b); ++b; }
      else { EMIT(a_keys, a_values, a); ++a; if (!first_before) ++b; }
      break;
    case ORACLE_SET_INTERSECTION:
      if (first_before) ++a;
      else if (second_before) ++b;
      else { EMIT(a_keys, a_values, a); ++a; ++b; }
      break;
    case ORACLE_SET_DIFFERENCE:
      if (first_before) { EMIT(a_keys, a_values, a); ++a; }
      else if (second_before) ++b;
      else { ++a; ++b; }
      break;
    default:
      if (first_before) { EMIT(a_keys, a_values, a); ++a; }
      else if (second_before) { EMIT(b_keys, b_values, b); ++b; }
      else { ++a; ++b; }
      break;
    }
  }
  if (op == ORACLE_SET_UNION || op == ORACLE_SET_SYMMETRIC_DIFFERENCE) {
    for (; a < na; ++a) EMIT(a_keys, a_values, a);
    for (; b < nb; ++b) EMIT(b_keys, b_values, b);
  } else if (op == ORACLE_SET_DIFFERENCE) {
    for (; a < na; ++a) EMIT(a_keys, a_values, a);
  }
#undef EMIT
  return o;
}

/* Adjacent-run compactions: rccl-cub/src/compaction_kernels.rs:64-93 (an item
 * starts a run when it is first or not equivalent to its predecessor),
 * :95-131 (stable scatter of the heads) and :180-236 (one left fold per run,
 * in index order), with the natural equivalence: == on the key's value
 * (floats by IEEE ==), every column for rows. */
static int key_equal(int kind, unsigned arity, const void *keys, size_t i, size_t j) {
  if (arity > 1) {
    const uint32_t *r = (const uint32_t *)keys;
    for (unsigned c = 0; c < arity; ++c)
      if (r[i * arity + c] != r[j * arity + c]) return 0;
    return 1;
  }
  switch (kind) {
  case ORACLE_KEY_F32: return ((const float *)keys)[i] == ((const float *)keys)[j];
  case ORACLE_KEY_F64: return ((const double *)keys)[i] == ((const double *)keys)[j];
  default: {
    const int kb = kind_bytes(kind);
    return memcmp((const char *)keys + i * kb, (const char *)keys + j * kb, (size_t)kb) == 0;
  }
  }
}

static size_t key_width(int kind, unsigned arity) {
  return arity > 1 ? (size_t)arity * 4u : (size_t)kind_bytes(kind);
}

static int valid_key(int kind, unsigned arity) {
  if (arity == 1) return kind_bytes(kind) > 0;
  return kind == ORACLE_KEY_U32 && arity >= 2 && arity <= 6;
}

long long oracle_unique(int kind, unsigned arity, const void *in, void *out, size_t n) {
  if (!valid_key(kind, arity)) return -1;
  const size_t kb = key_width(kind, arity);
  size_t count = 0;
  for (size_t i = 0; i < n; ++i) {
    if (i == 0 || !key_equal(kind, arity, in, i - 1, i)) {
      memcpy((char *)out + count * kb, (const char *)in + i * kb, kb);
      ++count;
    }
  }
  return (long long)count;
}

/* The sealed operators of rccl-cub/src/grouped_reduction.rs:17-75. */
static uint64_t bag_add(uint64_t l, uint64_t r) { return l + r; }
static uint8_t bool_or(uint8_t l, uint8_t r) { return (l != 0 || r != 0) ? 1 : 0; }
static double prob_or(double l, double r) {
  /* (l + r) - (l * r), each step rounded (built with -ffp-contract=off). */
  volatile double s = l + r;
  volatile double p = l * r;
  double c = s - p;
  if (c < 0.0) return 0.0;
  if (c > 1.0) return 1.0;
  return c;
}

long long oracle_reduce_by_key(int kind, unsigned arity, int op, const void *keys,
                               const void *values, void *out_keys, void *out_values, size_t n) {
  if (!valid_key(kind, arity) || op < ORACLE_GROUP_NATURAL_BAG_ADD ||
      op > ORACLE_GROUP_INDEPENDENT_PROBABILITY_OR)
    return -1;
  const size_t kb = key_width(kind, arity);
  size_t count = 0;
  size_t i = 0;
  while (i < n) {
    size_t j = i + 1;
    while (j < n && key_equal(kind, arity, keys, j - 1, j)) ++j;
    memcpy((char *)out_keys + count * kb, (const char *)keys + i * kb, kb);
    if (op == ORACLE_GROUP_NATURAL_BAG_ADD) {
      const uint64_t *v = (const uint64_t *)values;
      uint64_t agg = v[i];
      for (size_t k = i + 1; k < j; ++k) agg = bag_add(agg, v[k]);
      ((uint64_t *)out_values)[count] = agg;
    } else if (op == ORACLE_GROUP_BOOLEAN_OR) {
      const uint8_t *v = (const uint8_t *)values;
      uint8_t agg = v[i];
      for (size_t k = i + 1; k < j; ++k) agg = bool_or(agg, v[k]);
      ((uint8_t *)out_values)[count] = agg;
    } else {
      const double *v = (const double *)values;
      double agg = v[i];
      for (size_t k = i + 1; k < j; ++k) agg = prob_or(agg, v[k]);
      ((double *)out_values)[count] = agg;
    }
    ++count;
    i = j;
  }
  return (long long)count;
}

/* One operator step, for the known-answer tests. */
double oracle_prob_or(double l, double r) { return prob_or(l, r); }
