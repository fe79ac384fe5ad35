// CPU checks of the radix sort's pass planner (assign_plan) and workspace
// layout (layout), built from the library's own header (radix_plan.hpp) with
// AddressSanitizer and UndefinedBehaviorSanitizer by
// tests/test_radix_plan_native.py. Exit status 0 when every check passes;
// each failure prints the case.
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "radix_plan.hpp"

using namespace rccl_hip;
using namespace rccl_hip::radix;

static long g_failures = 0;

#define CHECK(cond, ...)                                                   \
  do {                                                                     \
    if (!(cond)) {                                                         \
      if (++g_failures <= 20) {                                            \
        std::printf("FAIL %s:%d %s | ", __FILE__, __LINE__, #cond);        \
        std::printf(__VA_ARGS__);                                          \
        std::printf("\n");                                                 \
      }                                                                    \
    }                                                                      \
  } while (0)

// Data flow of one stream through a plan. Buffers 0 (input), 1 (output) and
// 2 (scratch); an in-place stream's input and output are one buffer. Each
// buffer's content is the list of passes applied to the original input.
static void simulate(int P, uint32_t trivial, uint32_t flags, const PassPlan *plan,
                     bool in_place) {
  std::vector<int> content[3];
  auto storage = [&](uint32_t b) { return in_place && b == 1 ? 0u : b; };
  bool written_output = false;
  for (int p = 0; p < P; ++p) {
    const PassPlan &e = plan[p];
    if (!e.active) continue;
    const uint32_t s = storage(e.src), d = storage(e.dst);
    CHECK(s != d, "P=%d trivial=%#x flags=%u pass %d reads and writes one buffer (%u -> %u, in "
          "place %d)", P, trivial, flags, p, e.src, e.dst, in_place);
    std::vector<int> next = content[s];
    next.push_back(p);
    content[d] = next;
    if (e.dst == 1) written_output = true;
  }
  // The output holds every non-trivial pass, in order (trivial passes are
  // identity permutations and may appear in between).
  const std::vector<int> &out = content[storage(1)];
  std::vector<int> want;
  for (int p = 0; p < P; ++p)
    if (!(trivial >> p & 1u)) want.push_back(p);
  std::vector<int> got;
  for (int p : out)
    if (!(trivial >> p & 1u)) got.push_back(p);
  CHECK(got == want, "P=%d trivial=%#x flags=%u in place %d: output misses a pass", P, trivial,
        flags, in_place);
  for (size_t i = 1; i < out.size(); ++i)
    CHECK(out[i - 1] < out[i], "P=%d trivial=%#x flags=%u: passes out of order", P, trivial,
          flags);
  // A stream that is not in place must have its output written.
  if (!in_place)
    CHECK(written_output, "P=%d trivial=%#x flags=%u: a copied stream's output is never "
          "written", P, trivial, flags);
}

static void check_plan(int P, uint32_t trivial, uint32_t flags) {
  std::vector<PassPlan> plan(P + 1);
  plan[P] = PassPlan{0xdead, 0xdead, 0xdead, 0xdead, 0xdead};  // guard
  assign_plan(P, trivial, flags, plan.data());
  CHECK(plan[P].active == 0xdead, "P=%d: assign_plan wrote past P entries", P);
  int k = 0, first = -1, last = -1;
  uint32_t prev_dst = 0;
  for (int p = 0; p < P; ++p) {
    const PassPlan &e = plan[p];
    CHECK(e.active <= 1, "P=%d pass %d: active %u", P, p, e.active);
    if (!e.active) {
      CHECK(e.src == 0 && e.dst == 0 && e.lb == 0 && e.conv == 0,
            "P=%d trivial=%#x pass %d: inactive entry not cleared", P, trivial, p);
      CHECK(trivial >> p & 1u, "P=%d trivial=%#x flags=%u: non-trivial pass %d skipped", P,
            trivial, flags, p);
      continue;
    }
    if (first < 0) first = p;
    last = p;
    CHECK(e.src == (k == 0 ? 0u : prev_dst),
          "P=%d trivial=%#x flags=%u pass %d reads %u, not the previous output %u", P, trivial,
          flags, p, e.src, k == 0 ? 0u : prev_dst);
    CHECK(e.dst == 1 || e.dst == 2, "P=%d pass %d writes buffer %u", P, p, e.dst);
    CHECK(e.src != e.dst, "P=%d pass %d reads and writes buffer %u", P, p, e.dst);
    CHECK(e.lb == uint32_t(k & 1), "P=%d trivial=%#x pass %d look-back buffer %u, want %d", P,
          trivial, p, e.lb, k & 1);
    prev_dst = e.dst;
    ++k;
  }
  for (int p = 0; p < P; ++p) {
    const PassPlan &e = plan[p];
    if (!e.active) continue;
    const uint32_t want = (p == first ? CONV_IN : 0u) | (p == last ? CONV_OUT : 0u);
    CHECK(e.conv == want, "P=%d trivial=%#x flags=%u pass %d conv %u want %u", P, trivial, flags,
          p, e.conv, want);
  }
  if (k > 0) CHECK(prev_dst == 1, "P=%d trivial=%#x flags=%u: the last pass writes %u", P,
                   trivial, flags, prev_dst);
  if (flags & PLAN_IN_PLACE) {
    CHECK(k % 2 == 0, "P=%d trivial=%#x flags=%u: odd active count %d with a stream in place", P,
          trivial, flags, k);
    simulate(P, trivial, flags, plan.data(), true);
  }
  if ((flags & PLAN_COPIES) || flags == 0) {
    CHECK(k >= 1, "P=%d trivial=%#x flags=%u: no pass writes the copied output", P, trivial,
          flags);
    simulate(P, trivial, flags, plan.data(), false);
  }
}

static uint64_t g_rng = 0x9E3779B97F4A7C15ull;
static uint64_t next_rand() {
  uint64_t z = (g_rng += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static void check_plans() {
  // P = 4 and 8 (the merge-sort lowering of 32- and 64-bit keys) and 4N for
  // the record sort's N-word rows (N = 2..6): every trivial mask up to P = 16,
  // then structured and random masks.
  const int sizes[] = {4, 8, 12, 16, 20, 24};
  long plans = 0;
  for (int P : sizes) {
    const uint32_t all = (1u << P) - 1u;
    std::vector<uint32_t> masks;
    if (P <= 16) {
      for (uint32_t m = 0; m <= all; ++m) masks.push_back(m);
    } else {
      masks.push_back(0);
      masks.push_back(all);
      for (int p = 0; p < P; ++p) {
        masks.push_back(1u << p);
        masks.push_back(all & ~(1u << p));
        masks.push_back((1u << p) - 1u);
        masks.push_back(all & ~((1u << p) - 1u));
      }
      for (int i = 0; i < 200000; ++i) masks.push_back(uint32_t(next_rand()) & all);
    }
    for (uint32_t m : masks)
      for (uint32_t flags = 0; flags < 4; ++flags) {
        check_plan(P, m, flags);
        ++plans;
      }
  }
  std::printf("plans checked: %ld\n", plans);
}

// Layout arithmetic, recomputed in 128 bits: regions aligned and disjoint,
// sized for the tiles and groups of n items, and descriptor width switching
// at 2^30 items (30-bit look-back counts).
typedef unsigned __int128 u128;
static u128 up(u128 x, u128 a) { return (x + a - 1) / a * a; }

static void check_layout(size_t kb, size_t vb, size_t n, bool planned) {
  const Layout l = layout(kb, vb, n, planned);
  if (n == 0) {
    CHECK(l.total == 0, "n=0 total %zu", l.total);
    return;
  }
  const bool small = small_tiles(kb, vb, n, planned);
  const u128 tile = small ? small_tile_items(kb, vb) : tile_items(kb, vb);
  const u128 tiles = (u128(n) + tile - 1) / tile;
  const u128 groups = (tiles + GROUP - 1) / GROUP;
  const u128 desc = n < (size_t(1) << 30) ? 4 : 8;
  const u128 passes = kb;
  const u128 bins = up(passes * BINS * 4, 256);
  const u128 skew = up(passes * 4, 256);
  const u128 ginc = up(tiles * BINS * desc, 256);
  const u128 gagg = ginc + up(groups * BINS * desc, 256);
  const u128 ticket = gagg + up(groups * BINS * 4, 256);
  const u128 lb_bytes = ticket + up(XCDS * 4, 256);
  const u128 total = bins + skew + 2 * lb_bytes;
  CHECK(l.small == small && l.tiles == tiles && l.groups == groups && l.desc_bytes == desc,
        "kb=%zu vb=%zu n=%zu planned=%d: tiles %zu groups %zu desc %zu", kb, vb, n, planned,
        l.tiles, l.groups, l.desc_bytes);
  CHECK(tiles * tile >= n && (tiles - 1) * tile < n, "n=%zu: tiles do not cover n", n);
  CHECK(l.bins == 0 && l.skew == bins && l.lb[0] == bins + skew && l.lb[1] == l.lb[0] + lb_bytes,
        "kb=%zu vb=%zu n=%zu: region offsets", kb, vb, n);
  CHECK(l.lb_ginc == ginc && l.lb_gagg == gagg && l.lb_ticket == ticket &&
            l.lb_bytes == lb_bytes,
        "kb=%zu vb=%zu n=%zu: look-back regions", kb, vb, n);
  CHECK(l.total == total && total < (u128(1) << 63), "kb=%zu vb=%zu n=%zu: total %zu", kb, vb,
        n, l.total);
  CHECK(l.skew % 256 == 0 && l.lb[0] % 256 == 0 && l.lb[1] % 256 == 0 && l.lb_ginc % 256 == 0 &&
            l.lb_gagg % 256 == 0 && l.lb_ticket % 256 == 0 && l.lb_bytes % 256 == 0,
        "kb=%zu n=%zu: a region is not 256-byte aligned", kb, n);
  // Every digit count of the sort fits the descriptor's count field.
  CHECK(desc == 8 || n <= (size_t(1) << 30) - 1, "n=%zu: counts overflow 30 bits", n);
  // A planned sort's pass plan sits after the layout.
  CHECK(plan_bytes() >= passes * sizeof(PassPlan), "plan bytes");
}

static void check_layouts() {
  const size_t keys[] = {4, 8};
  const size_t values[] = {0, 1, 2, 4, 8, 16};
  long cases = 0;
  for (size_t kb : keys)
    for (size_t vb : values)
      for (int planned = 0; planned < 2; ++planned) {
        const size_t small_max =
            size_t(RCCL_RADIX_SMALL_MAX_TILES) * small_tile_items(kb, vb);
        const size_t tile = tile_items(kb, vb);
        const size_t ns[] = {0,           1,           2,           small_max - 1,
                             small_max,   small_max + 1, tile - 1,  tile,
                             tile + 1,    size_t(1) << 20, size_t(1) << 28,
                             (size_t(1) << 30) - 1, size_t(1) << 30, (size_t(1) << 30) + 1,
                             size_t(1) << 31, (size_t(1) << 32) - 2, (size_t(1) << 32) - 1};
        for (size_t n : ns) {
          check_layout(kb, vb, n, planned != 0);
          ++cases;
        }
      }
  std::printf("layouts checked: %ld\n", cases);
}

int main() {
  check_plans();
  check_layouts();
  if (g_failures) {
    std::printf("%ld failures\n", g_failures);
    return 1;
  }
  std::printf("all radix plan and layout checks passed\n");
  return 0;
}
