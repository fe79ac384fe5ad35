"""The radix sort's tile policy (rccl_amd/csrc/radix_kernels.hpp), restated
for tests that must land on either side of the small-tile threshold. A CPU
test (test_host_cpu.py) checks it against the library's workspace sizes."""

SMALL_THREADS = 256
SMALL_MAX_TILES = 512


def items(key_bytes, value_bytes):
    """Items per thread of a large tile."""
    if value_bytes == 0:
        return 34 if key_bytes <= 4 else 17
    stage = max(key_bytes, value_bytes)
    return 28 if stage <= 4 else (16 if stage <= 8 else 8)


def small_tile_max(key_bytes, value_bytes):
    """Largest plain sort that uses the small tiles."""
    return SMALL_MAX_TILES * SMALL_THREADS * max(1, items(key_bytes, value_bytes) // 2)
