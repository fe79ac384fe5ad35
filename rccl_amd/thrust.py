"""Python mirror of the reference's rccl-thrust ordering facade over the C ABI.

Names, routing and error behaviour follow rccl-thrust (paths relative to the
StarGazerM/rccl tree):
  Program.load / Program.par           rccl-thrust/src/cuda.rs:85-109
  sort, sort_unstable (natural order)  ordering.rs:13-44  -> radix sort, ascending
  sort_by, sort_unstable_by (closure)  ordering.rs:13-44  -> stable merge sort
  view().with_values(..)               range.rs:100-163, ordering.rs:96-129
  a.merge(b).write_into(out, exec)     merge.rs:16-247
  arithmetic_range(..).difference(..)  set.rs:127-244,477-690 (unmaterialised inputs)
  a.union(b).write_into / .count       set.rs:357-898 (also intersection,
                                       difference, symmetric_difference)
  unique_copy_by, unique_by            compaction.rs:224-378
  reduce_by_key + NaturalBagAdd,       grouped_reduction.rs:102-216
    BooleanOr, IndependentProbabilityOr
Every call allocates its temporary workspace on the device, runs on the
execution's stream and synchronizes before returning, as Thrust's
synchronous policy does (rccl-thrust/src/backend.rs:8-150).
"""
from __future__ import annotations

import numpy as np
import torch

from . import _abi, cub
from ._abi import DeviceAlgorithmError  # noqa: F401  (re-export)
from .device import DeviceBuffer, kind_of

ascending = cub.ascending
descending = cub.descending


class Program:
    """Loaded kernel program for one device."""

    def __init__(self, inner: cub.Program):
        self._inner = inner

    @staticmethod
    def load(device: int = 0) -> "Program":
        return Program(cub.Program.load(device))

    @property
    def device(self) -> int:
        return self._inner.device

    def par(self, stream: torch.cuda.Stream | None = None) -> "Execution":
        return Execution(self._inner.on(stream))


class Execution:
    """A synchronous execution policy bound to one stream."""

    def __init__(self, launch: cub.Launch):
        self._launch = launch

    def launch(self) -> cub.Launch:
        return self._launch

    def synchronize(self) -> None:
        self._launch.synchronize()


# ---------------------------------------------------------------------------
# Views.
# ---------------------------------------------------------------------------
class _SortMethodsForward:
    """Sort methods of a mutable view (the reference calls them on the
    DeviceBuffer itself: rccl-thrust/src/ordering.rs:46-89)."""

    def sort_unstable(self, execution: "Execution") -> None:
        sort_unstable(self, execution)

    def sort(self, execution: "Execution") -> None:
        sort(self, execution)

    def sort_unstable_by(self, execution: "Execution", order) -> None:
        sort_unstable_by(self, execution, order)

    def sort_by(self, execution: "Execution", order) -> None:
        sort_by(self, execution, order)


class DeviceView:
    def __init__(self, buffer: DeviceBuffer):
        self.buffer = buffer

    def len(self) -> int:
        return self.buffer.len()

    def with_values(self, values: "DeviceView | DeviceBuffer") -> "KeyValueRange":
        values = values if isinstance(values, DeviceView) else DeviceView(values)
        if values.len() != self.len():
            cub._check_len("values", self.len(), values.len())
        return KeyValueRange(self, values)

    def merge(self, second: "DeviceView") -> "_Merge":
        return _Merge(self, second, ascending)

    def merge_by(self, second: "DeviceView", order) -> "_Merge":
        return _Merge(self, second, order)

    def union(self, second):
        return _SetExpression("union", self, second, ascending)

    def union_by(self, second, order):
        return _SetExpression("union", self, second, order)

    def intersection(self, second):
        return _SetExpression("intersection", self, second, ascending)

    def intersection_by(self, second, order):
        return _SetExpression("intersection", self, second, order)

    def difference(self, second):
        return _SetExpression("difference", self, second, ascending)

    def difference_by(self, second, order):
        return _SetExpression("difference", self, second, order)

    def symmetric_difference(self, second):
        return _SetExpression("symmetric_difference", self, second, ascending)

    def symmetric_difference_by(self, second, order):
        return _SetExpression("symmetric_difference", self, second, order)


class DeviceViewMut(DeviceView, _SortMethodsForward):
    def as_view(self) -> DeviceView:
        return DeviceView(self.buffer)

    def with_values(self, values) -> "KeyValueRangeMut":
        values = values if isinstance(values, DeviceView) else DeviceView(values)
        if values.len() != self.len():
            cub._check_len("values", self.len(), values.len())
        return KeyValueRangeMut(self, values)


class KeyValueRange:
    """Structure-of-arrays keys plus values; orderings examine keys only."""

    def __init__(self, keys: DeviceView, values: DeviceView):
        self.keys = keys
        self.values = values

    def len(self) -> int:
        return self.keys.len()

    def merge(self, second: "KeyValueRange") -> "_Merge":
        return _Merge(self, second, ascending)

    def merge_by(self, second: "KeyValueRange", order) -> "_Merge":
        return _Merge(self, second, order)

    def union(self, second):
        return _SetExpression("union", self, second, ascending)

    def union_by(self, second, order):
        return _SetExpression("union", self, second, order)

    def intersection(self, second):
        return _SetExpression("intersection", self, second, ascending)

    def intersection_by(self, second, order):
        return _SetExpression("intersection", self, second, order)

    def difference(self, second):
        return _SetExpression("difference", self, second, ascending)

    def difference_by(self, second, order):
        return _SetExpression("difference", self, second, order)

    def symmetric_difference(self, second):
        return _SetExpression("symmetric_difference", self, second, ascending)

    def symmetric_difference_by(self, second, order):
        return _SetExpression("symmetric_difference", self, second, order)


class _SortMethods:
    """DeviceSortExt / DeviceKeyValueSortExt (rccl-thrust/src/ordering.rs:13-182):
    natural-order sorts take the radix sort, comparator sorts the stable
    merge sort; every call synchronizes."""

    def sort_unstable(self, execution: "Execution") -> None:
        sort_unstable(self, execution)

    def sort(self, execution: "Execution") -> None:
        sort(self, execution)

    def sort_unstable_by(self, execution: "Execution", order) -> None:
        sort_unstable_by(self, execution, order)

    def sort_by(self, execution: "Execution", order) -> None:
        sort_by(self, execution, order)


class KeyValueRangeMut(KeyValueRange, _SortMethods):
    pass


class ArithmeticRange(cub.ArithmeticRange):
    """An unmaterialised arithmetic range with the fluent set operations of
    ArithmeticSetRangeExt (rccl-thrust/src/set.rs:544-690). Both sides of an
    expression are arithmetic ranges of the same item type."""

    def union(self, second):
        return _SetExpression("union", self, second, ascending)

    def union_by(self, second, order):
        return _SetExpression("union", self, second, order)

    def intersection(self, second):
        return _SetExpression("intersection", self, second, ascending)

    def intersection_by(self, second, order):
        return _SetExpression("intersection", self, second, order)

    def difference(self, second):
        return _SetExpression("difference", self, second, ascending)

    def difference_by(self, second, order):
        return _SetExpression("difference", self, second, order)

    def symmetric_difference(self, second):
        return _SetExpression("symmetric_difference", self, second, ascending)

    def symmetric_difference_by(self, second, order):
        return _SetExpression("symmetric_difference", self, second, order)


def arithmetic_range(start, step, length: int, dtype=None) -> ArithmeticRange:
    """rccl_thrust::arithmetic_range (rccl-cub/src/range.rs:76-78)."""
    return ArithmeticRange(start, step, length, dtype)


def view(buffer: DeviceBuffer) -> DeviceView:
    return DeviceView(buffer)


def view_mut(buffer: DeviceBuffer) -> DeviceViewMut:
    return DeviceViewMut(buffer)


# ---------------------------------------------------------------------------
# Sorting (rccl-thrust/src/ordering.rs, backend.rs).
# ---------------------------------------------------------------------------
def _split(target):
    if isinstance(target, KeyValueRange):
        return target.keys.buffer, target.values.buffer
    if isinstance(target, DeviceView):
        return target.buffer, None
    return target, None


def _radix(execution: Execution, target) -> None:
    keys, values = _split(target)
    launch = execution.launch()
    if values is None:
        ws = cub.device_radix_sort_workspace(launch, keys.dtype, keys.len())
        cub.device_radix_sort_keys(launch, keys, ws)
    else:
        ws = cub.device_radix_sort_pairs_workspace(launch, keys.dtype, values.dtype, keys.len())
        cub.device_radix_sort_pairs(launch, keys, values, ws)
    execution.synchronize()


def _merge_sort(execution: Execution, target, order) -> None:
    keys, values = _split(target)
    cub.order_code(order, keys.dtype)  # rejects an unsupported closure before any allocation
    launch = execution.launch()
    if values is None:
        ws = cub.device_merge_sort_workspace(launch, keys.dtype, keys.len())
        cub.device_merge_sort_keys(launch, keys, ws, order)
    else:
        ws = cub.device_merge_sort_pairs_workspace(launch, keys.dtype, values.dtype, keys.len())
        cub.device_merge_sort_pairs(launch, keys, values, ws, order)
    execution.synchronize()


def sort_unstable(target, execution: Execution) -> None:
    """Natural-order sort (radix, ascending)."""
    _radix(execution, target)


def sort(target, execution: Execution) -> None:
    """Stable natural-order sort (radix sort is stable)."""
    _radix(execution, target)


def sort_unstable_by(target, execution: Execution, order) -> None:
    """Sort by a comparator (stable merge sort)."""
    _merge_sort(execution, target, order)


def sort_by(target, execution: Execution, order) -> None:
    """Stable sort by a comparator (merge sort)."""
    _merge_sort(execution, target, order)


# ---------------------------------------------------------------------------
# Merge and set expressions (rccl-thrust/src/merge.rs, set.rs).
# ---------------------------------------------------------------------------
class _Merge:
    def __init__(self, first, second, order):
        self.first, self.second, self.order = first, second, order

    def write_into(self, output, execution: Execution) -> None:
        launch = execution.launch()
        ak, av = _split(self.first)
        bk, bv = _split(self.second)
        ok, ov = _split(output)
        if av is None:
            ws = cub.device_merge_workspace(launch, ak.dtype, ak.len(), bk.len())
            cub.device_merge_keys(launch, ak, bk, ws, ok, self.order)
        else:
            ws = cub.device_merge_pairs_workspace(launch, ak.dtype, av.dtype, ak.len(), bk.len())
            cub.device_merge_pairs(launch, ak, av, bk, bv, ws, ok, ov, self.order)
        execution.synchronize()


class _SetExpression:
    def __init__(self, operation, first, second, order):
        self.operation, self.first, self.second, self.order = operation, first, second, order

    def _run(self, output, execution: Execution) -> int:
        launch = execution.launch()
        if isinstance(self.first, cub.ArithmeticRange):
            # rccl-thrust/src/set.rs:127-244: both sides arithmetic, keys only.
            if not isinstance(self.second, cub.ArithmeticRange):
                raise TypeError("an arithmetic range combines with an arithmetic range")
            if self.first.len() + self.second.len() == 0:
                return 0
            ok = None if output is None else _split(output)[0]
            ws = cub.device_set_workspace(launch, self.operation, self.first.dtype,
                                          self.first.len(), self.second.len())
            cub.device_set_arithmetic(launch, self.operation, self.first, self.second, ws, ok,
                                      self.order)
            return ws.count()
        ak, av = _split(self.first)
        bk, bv = _split(self.second)
        ok, ov = (None, None) if output is None else _split(output)
        if ak.len() + bk.len() == 0:
            return 0  # rccl-thrust/src/set.rs:44-46: empty inputs return 0 without launching
        if av is None or ok is None:
            ws = cub.device_set_workspace(launch, self.operation, ak.dtype, ak.len(), bk.len())
            cub.device_set_keys(launch, self.operation, ak, bk, ws, ok, self.order)
        else:
            ws = cub.device_set_pairs_workspace(launch, self.operation, ak.dtype, av.dtype,
                                                ak.len(), bk.len())
            cub.device_set_pairs(launch, self.operation, ak, av, bk, bv, ws, ok, ov, self.order)
        return ws.count()  # reads the device count back (synchronizes)

    def write_into(self, output, execution: Execution) -> int:
        """Write the result and return its length."""
        return self._run(output, execution)

    def count(self, execution: Execution) -> int:
        """Execute the operation without materializing its keys."""
        return self._run(None, execution)


# ---------------------------------------------------------------------------
# Adjacent-run compaction (rccl-thrust/src/compaction.rs:224-378,
# grouped_reduction.rs:102-216).
# ---------------------------------------------------------------------------
# The natural equivalence, |a, b| a == b (on keys; key/value ranges compare by
# key). Other closures have no kernels.
equal = "equal"


class NaturalBagAdd:
    """u64 wrapping addition (rccl-cub/src/grouped_reduction.rs:22-31)."""
    code, dtype = _abi.GROUP_OPS["natural_bag_add"], np.dtype(np.uint64)


class BooleanOr:
    """BooleanProvenance (one byte) disjunction (grouped_reduction.rs:49-57)."""
    code, dtype = _abi.GROUP_OPS["boolean_or"], np.dtype(np.uint8)


class IndependentProbabilityOr:
    """f64 l + r - l * r, clamped to [0, 1] (grouped_reduction.rs:59-75)."""
    code, dtype = _abi.GROUP_OPS["independent_probability_or"], np.dtype(np.float64)


def _check_equivalent(equivalent):
    if equivalent is not equal and equivalent is not None:
        raise ValueError("only the natural equivalence (thrust.equal) has device kernels")


def _group_keys(rng):
    """(key kind code, arity, keys buffer, payload buffer | None) of a key
    range: a DeviceBuffer / view of scalars, a RowBuffer of rows, or a
    key/value range (keys compared, values carried as the key's payload)."""
    from .record_sort import RowBuffer

    payload = None
    if isinstance(rng, KeyValueRange):
        payload = rng.values.buffer
        rng = rng.keys
    elif isinstance(rng, tuple):
        rng, payload = rng
        payload = payload.buffer if isinstance(payload, DeviceView) else payload
    if isinstance(rng, DeviceView):
        rng = rng.buffer
    if isinstance(rng, RowBuffer):
        return _abi.KEY_KINDS["u32"], rng.arity, rng, payload
    return _abi.KEY_KINDS[kind_of(rng.dtype)], 1, rng, payload


def _capacity(role, needed, actual):
    if actual < needed:
        info = _abi.ErrorInfo()
        info.status, info.role, info.expected, info.actual = 2, role.encode(), needed, actual
        raise DeviceAlgorithmError(2, info)


def _count_buffer(count, role):
    _capacity(role, 1, count.len())


def _group_workspace(execution, kind, arity, op, pb, n):
    nbytes = _abi.workspace_bytes("rccl_hip_group_workspace_bytes", kind, arity, op, pb, n)
    return DeviceBuffer.bytes(nbytes, execution.launch().program.device), nbytes


def _unique(execution, kind, arity, keys, pay, out_keys, out_pay, n, count):
    pb = 0 if pay is None else pay.dtype.itemsize
    ws, nbytes = _group_workspace(execution, kind, arity, _abi.GROUP_UNIQUE, pb, n)
    _abi.check(_abi.load().rccl_hip_unique_copy(
        kind, arity, pb, keys.ptr, None if pay is None else pay.ptr, out_keys.ptr,
        None if out_pay is None else out_pay.ptr, n, count.ptr, ws.ptr, nbytes,
        execution.launch().handle))


def unique_copy_by(execution, input, output, selected_count, equivalent=equal):
    """Stably copy the first item of every run of equivalent adjacent items
    into output's prefix; the number kept lands in selected_count[0]."""
    _check_equivalent(equivalent)
    kind, arity, keys, pay = _group_keys(input)
    _, o_arity, out_keys, out_pay = _group_keys(output)
    n = keys.len()
    _capacity("unique-copy output", n, out_keys.len())
    if (pay is None) != (out_pay is None):
        raise TypeError("input and output must both carry values or neither")
    if pay is not None:
        _capacity("unique-copy output", n, out_pay.len())
    _count_buffer(selected_count, "selected-count output")
    _unique(execution, kind, arity, keys, pay, out_keys, out_pay, n, selected_count)
    execution.synchronize()


def unique_by(execution, values, scratch, selected_count, equivalent=equal):
    """In-place adjacent unique: values' prefix holds the first item of every
    run, the rest of values is left as it was; scratch (same length) is
    overwritten."""
    _check_equivalent(equivalent)
    kind, arity, keys, pay = _group_keys(values)
    _, _, s_keys, s_pay = _group_keys(scratch)
    n = keys.len()
    _capacity("unique scratch", n, s_keys.len())
    if s_keys.len() != n:
        cub._check_len("unique scratch", n, s_keys.len())
    _count_buffer(selected_count, "selected-count output")
    # The values are copied to the scratch on the execution's stream, then
    # compacted from the scratch back into the values.
    with torch.cuda.stream(execution.launch().stream()):
        if arity > 1:
            s_keys.words.tensor.copy_(keys.words.tensor)
        else:
            s_keys.tensor.copy_(keys.tensor)
        if pay is not None:
            s_pay.tensor.copy_(pay.tensor)
    _unique(execution, kind, arity, s_keys, s_pay, keys, pay, n, selected_count)
    execution.synchronize()


def reduce_by_key(execution, keys, values, output_keys, output_values, group_count,
                  equivalent=equal, operator=NaturalBagAdd):
    """For every run of equivalent adjacent keys: its first key (and key
    payload) and the left fold of its values with `operator`; the number of
    runs lands in group_count[0]."""
    _check_equivalent(equivalent)
    kind, arity, k, kp = _group_keys(keys)
    _, _, ok, okp = _group_keys(output_keys)
    vals = values.buffer if isinstance(values, DeviceView) else values
    outv = output_values.buffer if isinstance(output_values, DeviceView) else output_values
    n = k.len()
    if vals.len() != n:
        cub._check_len("reduce-by-key values", n, vals.len())
    _capacity("reduce-by-key key output", n, ok.len())
    _capacity("reduce-by-key aggregate output", n, outv.len())
    _count_buffer(group_count, "group-count output")
    if vals.dtype != operator.dtype or outv.dtype != operator.dtype:
        raise TypeError(f"{operator.__name__} reduces {operator.dtype} values")
    pb = 0 if kp is None else kp.dtype.itemsize
    ws, nbytes = _group_workspace(execution, kind, arity, operator.code, pb, n)
    _abi.check(_abi.load().rccl_hip_reduce_by_key(
        kind, arity, operator.code, pb, k.ptr, None if kp is None else kp.ptr, vals.ptr, ok.ptr,
        None if okp is None else okp.ptr, outv.ptr, n, group_count.ptr, ws.ptr, nbytes,
        execution.launch().handle))
    execution.synchronize()


# ---------------------------------------------------------------------------
# Vectorized binary search: thrust::lower_bound / upper_bound over a range of
# values (no counterpart in the reference, CCCL_RUST_CAPABILITY_CHECKLIST.md:107).
# ---------------------------------------------------------------------------
def _bound(execution, haystack, needles, output, order, upper):
    from .record_sort import RowBuffer

    h = haystack.buffer if isinstance(haystack, DeviceView) else haystack
    q = needles.buffer if isinstance(needles, DeviceView) else needles
    out = output.buffer if isinstance(output, DeviceView) else output
    if isinstance(h, RowBuffer):
        if not isinstance(q, RowBuffer) or q.arity != h.arity:
            raise TypeError("needles must be rows of the haystack's arity")
        kind, arity = _abi.KEY_KINDS["u32"], h.arity
    else:
        if q.dtype != h.dtype:
            raise TypeError("needles and haystack must have the same item type")
        kind, arity = _abi.KEY_KINDS[kind_of(h.dtype)], 1
    if out.dtype != np.dtype(np.uint64):
        raise TypeError("bound indices are u64")
    _capacity("bound-search output", q.len(), out.len())
    nbytes = _abi.workspace_bytes("rccl_hip_bound_search_workspace_bytes", kind, arity, h.len())
    ws = DeviceBuffer.bytes(nbytes, execution.launch().program.device)
    _abi.check(_abi.load().rccl_hip_bound_search(
        kind, arity, cub.order_code(order, np.uint32 if arity > 1 else h.dtype), int(upper), h.ptr,
        h.len(), q.ptr, q.len(), out.ptr,
        ws.ptr, nbytes, execution.launch().handle))
    execution.synchronize()


def lower_bound(execution, haystack, needles, output, order=ascending):
    """output[i] = first index j of the sorted haystack with !(h[j] < needles[i])."""
    _bound(execution, haystack, needles, output, order, False)


def upper_bound(execution, haystack, needles, output, order=ascending):
    """output[i] = first index j of the sorted haystack with needles[i] < h[j]."""
    _bound(execution, haystack, needles, output, order, True)
