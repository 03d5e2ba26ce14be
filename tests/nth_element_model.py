"""A plain-Python restatement of libstdc++'s std::nth_element (bits/stl_algo.h __introselect,
bits/stl_heap.h) for unique, comparable keys — a second, independent statement of the
algorithm the CPU oracle calls and the device restates (test infrastructure only).

MLX's CPU argpartition runs it on the index vector 0..n-1 with the comparator (value, index);
with keys (value, index) the comparisons are the same."""


def _adjust_heap(b, hole, length, value):
    top = hole
    child = hole
    while child < (length - 1) // 2:
        child = 2 * (child + 1)
        if b[child] < b[child - 1]:
            child -= 1
        b[hole] = b[child]
        hole = child
    if length % 2 == 0 and child == (length - 2) // 2:
        child = 2 * (child + 1)
        b[hole] = b[child - 1]
        hole = child - 1
    parent = (hole - 1) // 2
    while hole > top and b[parent] < value:
        b[hole] = b[parent]
        hole = parent
        parent = (hole - 1) // 2
    b[hole] = value


def _heap_select(a, first, middle, last):
    heap = a[first:middle]
    n = len(heap)
    if n >= 2:
        parent = (n - 2) // 2
        while True:
            _adjust_heap(heap, parent, n, heap[parent])
            if parent == 0:
                break
            parent -= 1
    for i in range(middle, last):
        if a[i] < heap[0]:
            v = a[i]
            a[i] = heap[0]
            _adjust_heap(heap, 0, n, v)
    a[first:middle] = heap


def nth_element(keys, nth):
    """Returns (list after std::nth_element(first, first + nth, last), whether the heap
    selection ran).  Scanning-pointer Hoare partition, as written in the library."""
    a = list(keys)
    n = len(a)
    if n == 0 or nth >= n:
        return a, False
    first, last = 0, n
    depth = 2 * (n.bit_length() - 1)
    while last - first > 3:
        if depth == 0:
            _heap_select(a, first, nth + 1, last)
            a[first], a[nth] = a[nth], a[first]
            return a, True
        depth -= 1
        mid = first + (last - first) // 2
        x, y, z = first + 1, mid, last - 1
        if a[x] < a[y]:
            m = y if a[y] < a[z] else (z if a[x] < a[z] else x)
        else:
            m = x if a[x] < a[z] else (z if a[y] < a[z] else y)
        a[first], a[m] = a[m], a[first]
        pivot = a[first]
        lo, hi = first + 1, last
        while True:
            while a[lo] < pivot:
                lo += 1
            hi -= 1
            while pivot < a[hi]:
                hi -= 1
            if not lo < hi:
                break
            a[lo], a[hi] = a[hi], a[lo]
            lo += 1
        cut = lo
        if cut <= nth:
            first = cut
        else:
            last = cut
    for i in range(first + 1, last):  # insertion sort
        v = a[i]
        j = i
        while j > first and v < a[j - 1]:
            a[j] = a[j - 1]
            j -= 1
        a[j] = v
    return a, False


def argpartition_slice(values, k):
    """MLX CPU argpartition(values, kth = n - k)[n - k:] for one row of comparable values."""
    n = len(values)
    keys = [(v, i) for i, v in enumerate(values)]
    out, _ = nth_element(keys, n - k)
    return [i for _, i in out[n - k:]]
