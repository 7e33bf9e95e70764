"""A model of libstdc++'s std::sort (bits/stl_algo.h: __introsort_loop, __unguarded_partition_pivot,
__final_insertion_sort, the heap steps of __partial_sort) over (key, index) pairs with ATen's descending comparator,
and McIlroy's adversary against it: writes tests/golden/sort_killers.npz, keys whose sort reaches the heapsort branch
(the depth limit exhausted), for tests/test_aten_sort.py. The model equals torch.argsort(descending=True) on the CPU
(checked here for each written case). Test data generation only.

Usage:  python tests/golden/make_sort_killers.py
"""
import math

import numpy as np
import torch

def comp(a, b):  # descending (key, idx) by key: NaN first, then larger
    ka, kb = a[0], b[0]
    return (math.isnan(ka) and not math.isnan(kb)) or ka > kb

def unguarded_linear_insert(v, last):
    val = v[last]; nxt = last - 1
    while comp(val, v[nxt]):
        v[last] = v[nxt]; last = nxt; nxt -= 1
    v[last] = val

def insertion_sort(v, first, last):
    if first == last: return
    for i in range(first + 1, last):
        if comp(v[i], v[first]):
            val = v[i]
            v[first + 1:i + 1] = v[first:i]
            v[first] = val
        else:
            unguarded_linear_insert(v, i)

def final_insertion_sort(v, first, last):
    if last - first > 16:
        insertion_sort(v, first, first + 16)
        for i in range(first + 16, last): unguarded_linear_insert(v, i)
    else:
        insertion_sort(v, first, last)

def move_median_to_first(v, result, a, b, c):
    if comp(v[a], v[b]):
        if comp(v[b], v[c]): v[result], v[b] = v[b], v[result]
        elif comp(v[a], v[c]): v[result], v[c] = v[c], v[result]
        else: v[result], v[a] = v[a], v[result]
    elif comp(v[a], v[c]): v[result], v[a] = v[a], v[result]
    elif comp(v[b], v[c]): v[result], v[c] = v[c], v[result]
    else: v[result], v[b] = v[b], v[result]

def unguarded_partition(v, first, last, pivot):
    while True:
        while comp(v[first], v[pivot]): first += 1
        last -= 1
        while comp(v[pivot], v[last]): last -= 1
        if not (first < last): return first
        v[first], v[last] = v[last], v[first]
        first += 1

# heap helpers (std::__adjust_heap / __push_heap / __make_heap / __pop_heap)
def push_heap(v, first, hole, top, value):
    parent = (hole - 1) // 2
    while hole > top and comp(v[first + parent], value):
        v[first + hole] = v[first + parent]; hole = parent; parent = (hole - 1) // 2
    v[first + hole] = value

def adjust_heap(v, first, hole, length, value):
    top = hole; second = hole
    while second < (length - 1) // 2:
        second = 2 * (second + 1)
        if comp(v[first + second], v[first + second - 1]): second -= 1
        v[first + hole] = v[first + second]; hole = second
    if (length & 1) == 0 and second == (length - 2) // 2:
        second = 2 * (second + 1)
        v[first + hole] = v[first + second - 1]; hole = second - 1
    push_heap(v, first, hole, top, value)

def make_heap(v, first, last):
    length = last - first
    if length < 2: return
    parent = (length - 2) // 2
    while True:
        value = v[first + parent]
        adjust_heap(v, first, parent, length, value)
        if parent == 0: return
        parent -= 1

def pop_heap(v, first, last, result):
    value = v[result]; v[result] = v[first]
    adjust_heap(v, first, 0, last - first, value)

def heap_select(v, first, middle, last):
    make_heap(v, first, middle)
    for i in range(middle, last):
        if comp(v[i], v[first]): pop_heap(v, first, middle, i)

def sort_heap(v, first, last):
    while last - first > 1:
        last -= 1
        pop_heap(v, first, last, last)

def introsort_loop(v, first, last, depth):
    while last - first > 16:
        if depth == 0:
            heap_select(v, first, last, last); sort_heap(v, first, last); return
        depth -= 1
        mid = first + (last - first) // 2
        move_median_to_first(v, first, first + 1, mid, last - 1)
        cut = unguarded_partition(v, first + 1, last, first)
        introsort_loop(v, cut, last, depth)
        last = cut

def std_sort_desc(keys):
    v = [(float(k), i) for i, k in enumerate(keys)]
    n = len(v)
    if n:
        introsort_loop(v, 0, n, 2 * (n.bit_length() - 1))
        final_insertion_sort(v, 0, n)
    return [i for _, i in v]



def killer(n):
    """McIlroy's adversary ("A killer adversary for quicksort", Software: Practice and Experience 29(4), 1999): the
    keys are fixed lazily as the sort compares them, so that every median-of-three pivot is near the end of its range
    and the depth limit runs out (the heapsort branch); the items never fixed stay equal (ties)."""
    global comp
    gas = n
    val = [gas] * n
    state = {"solid": 0, "cand": 0}

    def lazy(a, b):
        x, y = a[1], b[1]
        if val[x] == gas and val[y] == gas:
            if x == state["cand"]:
                val[x] = state["solid"]
            else:
                val[y] = state["solid"]
            state["solid"] += 1
        if val[x] == gas:
            state["cand"] = x
        elif val[y] == gas:
            state["cand"] = y
        return -val[x] > -val[y]
    saved, comp = comp, lazy
    try:
        v = [(0.0, i) for i in range(n)]
        introsort_loop(v, 0, n, 2 * (n.bit_length() - 1))
    finally:
        comp = saved
    return np.array([-(x if x != gas else n + 1) for x in val], dtype=np.float32)


def heap_hits(keys):
    """Times the introsort of keys falls back to heapsort."""
    global heap_select
    hits = [0]
    saved = heap_select

    def counted(*a):
        hits[0] += 1
        return saved(*a)
    heap_select = counted
    try:
        std_sort_desc(keys)
    finally:
        heap_select = saved
    return hits[0]


if __name__ == "__main__":
    import os
    out = {}
    for n in (64, 128, 256):
        k = killer(n)
        assert heap_hits(k.tolist()) > 0 and std_sort_desc(k.tolist()) == torch.from_numpy(k).argsort(
            -1, descending=True).tolist()
        out[f"n{n}"] = k
    np.savez_compressed(os.path.join(os.path.dirname(os.path.abspath(__file__)), "sort_killers.npz"), **out)
    print("sort killers written", {k: v.shape for k, v in out.items()})
