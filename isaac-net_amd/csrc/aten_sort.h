// The order of torch's CPU argsort(descending=True) over float keys, as the reference's retransmission admission
// ranks its candidates (isaac_net/core/mac.py:301, 307): ATen sorts (key, index) pairs with libstdc++'s std::sort and a
// descending comparator (a NaN key before any other, then the larger key first). std::sort is an introsort: while a
// range holds more than 16 elements, a median-of-three quicksort step (the median of the second, middle and last
// elements moved to the front, then an unguarded Hoare partition), or heapsort once the depth limit 2 floor(log2 n)
// is spent; then one insertion sort over the whole array (guarded over the first 16 elements, unguarded after). The
// order of equal keys is whatever those steps leave, not the index order, so an exact ranking with ties has to repeat
// them step for step. Ranges are independent once partitioned, so the quicksort recursion runs here from an explicit
// stack of ranges (in any order: each range's steps touch only its own elements).
//
// Plain C++ (host and device): the same header is compiled into the step kernels and, by the CPU tests, with g++
// against torch.argsort.
#pragma once

#ifndef INET_HD
#if defined(__HIPCC__)
#define INET_HD __host__ __device__
#else
#define INET_HD
#endif
#endif

namespace inet {

// std::sort over n (key, index) pairs, keys k[], indices v[] (in place), descending with NaN first. stk: room for
// 3 * (2 floor(log2 n) + 2) ints (the pending ranges and their depth budgets).
struct AtenSortDesc {
    float* k;
    int* v;
    INET_HD static bool comp(float a, float b) { return (a != a && b == b) || a > b; }
    INET_HD bool lt(int i, int j) const { return comp(k[i], k[j]); }
    INET_HD void swap_(int i, int j) const {
        const float tk = k[i]; k[i] = k[j]; k[j] = tk;
        const int tv = v[i]; v[i] = v[j]; v[j] = tv;
    }
    // __unguarded_linear_insert: the element at `last` moved down past every element it compares before
    INET_HD void linear_insert(int last) const {
        const float vk = k[last];
        const int vv = v[last];
        int nxt = last - 1;
        while (comp(vk, k[nxt])) {
            k[last] = k[nxt]; v[last] = v[nxt];
            last = nxt;
            --nxt;
        }
        k[last] = vk; v[last] = vv;
    }
    // __insertion_sort over [first, last)
    INET_HD void insertion_sort(int first, int last) const {
        if (first == last) return;
        for (int i = first + 1; i < last; ++i) {
            if (lt(i, first)) {
                const float vk = k[i];
                const int vv = v[i];
                for (int j = i; j > first; --j) { k[j] = k[j - 1]; v[j] = v[j - 1]; }
                k[first] = vk; v[first] = vv;
            } else {
                linear_insert(i);
            }
        }
    }
    // __move_median_to_first(result, a, b, c)
    INET_HD void median_to_first(int result, int a, int b, int c) const {
        if (lt(a, b)) {
            if (lt(b, c)) swap_(result, b);
            else if (lt(a, c)) swap_(result, c);
            else swap_(result, a);
        } else if (lt(a, c)) {
            swap_(result, a);
        } else if (lt(b, c)) {
            swap_(result, c);
        } else {
            swap_(result, b);
        }
    }
    // __unguarded_partition(first, last, pivot)
    INET_HD int partition(int first, int last, int pivot) const {
        while (true) {
            while (lt(first, pivot)) ++first;
            --last;
            while (lt(pivot, last)) --last;
            if (!(first < last)) return first;
            swap_(first, last);
            ++first;
        }
    }
    // heap steps of __partial_sort(first, last, last): __make_heap, __pop_heap, __adjust_heap, __push_heap (the heap is
    // over [first, first + len), element i at first + i)
    INET_HD void push_heap(int first, int hole, int top, float vk, int vv) const {
        int parent = (hole - 1) / 2;
        while (hole > top && comp(k[first + parent], vk)) {
            k[first + hole] = k[first + parent]; v[first + hole] = v[first + parent];
            hole = parent;
            parent = (hole - 1) / 2;
        }
        k[first + hole] = vk; v[first + hole] = vv;
    }
    INET_HD void adjust_heap(int first, int hole, int len, float vk, int vv) const {
        const int top = hole;
        int second = hole;
        while (second < (len - 1) / 2) {
            second = 2 * (second + 1);
            if (lt(first + second, first + second - 1)) --second;
            k[first + hole] = k[first + second]; v[first + hole] = v[first + second];
            hole = second;
        }
        if ((len & 1) == 0 && second == (len - 2) / 2) {
            second = 2 * (second + 1);
            k[first + hole] = k[first + second - 1]; v[first + hole] = v[first + second - 1];
            hole = second - 1;
        }
        push_heap(first, hole, top, vk, vv);
    }
    INET_HD void pop_heap(int first, int last, int result) const {
        const float vk = k[result];
        const int vv = v[result];
        k[result] = k[first]; v[result] = v[first];
        adjust_heap(first, 0, last - first, vk, vv);
    }
    INET_HD void heap_sort(int first, int last) const {
        const int len = last - first;
        if (len >= 2) {                                  // __make_heap
            for (int parent = (len - 2) / 2;; --parent) {
                adjust_heap(first, parent, len, k[first + parent], v[first + parent]);
                if (parent == 0) break;
            }
        }
        // (__heap_select with middle == last compares nothing more)
        while (last - first > 1) {                       // __sort_heap
            --last;
            pop_heap(first, last, last);
        }
    }
    INET_HD void sort(int n, int* stk) const {
        if (n <= 1) return;
        int lg = 0;
        while ((2 << lg) <= n) ++lg;                     // floor(log2 n)
        int top = 0;
        stk[0] = 0; stk[1] = n; stk[2] = 2 * lg;
        top = 1;
        while (top > 0) {
            --top;
            int first = stk[3 * top], last = stk[3 * top + 1], depth = stk[3 * top + 2];
            while (last - first > 16) {                  // __introsort_loop
                if (depth == 0) { heap_sort(first, last); break; }
                --depth;
                const int mid = first + (last - first) / 2;
                median_to_first(first, first + 1, mid, last - 1);
                const int cut = partition(first + 1, last, first);
                stk[3 * top] = cut; stk[3 * top + 1] = last; stk[3 * top + 2] = depth;   // the right range, later
                ++top;
                last = cut;
            }
        }
        if (n > 16) {                                    // __final_insertion_sort
            insertion_sort(0, 16);
            for (int i = 16; i < n; ++i) linear_insert(i);
        } else {
            insertion_sort(0, n);
        }
    }
};

}  // namespace inet
