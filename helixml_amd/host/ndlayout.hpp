// ndlayout.hpp — the strides ndarray 0.15 gives a CpuTensor's array, for the HipTensor mirror.
//
// A CpuTensor (crates/backend-cpu/src/lib.rs) wraps an ndarray ArrayD, and some of its operations
// keep a non-row-major memory order: transpose is `permuted_axes(..).to_owned()` (lib.rs:115-137),
// which keeps the permuted strides; elementwise maps keep the input's strides; binary operations
// (`&a + &b`, lib.rs:570-632) collect in C or F order by ndarray's Zip layout preference. Two
// things depend on that order and so must be mirrored:
//   * mean (lib.rs:995-1010) sums an axis with ndarray's eight-accumulator lane fold when the axis
//     is the array's minimum-stride axis and the lane is a contiguous slice, and in axis order
//     otherwise, so the order decides the rounding;
//   * cat, stack and broadcast_to read `data.as_slice().unwrap()` (lib.rs:233-318, 413, 513,
//     1392-1492), which panics unless the array is in standard (row-major) layout.
// HipTensor data are always row-major on the device; these functions track the strides the
// reference's array would have, as metadata. They restate ndarray 0.15's published rules
// (dimension/mod.rs: default_strides, is_layout_c/f, min_stride_axis, reshape_dim_c;
// layout/mod.rs: array_layout, tendency; zip/mod.rs: prefer_f, map_collect; impl_methods.rs:
// to_owned, map, sum_axis). Host-only, header-only.
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <vector>

namespace helix {
namespace ndlayout {

using Dims = std::vector<size_t>;
using Strides = std::vector<int64_t>;

inline bool has_zero(const Dims& d) {
    for (size_t x : d)
        if (x == 0) return true;
    return false;
}

// Dimension::default_strides (row-major; all zero for an empty array)
inline Strides c_strides(const Dims& d) {
    Strides s(d.size(), 0);
    if (has_zero(d)) return s;
    int64_t acc = 1;
    for (size_t i = d.size(); i-- > 0;) {
        s[i] = acc;
        acc *= (int64_t)d[i];
    }
    return s;
}

// Dimension::fortran_strides
inline Strides f_strides(const Dims& d) {
    Strides s(d.size(), 0);
    if (has_zero(d)) return s;
    int64_t acc = 1;
    for (size_t i = 0; i < d.size(); ++i) {
        s[i] = acc;
        acc *= (int64_t)d[i];
    }
    return s;
}

// is_layout_c / is_layout_f: axes of length 1 may carry any stride
inline bool is_layout_c(const Dims& d, const Strides& s) {
    if (has_zero(d)) return true;
    int64_t c = 1;
    for (size_t i = d.size(); i-- > 0;)
        if (d[i] != 1) {
            if (s[i] != c) return false;
            c *= (int64_t)d[i];
        }
    return true;
}

inline bool is_layout_f(const Dims& d, const Strides& s) {
    if (has_zero(d)) return true;
    int64_t c = 1;
    for (size_t i = 0; i < d.size(); ++i)
        if (d[i] != 1) {
            if (s[i] != c) return false;
            c *= (int64_t)d[i];
        }
    return true;
}

// ArrayBase::is_standard_layout (what as_slice() requires) — the same test as is_layout_c
inline bool is_standard_layout(const Dims& d, const Strides& s) { return is_layout_c(d, s); }

// Dimension::is_contiguous (what as_slice_memory_order() requires): the strides, taken from the
// smallest up, step through one dense block
inline bool is_contiguous(const Dims& d, const Strides& s) {
    if (s == c_strides(d)) return true;
    if (d.size() == 1) return s[0] == -1;
    std::vector<size_t> order(d.size());
    for (size_t i = 0; i < order.size(); ++i) order[i] = i;
    // _fastest_varying_stride_order: a stable sort by |stride|
    for (size_t i = 1; i < order.size(); ++i)
        for (size_t j = i; j > 0 && std::llabs(s[order[j]]) < std::llabs(s[order[j - 1]]); --j) {
            const size_t t = order[j];
            order[j] = order[j - 1];
            order[j - 1] = t;
        }
    int64_t c = 1;
    for (size_t i : order) {
        if (d[i] != 1 && std::llabs(s[i]) != c) return false;
        c *= (int64_t)d[i];
    }
    return true;
}

enum : unsigned { kCOrder = 1u, kFOrder = 2u, kCPrefer = 4u, kFPrefer = 8u };

// array_layout
inline unsigned array_layout(const Dims& d, const Strides& s) {
    const size_t n = d.size();
    if (is_layout_c(d, s)) {
        size_t long_axes = 0;
        for (size_t x : d) long_axes += x > 1;
        if (n <= 1 || long_axes <= 1) return kCOrder | kFOrder | kCPrefer | kFPrefer;
        return kCOrder | kCPrefer;
    }
    if (n > 1 && is_layout_f(d, s)) return kFOrder | kFPrefer;
    if (n > 1) {
        if (d[0] > 1 && s[0] == 1) return kFPrefer;
        if (d[n - 1] > 1 && s[n - 1] == 1) return kCPrefer;
    }
    return 0u;
}

inline int tendency(unsigned l) {
    return (int)((l & kCOrder) != 0) - (int)((l & kFOrder) != 0) + (int)((l & kCPrefer) != 0) -
           (int)((l & kFPrefer) != 0);
}

// Zip::map_collect over parts of one shape: the output is F-ordered when the Zip prefers F
// (no common C order, and a common F order or a negative summed tendency), else row-major.
inline Strides collect(const Dims& d, const std::vector<Strides>& parts) {
    unsigned lay = ~0u;
    int t = 0;
    for (const Strides& p : parts) {
        const unsigned l = array_layout(d, p);
        lay &= l;
        t += tendency(l);
    }
    const bool prefer_f = !(lay & kCOrder) && ((lay & kFOrder) || t < 0);
    return prefer_f ? f_strides(d) : c_strides(d);
}

// Dimension::min_stride_axis: the axis of least |stride|; ties go to the later axis
inline size_t min_stride_axis(const Dims& d, const Strides& s) {
    if (d.size() <= 1) return 0;
    size_t best = d.size() - 1;
    for (size_t i = d.size(); i-- > 0;)
        if (std::llabs(s[i]) < std::llabs(s[best])) best = i;
    return best;
}

// How mean_axis sums axis `ax` (sum_axis): with the lane fold when the axis is the minimum-stride
// axis and its lanes are contiguous slices (stride +-1, or at most one element), else in axis
// order (subviews added one by one into zeros, or the lanes' sequential fold).
inline bool sums_with_lane_fold(const Dims& d, const Strides& s, size_t ax) {
    if (ax != min_stride_axis(d, s)) return false;
    return d[ax] <= 1 || s[ax] == 1 || s[ax] == -1;
}

inline Dims remove_axis(const Dims& d, size_t ax) {
    Dims r(d);
    r.erase(r.begin() + (long)ax);
    return r;
}

inline Strides remove_axis(const Strides& s, size_t ax) {
    Strides r(s);
    r.erase(r.begin() + (long)ax);
    return r;
}

// Strides of mean_axis(ax)'s result: the lane path collects over the remaining axes' view (one
// part), the axis-order path accumulates into a row-major zeros array; the division by the count
// is in place.
inline Strides mean_axis_result(const Dims& d, const Strides& s, size_t ax) {
    const Dims rd = remove_axis(d, ax);
    if (ax == min_stride_axis(d, s)) return collect(rd, {remove_axis(s, ax)});
    return c_strides(rd);
}

// transpose: permuted_axes swaps two strides; to_owned keeps them (the array is contiguous in
// memory order)
inline Strides transposed(const Strides& s, size_t a, size_t b) {
    Strides r(s);
    const int64_t t = r[a];
    r[a] = r[b];
    r[b] = t;
    return r;
}

// to_owned of a view: its strides when the view is contiguous in memory order, else row-major
inline Strides owned(const Dims& d, const Strides& s) { return is_contiguous(d, s) ? s : c_strides(d); }

// reshape (lib.rs:94-113: to_shape in row-major order, then to_owned): the view strides
// reshape_dim_c finds when the new shape can be read from the old strides without a copy, else
// a row-major copy. `ok` is false when no view exists.
inline Strides reshape_view_c(const Dims& from, const Strides& strides, const Dims& to, bool* ok) {
    Strides ts(to.size(), 0);
    *ok = false;
    size_t fi = 0, ti = 0;
    while (fi < from.size() && ti < to.size()) {
        int64_t fd = (int64_t)from[fi], fs = strides[fi], td = (int64_t)to[ti];
        if (fd == td) {
            ts[ti] = strides[fi];
            ++fi;
            ++ti;
            continue;
        }
        if (fd == 1) {
            ++fi;
            continue;
        }
        if (td == 1) {
            ts[ti] = 1;
            ++ti;
            continue;
        }
        if (fd == 0 || td == 0) return ts;
        int64_t whole = fs * fd, fprod = fd, tprod = td;
        while (fprod != tprod) {
            if (fprod < tprod) {
                if (++fi >= from.size()) return ts;
                fd = (int64_t)from[fi];
                fprod *= fd;
                if (fd > 1) {
                    const int64_t old = fs;
                    fs = strides[fi];
                    if (old != fd * fs) return ts;  // not contiguous together: needs a copy
                }
            } else {
                whole /= td;
                ts[ti] = whole;
                if (++ti >= to.size()) return ts;
                td = (int64_t)to[ti];
                tprod *= td;
            }
        }
        whole /= td;
        ts[ti] = whole;
        ++fi;
        ++ti;
    }
    while (fi < from.size() && from[fi] == 1) ++fi;
    while (ti < to.size() && to[ti] == 1) {
        ts[ti] = 1;
        ++ti;
    }
    if (fi < from.size() || ti < to.size()) return ts;
    *ok = true;
    return ts;
}

inline Strides reshaped(const Dims& from, const Strides& s, const Dims& to) {
    size_t n = 1;
    for (size_t x : to) n *= x;
    if (n == 0) return c_strides(to);  // an empty array reshapes as a row-major view
    bool ok = false;
    const Strides v = reshape_view_c(from, s, to, &ok);
    return ok ? owned(to, v) : c_strides(to);
}

}  // namespace ndlayout
}  // namespace helix
