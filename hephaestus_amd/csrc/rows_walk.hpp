// Division-free walks of strided views as rows, shared by the full
// reductions and the map-reductions.  A view (RowsView, built on the host)
// is `rows` rows of `cols` elements under up to three outer dimensions;
// threads walk it in units -- 16-byte vectors of 4 elements when rows are
// contiguous, single elements otherwise -- tracking two linear forms over
// the row digits: `off`, the element offset of the walked operand, and
// `off2`, a second form (a logical index, or a second operand's offset).
#pragma once

#include "hx_device.hpp"
#include "hx_internal.hpp"

namespace hx {

// Unit u of a row sits at element u * ustride (form 1) and u * ustride2
// (form 2).  The walker's step of `step` units is split on the host into
// whole rows (as outer digits, innermost first, with their offsets
// step_off / step_off2) and leftover units (step_units, step_uoff /
// step_uoff2), so a step is adds and compares only.  ospan[k] =
// oshape[k] * ostride[k], and the same for form 2.
struct RowsGeom {
    uint64_t rows, cols, units;
    int64_t ustride, units_span, cstride2, ustride2, units_span2;
    uint32_t orank;
    uint64_t oshape[3];
    int64_t ostride[3], ospan[3], ostride2[3], ospan2[3];
    uint64_t step_units, step_rows;
    uint64_t step_digits[3];
    int64_t step_uoff, step_off, step_uoff2, step_off2;
};

// Walks a thread's units of a RowsGeom view: unit `item` is unit
// item % units of row item / units.  Divisions only at the start; each
// advance adds the precomputed step with carries.  `off` and `off2` are
// the two forms at the walker's unit.
struct RowWalker {
    uint64_t unit;
    uint64_t dig[3]; // outer digits of the row, innermost first (the outermost unwrapped)
    int64_t off, off2;
    __device__ __forceinline__ void init(const RowsGeom &g, int64_t base, int64_t base2, uint64_t item) {
        const uint64_t row = item / g.units;
        unit = item - row * g.units;
        off = base + (int64_t)unit * g.ustride;
        off2 = base2 + (int64_t)unit * g.ustride2;
        uint64_t r = row;
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            if ((uint32_t)k + 1 < g.orank) {
                const uint64_t q = r / g.oshape[k];
                dig[k] = r - q * g.oshape[k];
                r = q;
            } else {
                dig[k] = r;
                r = 0;
            }
            if ((uint32_t)k < g.orank) {
                off += (int64_t)dig[k] * g.ostride[k];
                off2 += (int64_t)dig[k] * g.ostride2[k];
            }
        }
    }
    __device__ __forceinline__ void advance(const RowsGeom &g) {
        unit += g.step_units;
        off += g.step_uoff + g.step_off;
        off2 += g.step_uoff2 + g.step_off2;
        uint64_t carry = 0;
        if (unit >= g.units) {
            unit -= g.units;
            off -= g.units_span;
            off2 -= g.units_span2;
            carry = 1;
        }
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            if ((uint32_t)k < g.orank) {
                dig[k] += g.step_digits[k] + carry;
                if (carry) {
                    off += g.ostride[k];
                    off2 += g.ostride2[k];
                }
                carry = 0;
                if ((uint32_t)k + 1 < g.orank && dig[k] >= g.oshape[k]) {
                    dig[k] -= g.oshape[k];
                    off -= g.ospan[k];
                    off2 -= g.ospan2[k];
                    carry = 1;
                }
            }
        }
    }
};

// The walker geometry of a row view: units per row (vectors of 4 elements
// or single elements) and a step of `step` units as whole rows, outer
// digits of those rows (innermost first; the outermost unwrapped) and
// leftover units.
inline RowsGeom rows_geom(const RowsView &v, bool vec, uint64_t step) {
    RowsGeom g{};
    g.rows = v.rows;
    g.cols = v.cols;
    g.units = vec ? ceil_div(v.cols, 4) : v.cols;
    g.ustride = vec ? 4 : v.cstride;
    g.units_span = (int64_t)g.units * g.ustride;
    g.cstride2 = v.cstride2;
    g.ustride2 = vec ? 4 * v.cstride2 : v.cstride2;
    g.units_span2 = (int64_t)g.units * g.ustride2;
    g.orank = v.orank;
    for (int k = 0; k < 3; ++k) {
        g.oshape[k] = v.oshape[k];
        g.ostride[k] = v.ostride[k];
        g.ospan[k] = (int64_t)v.oshape[k] * v.ostride[k];
        g.ostride2[k] = v.ostride2[k];
        g.ospan2[k] = (int64_t)v.oshape[k] * v.ostride2[k];
    }
    g.step_units = step % g.units;
    g.step_rows = step / g.units;
    g.step_uoff = (int64_t)g.step_units * g.ustride;
    g.step_uoff2 = (int64_t)g.step_units * g.ustride2;
    uint64_t r = g.step_rows;
    for (uint32_t k = 0; k < 3; ++k) {
        if (k + 1 < g.orank) {
            g.step_digits[k] = r % g.oshape[k];
            r /= g.oshape[k];
        } else if (k + 1 == g.orank) {
            g.step_digits[k] = r;
            r = 0;
        } else {
            g.step_digits[k] = 0;
        }
        if (k < g.orank) {
            g.step_off += (int64_t)g.step_digits[k] * g.ostride[k];
            g.step_off2 += (int64_t)g.step_digits[k] * g.ostride2[k];
        }
    }
    return g;
}

} // namespace hx
