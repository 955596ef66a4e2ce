// Attention mask rules shared by every kernel, as plain integer code: device
// functions when compiled as HIP, ordinary inline functions otherwise, so that
// host tests can check them exhaustively (tests/cxx/mask_check.cpp).
#pragma once

#include <cstdint>

#if defined(__HIP__)
#define RDNA_MASK_FN __host__ __device__ __forceinline__
#else
#define RDNA_MASK_FN inline
#endif

namespace rdna_amd {

RDNA_MASK_FN int mask_imin(int a, int b) {
    return a < b ? a : b;
}
RDNA_MASK_FN int mask_imax(int a, int b) {
    return a > b ? a : b;
}

// Masking rule of the reference (src/rdna/fa2_forward_f16.hip:325-348 and
// docs/api.md:150-165), with delta = Sk - Sq:
//   causal:             key <= q + delta
//   causal + window w:  q + delta - key < w
//   window w (no causal): |q + delta - key| <= w / 2
//   always:             key < Sk
struct MaskSpec {
    int32_t sk;
    int32_t delta;
    int32_t causal;
    int32_t window; // > 0 enables; 0 = off
};

RDNA_MASK_FN bool key_visible(const MaskSpec& m, int q, int key) {
    bool ok = key < m.sk;
    int rel = q + m.delta - key;
    if (m.causal) {
        ok = ok && rel >= 0;
    }
    if (m.window > 0) {
        if (m.causal) {
            ok = ok && rel < m.window;
        } else {
            int a = rel < 0 ? -rel : rel;
            ok = ok && a <= (m.window >> 1);
        }
    }
    return ok;
}

// Inclusive key interval [lo, hi] any row in [q_lo, q_hi] can see.
// Empty when hi < lo.
RDNA_MASK_FN void visible_key_range(const MaskSpec& m, int q_lo, int q_hi, int& lo, int& hi) {
    lo = 0;
    hi = m.sk - 1;
    if (m.causal) {
        hi = mask_imin(hi, q_hi + m.delta);
    }
    if (m.window > 0) {
        if (m.causal) {
            lo = mask_imax(lo, q_lo + m.delta - m.window + 1);
        } else {
            int hw = m.window >> 1;
            lo = mask_imax(lo, q_lo + m.delta - hw);
            hi = mask_imin(hi, q_hi + m.delta + hw);
        }
    }
}

// Classify a key tile [k_lo, k_hi] against rows [q_lo, q_hi]:
//   0 = no key visible to any row (skip), 1 = every pair visible (no mask),
//   2 = mixed (apply the per-element mask).
RDNA_MASK_FN int classify_tile(const MaskSpec& m, int q_lo, int q_hi, int k_lo, int k_hi) {
    int lo, hi;
    visible_key_range(m, q_lo, q_hi, lo, hi);
    if (hi < lo || k_hi < lo || k_lo > hi) {
        return 0;
    }
    bool full = k_hi < m.sk;
    if (m.causal) {
        full = full && (k_hi <= q_lo + m.delta);
    }
    if (m.window > 0) {
        if (m.causal) {
            full = full && (k_lo > q_hi + m.delta - m.window);
        } else {
            int hw = m.window >> 1;
            full = full && (k_lo >= q_hi + m.delta - hw) && (k_hi <= q_lo + m.delta + hw);
        }
    }
    return full ? 1 : 2;
}

// Visible keys of one query row q form the interval [lo, hi] (empty when
// hi < lo).  Same rule as key_visible, evaluated once per row so that masking a
// tile is two compares per score instead of a branchy predicate.
RDNA_MASK_FN void row_key_bounds(const MaskSpec& m, int q, int& lo, int& hi) {
    visible_key_range(m, q, q, lo, hi);
}

// classify_tile for every key tile of BN keys (tile t = keys [BN t, BN t + BN
// - 1], t >= 0) against rows [q_lo, q_hi], as two index ranges computed once:
// tile t is visible iff vis_lo <= t <= vis_hi, and mask-free iff it is visible
// and full_lo <= t <= full_hi.  A kernel then classifies each tile with four
// compares of wave-uniform values instead of re-deriving the mask bounds.
struct TileClasses {
    int vis_lo, vis_hi, full_lo, full_hi;
};

template <int BN>
RDNA_MASK_FN TileClasses tile_classes(const MaskSpec& m, int q_lo, int q_hi) {
    TileClasses c{1, 0, 1, 0}; // empty ranges
    int lo, hi;
    visible_key_range(m, q_lo, q_hi, lo, hi);
    if (hi < lo) {
        return c;
    }
    // BN t + BN - 1 >= lo and BN t <= hi, with 0 <= lo <= hi
    c.vis_lo = lo / BN;
    c.vis_hi = hi / BN;
    // mask-free: BN t + BN - 1 <= key_hi and BN t >= key_lo
    int key_hi = m.sk - 1;
    int key_lo = 0;
    if (m.causal) {
        key_hi = mask_imin(key_hi, q_lo + m.delta);
    }
    if (m.window > 0) {
        if (m.causal) {
            key_lo = q_hi + m.delta - m.window + 1;
        } else {
            const int hw = m.window >> 1;
            key_lo = q_hi + m.delta - hw;
            key_hi = mask_imin(key_hi, q_lo + m.delta + hw);
        }
    }
    c.full_hi = key_hi >= BN - 1 ? (key_hi - (BN - 1)) / BN : -1;
    c.full_lo = key_lo > 0 ? (key_lo + BN - 1) / BN : 0;
    return c;
}

RDNA_MASK_FN int tile_class(const TileClasses& c, int t) {
    if (t < c.vis_lo || t > c.vis_hi) {
        return 0;
    }
    return (t >= c.full_lo && t <= c.full_hi) ? 1 : 2;
}

} // namespace rdna_amd
