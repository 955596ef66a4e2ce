// Exhaustive host check of the mask helpers in rdnattention_amd/csrc/fa_mask.hpp:
// tile_classes/tile_class (the per-row-tile ranges the kernels use) must equal
// classify_tile for every key tile, and classify_tile must agree with
// key_visible evaluated pair by pair.  Prints "ok <cases>" or the first
// mismatch and exits 1.
#include <cstdio>
#include <initializer_list>

#include "fa_mask.hpp"

using namespace rdna_amd;

template <int BN>
static bool check(const MaskSpec& m, int q_lo, int q_hi, long& cases) {
    const TileClasses tc = tile_classes<BN>(m, q_lo, q_hi);
    const int n_tiles = (m.sk + BN - 1) / BN + 2;
    for (int t = 0; t < n_tiles; t++) {
        const int k_lo = BN * t, k_hi = BN * t + BN - 1;
        const int want = classify_tile(m, q_lo, q_hi, k_lo, k_hi);
        const int got = tile_class(tc, t);
        // brute force: 0 if no pair visible, 1 if every pair visible
        int vis = 0, all = 1;
        for (int q = q_lo; q <= q_hi; q++) {
            for (int k = k_lo; k <= k_hi; k++) {
                const bool v = key_visible(m, q, k);
                vis |= v;
                all &= v;
            }
        }
        const int brute = vis ? (all ? 1 : 2) : 0;
        cases++;
        if (want != got || (brute == 0) != (want == 0) || (brute == 1) != (want == 1)) {
            std::printf("mismatch BN=%d sk=%d delta=%d causal=%d window=%d rows [%d,%d] tile %d: "
                        "classify_tile %d tile_class %d brute %d\n",
                        BN, m.sk, m.delta, m.causal, m.window, q_lo, q_hi, t, want, got, brute);
            return false;
        }
    }
    return true;
}

int main() {
    long cases = 0;
    const int sks[] = {1, 5, 31, 32, 33, 63, 64, 65, 100, 128, 129, 200};
    const int windows[] = {0, 1, 2, 3, 4, 7, 16, 31, 32, 33, 64, 65, 96, 1000};
    for (int sk : sks) {
        for (int sq : {1, 3, 32, 64, 97, 150, 200}) {
            for (int causal = 0; causal < 2; causal++) {
                for (int w : windows) {
                    const MaskSpec m{sk, sk - sq, causal, w};
                    for (int q_lo = 0; q_lo < sq; q_lo += 7) {
                        for (int len : {1, 2, 16, 32}) {
                            const int q_hi = q_lo + len - 1 < sq ? q_lo + len - 1 : sq - 1;
                            if (!check<32>(m, q_lo, q_hi, cases) || !check<64>(m, q_lo, q_hi, cases)) {
                                return 1;
                            }
                        }
                    }
                }
            }
        }
    }
    std::printf("ok %ld\n", cases);
    return 0;
}
