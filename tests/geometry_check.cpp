// CPU-only sweep of the launch geometry (tr-infer_amd/csrc/geometry.hpp): for every layer shape and
// call size below, each grid tiles or covers its matrix, and every workspace extent a call indexes
// stays within what trk_create sizes.  Built with g++ by tests/test_geometry.py; prints the number
// of (shape, call) cases checked, or the first failing case and exits 1.
#include <cstdio>

#include "geometry.hpp"

using namespace trk::geo;

int main() {
    const unsigned Hs[] = {256, 512, 768, 1024, 2048, 2560, 4096};
    const unsigned Fs[] = {256, 512, 768, 1024, 2048};
    const unsigned Es[] = {1, 16, 24, 32, 512, 600, 1024};
    const unsigned Ms[] = {1, 2, 16, 64, 300, 512, 3072};
    const unsigned Ks[] = {1, 2, 10, 32};
    unsigned long long n = 0;
    for (unsigned H : Hs)
        for (unsigned F : Fs)
            for (unsigned E : Es)
                for (unsigned m_max : Ms)
                    for (unsigned k_cap : Ks) {
                        const Caps c{H, E, F, m_max, k_cap};
                        for (unsigned m = 1; m <= m_max; m += (m < 80 ? 1 : 37)) {
                            for (unsigned kcap = 1; kcap <= k_cap; kcap++) {
                                const char* why = check_call(c, m, kcap);
                                n++;
                                if (why) {
                                    std::printf("FAIL H=%u E=%u F=%u m_max=%u k_cap=%u m=%u kcap=%u: %s\n", H, E, F,
                                                m_max, k_cap, m, kcap, why);
                                    return 1;
                                }
                            }
                        }
                        // rejected: more rows than the capacity, more selections than k_cap
                        if (!check_call(c, m_max + 1, 1) || !check_call(c, 1, k_cap + 1)) {
                            std::printf("FAIL: an over-capacity call passed (H=%u F=%u)\n", H, F);
                            return 1;
                        }
                    }
    std::printf("ok %llu\n", n);
    return 0;
}
