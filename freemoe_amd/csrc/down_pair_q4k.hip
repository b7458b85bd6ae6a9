// down_pair_q4k.hip — the 16-lane down kernel for Q4_K down matrices, in its
// own code object (down_pair.hpp).
#include "down_pair.hpp"

namespace fmx {

int launch_down_pair_q4k(const ExpertArgs &a, const float *x, const float *act, const uint32_t *ids, const float *w,
                         float *out, uint32_t *status, hipStream_t s, const hipEvent_t *kev) {
    return launch_down_pair<PairQ4K>(a, x, act, ids, w, out, status, s, kev);
}

} // namespace fmx
