// gemv_lane_b8.hip -- lane-chain k4 GEMV instances for a batch of 8 activation
// rows.  Only 32-block rows (1024 columns): with more blocks per lane the
// eight batch columns' terms no longer fit in registers, and the tile kernel
// is the faster choice.
#include "gemv_lane.h"

namespace mantle {

template <int PRO>
static hipError_t launch_lane_gemv_b8(GemvParams& p, hipStream_t stream) {
    int rows = 0;
    for (int i = 0; i < p.nmat; i++) rows += p.mats[i].rows;
    if (rows <= lane_small_rows()) return launch_lane_gemv<kEpiStore, 8, 4, 8, 1, PRO>(p, stream);
    return launch_lane_gemv<kEpiStore, 8, 4, 8, 4, PRO, 1>(p, stream);  // one unit per workgroup, as at batch 1
}

hipError_t lane_gemv_batch8(GemvParams& p, int pro, hipStream_t stream, bool* used) {
    *used = false;
    if (p.bpr != 32) return hipSuccess;
    *used = true;
    switch (pro) {
        case kProQx: return launch_lane_gemv_b8<kProQx>(p, stream);
        case kProQuant: return launch_lane_gemv_b8<kProQuant>(p, stream);
        case kProNorm: return launch_lane_gemv_b8<kProNorm>(p, stream);
        default: *used = false; return hipSuccess;
    }
}

#ifdef MANTLE_PHASE_TRACE
MANTLE_PHASE_READER(phase_read_lane_b8)
#endif

}  // namespace mantle
