// gemv_lane_store.hip -- lane-chain k4 GEMV instances, batch 1, plain store
// epilogue (QKV projections, the logits and the kernel-level W4A8 entry points).
#include "gemv_lane.h"

namespace mantle {

hipError_t lane_gemv_store(GemvParams& p, int pro, hipStream_t stream, bool* used) {
    switch (pro) {
        case kProQx: return try_lane_gemv<kEpiStore, 1, kProQx>(p, stream, used);
        case kProQuant: return try_lane_gemv<kEpiStore, 1, kProQuant>(p, stream, used);
        case kProNorm: return try_lane_gemv<kEpiStore, 1, kProNorm>(p, stream, used);
        default: *used = false; return hipSuccess;
    }
}

#ifdef MANTLE_PHASE_TRACE
MANTLE_PHASE_READER(phase_read_lane_store)
#endif

}  // namespace mantle
