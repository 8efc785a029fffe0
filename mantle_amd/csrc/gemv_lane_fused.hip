// gemv_lane_fused.hip -- lane-chain k4 GEMV instances, batch 1, with the
// decode step's fused epilogues: residual add (attention output and MLP down
// projections), SiLU(gate)*up, and the greedy argmax over the logits.
#include "gemv_lane.h"

namespace mantle {

hipError_t lane_gemv_fused(GemvParams& p, GemvEpi epi, int pro, hipStream_t stream, bool* used) {
    *used = false;
    switch (epi * 4 + pro) {
        case kEpiResAdd * 4 + kProQx: return try_lane_gemv<kEpiResAdd, 1, kProQx>(p, stream, used);
        case kEpiResAdd * 4 + kProQuant: return try_lane_gemv<kEpiResAdd, 1, kProQuant>(p, stream, used);
        case kEpiResAdd * 4 + kProNorm: return try_lane_gemv<kEpiResAdd, 1, kProNorm>(p, stream, used);
        case kEpiSiluMul * 4 + kProQuant: return try_lane_gemv<kEpiSiluMul, 1, kProQuant>(p, stream, used);
        case kEpiSiluMul * 4 + kProNorm: return try_lane_gemv<kEpiSiluMul, 1, kProNorm>(p, stream, used);
        case kEpiArgmax * 4 + kProNorm: return try_lane_gemv<kEpiArgmax, 1, kProNorm>(p, stream, used);
        default: return hipSuccess;
    }
}

#ifdef MANTLE_PHASE_TRACE
MANTLE_PHASE_READER(phase_read_lane_fused)
#endif

}  // namespace mantle
