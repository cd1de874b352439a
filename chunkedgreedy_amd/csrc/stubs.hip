// stubs.hip -- reference entry points outside the Chunked Greedy path.
//
// The symbols exist so that a binding written against the reference's C ABI
// links unchanged; calling one aborts with a diagnostic, the reference's
// failure behaviour for invalid use (sporder/src/common/error_checking.h:55-61).
//   sporder_hierarchical_matching   reference sporder.h:119-123 (hm/)
//   sporder_similarity_graph_exact  reference sporder.h:373-377
#include "common.hpp"

using namespace sporder_hip;

extern "C" {

void sporder_hierarchical_matching(sporder_context_t, int32_t, int32_t,
                                   const int32_t *, const int32_t *, bool, int32_t,
                                   const sporder_options_t *, int32_t *,
                                   sporder_hm_timing_t *, sporder_hm_stats_t *) {
  SP_EXPECT(false, "sporder_hierarchical_matching is not part of this build");
}

void sporder_similarity_graph_exact(sporder_context_t, int32_t, int32_t,
                                    const int32_t *, const int32_t *, bool, int32_t,
                                    int32_t *, float *, sporder_sim_exact_timing_t *,
                                    sporder_sim_exact_stats_t *) {
  SP_EXPECT(false, "sporder_similarity_graph_exact is not part of this build");
}

} // extern "C"
