// Two-stream submission of one training step from its captured graphs.
//
// A step splits into a front part (batch preparation, sampling, GRU memory
// update), the memory commit, and a back part (attention forward, edge
// predictor, backward, fused Adam). Step t+1's front part only needs step t's
// commit (the memory table, the node bitmap) and reads nothing the back part
// writes as long as consecutive steps use different step buffers, so it runs
// on its own stream beside step t's back part:
//
//   front stream:  wait(committed) -> front graph -> record(fronted)
//   back stream:   wait(fronted) -> commit graph -> record(committed) -> back graph
//
// The events carry the cross-stream order: the front part of the next call
// waits for this call's commit, this call's commit for its own front part.
// Everything queued on the back stream before the commit (the previous back
// part included) precedes the commit, so a front part never overlaps the
// back part that still reads the buffers it is about to fill.
#include "common.h"

extern "C" int sgl_graph_pipeline(void *front_exec, void *commit_exec, void *back_exec, hipStream_t front,
                                  hipStream_t back, hipEvent_t committed, hipEvent_t fronted) {
  SGL_REQUIRE(front_exec && commit_exec && back_exec, "graph_pipeline: NULL graph executable");
  SGL_REQUIRE(committed && fronted, "graph_pipeline: NULL event");
  SGL_REQUIRE(front != back, "graph_pipeline: the front and back streams must differ");
  SGL_CHECK_HIP(hipStreamWaitEvent(front, committed, 0));
  SGL_CHECK_HIP(hipGraphLaunch(static_cast<hipGraphExec_t>(front_exec), front));
  SGL_CHECK_HIP(hipEventRecord(fronted, front));
  SGL_CHECK_HIP(hipStreamWaitEvent(back, fronted, 0));
  SGL_CHECK_HIP(hipGraphLaunch(static_cast<hipGraphExec_t>(commit_exec), back));
  SGL_CHECK_HIP(hipEventRecord(committed, back));
  SGL_CHECK_HIP(hipGraphLaunch(static_cast<hipGraphExec_t>(back_exec), back));
  return SGL_OK;
}
