// k_dense.hip -- dense bipartite half-sweep (not yet built).
#include "internal.hpp"
namespace thrml {
int launch_dense_half(thrml_prog *, thrml_state *, uint32_t, const uint32_t *) {
  return fail(THRML_EUNSUPPORTED, "dense programs are not built yet");
}
int launch_dense_sync_act(thrml_state *, uint32_t) { return THRML_OK; }
}  // namespace thrml
extern "C" int thrml_rbm_program_create(thrml_ctx *, const thrml_rbm_desc *, thrml_prog **) {
  return thrml::fail(THRML_EUNSUPPORTED, "dense programs are not built yet");
}
extern "C" int thrml_rbm_half_sweep(thrml_prog *, thrml_state *, int, const uint32_t *) {
  return thrml::fail(THRML_EUNSUPPORTED, "dense programs are not built yet");
}
