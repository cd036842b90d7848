// k_potts.hip -- categorical (Potts) half-sweep (not yet built).
#include "internal.hpp"
namespace thrml {
int launch_potts_half(thrml_prog *, thrml_state *, uint32_t, const uint32_t *) {
  return fail(THRML_EUNSUPPORTED, "categorical programs are not built yet");
}
}  // namespace thrml
extern "C" int thrml_potts_program_create(thrml_ctx *, const thrml_potts_desc *, thrml_prog **) {
  return thrml::fail(THRML_EUNSUPPORTED, "categorical programs are not built yet");
}
