// Adjoint driver (implicit VJP through the CP fixed point).
#include "forward.hpp"
#include "plan.hpp"

using namespace purin;

extern "C" int purin_cp_adjoint(purin_cp_plan* p, void* stream, int64_t batch, const void* saved,
                                const void* target, const void* rhs, const void* cot_y,
                                const purin_cp_adjoint_options* opts, void* g_target, void* g_rhs,
                                void* g_lower, void* g_upper, uint8_t* valid, int32_t* info,
                                void* gmres_residual) {
  return set_error(PURIN_CP_ERR_UNSUPPORTED, "adjoint not built yet");
}
