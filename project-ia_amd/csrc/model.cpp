// model.cpp -- Llama-3 decode plan on MI355X (device state of a built model).
#include "qh_runtime.hpp"

namespace qh {

void plan_destroy(CtxState* st) { st->plan = nullptr; }

}  // namespace qh
