// Internal interface between the one-sequence engine and the batch decoder
// built on it (not exported in the public headers).
#pragma once

#include "jinf/engine_hip.h"

namespace jinf {

// The engine's model: device weights, hyper-parameters, output resolved
// (tied to token_embd when the model has none), layers valid while the
// engine exists.
const jinf_hip_engine_desc* engine_desc(const jinf_hip_engine* e);

}  // namespace jinf
