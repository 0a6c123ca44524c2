#pragma once
#include <cstdint>
#include <functional>
#include <string>

#include "../../../include/qpack_hip.h"

namespace qph {
using SynthSpec = qph_synth_spec;
void synth_write(const SynthSpec &s, const std::string &path, int threads);
}  // namespace qph
