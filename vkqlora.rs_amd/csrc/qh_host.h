// qh_host.h -- host-side helpers shared by the runtime's translation units
// (not part of the public ABI).
#pragma once
#include <string>

#include "qlora_hip.h"

namespace qh {
// Records `msg` as this thread's qh_last_error() in the Display format of the
// status's error variant and returns the status.
qh_status host_fail(qh_status st, const std::string &msg);
}  // namespace qh
