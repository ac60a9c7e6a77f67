// Event timing of the dominant kernel of each call (see profile.hip).
#pragma once

#include "rt_common.h"

namespace rt {

bool profile_on();
// Records a start event on `stream` when profiling is on; *stop is the matching stop event
// (null when off).
void profile_begin(hipStream_t stream, hipEvent_t* stop);
void profile_end(hipStream_t stream, hipEvent_t stop);

}  // namespace rt
