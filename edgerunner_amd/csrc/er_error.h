// er_error.h -- the calling thread's last-error message, shared by the
// translation units of libedgerunner_hip (er_hip_last_error returns it).
#pragma once
#include "er_hip.h"

namespace er_detail {
extern thread_local char g_last_error[512];
// Formats the message for er_hip_last_error and returns st.
er_status fail(er_status st, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
}  // namespace er_detail
