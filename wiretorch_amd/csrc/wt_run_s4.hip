// The persistent forward kernel for S = 4 synapse types (see wt_run.h).
#include "wt_run.h"

template struct wt::RunLaunch<4>;
