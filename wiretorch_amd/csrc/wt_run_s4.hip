// The persistent forward kernel and the backward for S = 4 synapse types (see wt_run.h).
#include "wt_back.h"
#include "wt_run.h"

template struct wt::RunLaunch<4>;
template struct wt::BackLaunch<4>;
