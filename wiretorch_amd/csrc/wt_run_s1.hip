// The persistent forward kernel and the backward for S = 1 synapse types (see wt_run.h).
#include "wt_back.h"
#include "wt_run.h"

template struct wt::RunLaunch<1>;
template struct wt::BackLaunch<1>;
