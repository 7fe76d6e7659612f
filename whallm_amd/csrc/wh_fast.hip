// wh_fast.hip -- single-read sliced sampler engine (filled in by the fast path).
#include "wh_internal.h"
