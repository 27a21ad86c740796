// Q8_0 (re-laid-out: int8 quants + f16 block scales) Q8-input matvecs.
#include "launch.h"
#define MV_FMT F_Q8_0
#define MV_SUFFIX q8_0
#include "mv_q8in.inc"
