// Q4_K (GGUF bytes, flarellm nibble layout) Q8-input matvecs.
#include "launch.h"
#define MV_FMT F_Q4K
#define MV_SUFFIX q4k
#include "mv_q8in.inc"
