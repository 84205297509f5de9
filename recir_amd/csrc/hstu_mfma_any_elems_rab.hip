// General MFMA kernels (hstu_mfma_any.h): the instantiations with a bias table for rows aligned to the
// element only (head dims or addresses that are not multiples of 16 bytes).
#define HSTU_ANY_HAS_RAB 1
#define HSTU_ANY_ALIGNED 0
#include "hstu_mfma_any_launch.h"
