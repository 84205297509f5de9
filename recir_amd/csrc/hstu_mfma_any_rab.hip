// General MFMA kernels (hstu_mfma_any.h): the instantiations with a bias table, rows at multiples of 16 bytes.
#define HSTU_ANY_HAS_RAB 1
#define HSTU_ANY_ALIGNED 1
#include "hstu_mfma_any_launch.h"
