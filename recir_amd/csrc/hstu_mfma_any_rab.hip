// General MFMA kernels (hstu_mfma_any.h): the instantiations with a bias table.
#define HSTU_ANY_HAS_RAB 1
#include "hstu_mfma_any_launch.h"
