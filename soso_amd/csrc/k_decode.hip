// k_decode.hip -- placeholder (decode step kernels)
#include "internal.hpp"
