// Host build of the kernels' rotary sincos (csrc/kernels/common.h) for tests/test_rotary.py.
#include "common.h"

extern "C" void rot_sincos(const float* x, float* s, float* c, long long n) {
  for (long long i = 0; i < n; ++i) sincos_rot(x[i], s + i, c + i);
}
