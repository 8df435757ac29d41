// Compile-time check of the oracle's kernel prelude (see cpu_device.py).
#include <cmath>
#include <cstddef>
#include <vector>
using std::exp2; using std::log2; using std::sin; using std::sqrt; using std::fabs;
extern "C" float oracle_prelude_check(float x) {
  float a = exp2(x), b = log2(x), c = sin(x), d = sqrt(fabs(x));
  float e = 1.0 / x;           // double, as an unsuffixed OpenCL literal
  return a + b + c + d + e + std::fmax(a, b);
}
