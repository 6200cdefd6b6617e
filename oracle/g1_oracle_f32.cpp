// TEST INFRASTRUCTURE ONLY: the oracle's restatement (g1_oracle.cpp) evaluated in float32, as a yardstick of the error
// that float32 arithmetic alone gives a step (tests/ only, never the product path).
//
// Every `double` of g1_oracle.cpp becomes `float` (its entry points then take and return float32 arrays); its
// floating-point literals stay double, so an expression with one is evaluated in double and rounded to float when
// stored. The result follows the float64 oracle's algorithm step for step with float32 storage and mostly float32
// arithmetic: an estimate of the float32 rounding floor of each output, not a bitwise model of any float32 code.
// The standard headers are included first so that only the restatement's own text is affected.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>
#define double float
#include "g1_oracle.cpp"
