// Host driver for the __host__ __device__ helpers of tca/hip/device.h (test
// program): reads "ceil_div a b" and "col_split rows col_blocks rows_min
// blocks" lines on stdin and prints one result per line, so the tests can
// hold the device's chunk arithmetic to the launch plan's 64-bit numbers.
#include <cstdio>
#include <cstring>

#include "tca/hip/device.h"

int main() {
  char op[32];
  while (std::scanf("%31s", op) == 1) {
    if (std::strcmp(op, "ceil_div") == 0) {
      unsigned a = 0, b = 0;
      if (std::scanf("%u %u", &a, &b) != 2 || b == 0) return 2;
      std::printf("%u\n", tca::hip::ceil_div(a, b));
    } else if (std::strcmp(op, "col_split") == 0) {
      unsigned r = 0, cb = 0, rm = 0, bl = 0;
      if (std::scanf("%u %u %u %u", &r, &cb, &rm, &bl) != 4 || rm == 0) return 2;
      std::printf("%u\n", tca::hip::col_split(r, cb, rm, bl));
    } else {
      return 2;
    }
  }
  return 0;
}
