// Host harness for sincos_rope (vsa-lm_amd/csrc/bolt3_math.h): reads fp32 angles (raw bytes)
// on stdin, writes sin then cos (raw fp32) on stdout.  Built by tests/test_rope_math.py.
#include <cstdio>
#include <vector>
#include "bolt3_math.h"

int main() {
  std::vector<float> x;
  float v;
  while (std::fread(&v, sizeof v, 1, stdin) == 1) x.push_back(v);
  std::vector<float> out(2 * x.size());
  for (size_t i = 0; i < x.size(); ++i) b3::sincos_rope(x[i], &out[i], &out[x.size() + i]);
  std::fwrite(out.data(), sizeof(float), out.size(), stdout);
  return 0;
}
