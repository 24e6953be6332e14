// Host build of the device cosine (tgengine_amd/csrc/tgx_cos.h) for the CPU
// accuracy test: reads n float32 arguments on stdin (binary), writes n float32.
#include <cstdio>
#include <vector>

#include "tgx_cos.h"

int main() {
  std::vector<float> x;
  float buf[4096];
  size_t got;
  while ((got = fread(buf, sizeof(float), 4096, stdin)) > 0) x.insert(x.end(), buf, buf + got);
  std::vector<float> y(x.size());
  for (size_t i = 0; i < x.size(); ++i) y[i] = tgx::cos_any(x[i]);
  fwrite(y.data(), sizeof(float), y.size(), stdout);
  return 0;
}
