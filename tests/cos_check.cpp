// Host build of the time-encoding reduction (tgengine_amd/csrc/tgx_cos.h) for the
// CPU accuracy test: reads n float32 arguments on stdin (binary) and writes, per
// argument, the float64 revolution fraction f of rev_frac (cos(x) = cos(2 pi f)).
#include <cstdio>
#include <vector>

#include "tgx_cos.h"

static const double kTab[][2] = {TGX_REV_TABLE_ROWS};

int main() {
  std::vector<float> x;
  float buf[4096];
  size_t got;
  while ((got = fread(buf, sizeof(float), 4096, stdin)) > 0) x.insert(x.end(), buf, buf + got);
  std::vector<double> f(x.size());
  for (size_t i = 0; i < x.size(); ++i) f[i] = tgx::rev_frac(x[i], kTab);
  fwrite(f.data(), sizeof(double), f.size(), stdout);
  return 0;
}
