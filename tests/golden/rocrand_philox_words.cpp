// Prints Philox4x32-10 words from rocRAND's host-callable engine, used to pin
// the oracle's (seed, stream, offset) -> word mapping against an independent
// implementation.  Build: see make_philox_golden.sh.
#include <cstdio>
#include <cstdlib>
#include <rocrand/rocrand_philox4x32_10.h>

int main(int argc, char** argv) {
  if (argc != 5) { std::fprintf(stderr, "usage: seed stream offset n\n"); return 2; }
  unsigned long long seed = std::strtoull(argv[1], nullptr, 0);
  unsigned long long stream = std::strtoull(argv[2], nullptr, 0);
  unsigned long long offset = std::strtoull(argv[3], nullptr, 0);
  int n = std::atoi(argv[4]);
  rocrand_device::philox4x32_10_engine eng(seed, stream, offset);
  for (int i = 0; i < n; ++i) std::printf("%u\n", eng());
  return 0;
}
