// chpe_pack -- writes a seeded synthetic .chpe archive (libchpe_pack.so, include/chpe_pack.h).
//
//   chpe_pack <kind> <path> [--seed N] [--threads N]
// kind: 3b-fp16-raw, 3b-bf16-raw, 3b-w4, 3b-w2, 3b-w4-std, 72b-w4, 72b-w2, 9b-w4 (or its number).
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include "../../include/chpe_pack.h"

int main(int argc, char** argv) {
  static const char* kNames[] = {"3b-fp16-raw", "3b-bf16-raw", "3b-w4", "3b-w2", "3b-w4-std", "72b-w4", "72b-w2", "9b-w4"};
  constexpr int kKinds = int(sizeof(kNames) / sizeof(kNames[0]));
  if (argc < 3) {
    std::fprintf(stderr, "usage: chpe_pack <kind> <path> [--seed N] [--threads N]\nkinds:");
    for (int k = 0; k < kKinds; ++k) std::fprintf(stderr, " %s", kNames[k]);
    std::fprintf(stderr, "\n");
    return 2;
  }
  int kind = -1;
  for (int k = 0; k < kKinds; ++k)
    if (std::strcmp(argv[1], kNames[k]) == 0) kind = k;
  if (kind < 0) {
    char* end = nullptr;
    const long v = std::strtol(argv[1], &end, 10);
    if (end && *end == 0 && v >= 0 && v < kKinds) kind = int(v);
  }
  if (kind < 0) {
    std::fprintf(stderr, "chpe_pack: unknown kind '%s'\n", argv[1]);
    return 2;
  }
  unsigned long long seed = 0;
  int threads = 0;
  for (int i = 3; i + 1 < argc; i += 2) {
    if (std::strcmp(argv[i], "--seed") == 0) seed = std::strtoull(argv[i + 1], nullptr, 10);
    else if (std::strcmp(argv[i], "--threads") == 0) threads = std::atoi(argv[i + 1]);
  }
  const int rc = chpe_pack_write(argv[2], kind, seed, threads);
  if (rc != 0) {
    std::fprintf(stderr, "chpe_pack: writing %s failed (%d)\n", argv[2], rc);
    return 1;
  }
  std::fprintf(stderr, "chpe_pack: %s (%s, seed %llu, %llu bytes)\n", argv[2], kNames[kind], seed,
               (unsigned long long)chpe_pack_size(kind));
  return 0;
}
