// Sanitizer driver for the front end (host code only; built by
// tests/test_frontend_fuzz.py with g++ -fsanitize=address,undefined).
// Reads records "program \x01 options" separated by NUL bytes from stdin and
// runs parse -> verify -> options -> plan on each; prints how far records got.
#include <cstdio>
#include <iostream>
#include <iterator>
#include <string>

#include "frontend.h"

int main() {
  std::string all((std::istreambuf_iterator<char>(std::cin)), std::istreambuf_iterator<char>());
  size_t pos = 0, n = 0, reach[5] = {0, 0, 0, 0, 0};
  while (pos < all.size()) {
    size_t end = all.find('\0', pos);
    if (end == std::string::npos) end = all.size();
    const std::string rec = all.substr(pos, end - pos);
    pos = end + 1;
    const size_t sep = rec.find('\x01');
    const std::string prog = rec.substr(0, sep), opts = sep == std::string::npos ? "" : rec.substr(sep + 1);
    tff::Program p;
    tff::Options o;
    tff::Plan pl;
    std::string err;
    int depth = 0;
    if (tff::parse_program(prog, "f.mlir", p, err)) {
      ++depth;
      if (tff::verify_program(p, err)) {
        ++depth;
        if (tff::parse_options(opts, o, err)) {
          ++depth;
          if (tff::plan_program(p, o, pl, err)) ++depth;
        }
      }
    }
    ++reach[depth];
    ++n;
  }
  std::printf("records %zu parse_fail %zu verify_fail %zu options_fail %zu plan_fail %zu planned %zu\n", n, reach[0],
              reach[1], reach[2], reach[3], reach[4]);
  return 0;
}
