// ctd_generate -- token generation subprocess over include/ctd/generate.h.
// Reads one JSON request from stdin, streams JSON reply lines to stdout.
// Usage: ctd_generate --model <path-to-fp32.safetensors> [--config <model.json>]
// (tools/ctd_generate/main.cpp:36-47; --config is an addition for architectures
// that autodetection does not know, e.g. small test models).
#include <iostream>
#include <iterator>
#include <string>

#include "ctd/generate.h"

int main(int argc, char** argv) {
  std::string model, config;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    if (a == "--model" && i + 1 < argc) model = argv[++i];
    else if (a == "--config" && i + 1 < argc) config = argv[++i];
  }
  if (model.empty()) {
    std::cerr << "usage: " << argv[0]
              << " --model <path-to-fp32.safetensors> [--config <model.json>]\n";
    return 2;
  }
  const std::string request((std::istreambuf_iterator<char>(std::cin)),
                            std::istreambuf_iterator<char>());
  return ctd::generate::run(model, request, std::cout, std::cerr, config);
}
