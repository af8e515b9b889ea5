// ctd_train -- the training CLI over include/ctd/train.h.
// Usage: ctd_train --config runs/<name>/config.json   (tools/ctd_train/main.cpp:33-43)
#include <exception>
#include <iostream>
#include <string>

#include "ctd/train.h"

int main(int argc, char** argv) {
  std::string cfg;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    if (a == "--config" && i + 1 < argc) cfg = argv[++i];
  }
  if (cfg.empty()) {
    std::cerr << "usage: " << argv[0] << " --config <path-to-config.json>\n";
    return 2;
  }
  try {
    return ctd::train::run(ctd::train::load_config(cfg));
  } catch (const std::exception& e) {
    std::cerr << "ctd_train: error: " << e.what() << "\n";
    return 1;
  }
}
