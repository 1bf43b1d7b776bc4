// test_safetensors -- host-only checks of mi_bridge::SafetensorsFile (no GPU call):
// prints one line per file given on the command line, "OK <n> <name>:<dtype>:<d0>x<d1>..:<begin>-<end> ..."
// or "ERR <message>", for tests/test_checkpoint_oracle.py to compare with Python's own
// reading of the same files.
#include <cstdio>
#include <string>

#include "gemm_bridge.hpp"

int main(int argc, char** argv) {
  for (int i = 1; i < argc; ++i) {
    mi_bridge::SafetensorsFile f;
    if (!f.open(argv[i])) {
      std::printf("ERR %s\n", f.error().c_str());
      continue;
    }
    std::printf("OK %zu python=%d", f.tensors().size(), f.is_python_format() ? 1 : 0);
    for (const auto& t : f.tensors()) {
      std::string shape;
      for (size_t k = 0; k < t.shape.size(); ++k) shape += (k ? "x" : "") + std::to_string(t.shape[k]);
      std::printf(" %s:%s:%s:%zu-%zu", t.name.c_str(), t.dtype.c_str(), shape.c_str(), t.begin, t.end);
    }
    std::printf("\n");
  }
  return 0;
}
