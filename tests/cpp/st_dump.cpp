// Prints what fiber::safetensors reads from a file or directory, one JSON
// object per tensor ({"name", "dtype", "shape", "bits" (fp32 bit patterns,
// float tensors only)}), or {"error": message}. Driven by tests/test_host_formats.py.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <sys/stat.h>

#include "safetensors.hpp"

using namespace fiber::safetensors;

static void jstr(const std::string& s) {
  std::putchar('"');
  for (char c : s) {
    if (c == '"' || c == '\\') std::printf("\\%c", c);
    else std::putchar(c);
  }
  std::putchar('"');
}

int main(int argc, char** argv) {
  if (argc != 2) {
    std::fprintf(stderr, "usage: st_dump <file.safetensors | dir>\n");
    return 2;
  }
  struct stat st;
  const bool dir = stat(argv[1], &st) == 0 && S_ISDIR(st.st_mode);
  try {
    File f = dir ? File::OpenDir(argv[1]) : File::Open(argv[1]);
    for (const auto& kv : f.Metadata()) {
      std::printf("{\"meta\": ");
      jstr(kv.first);
      std::printf(", \"value\": ");
      jstr(kv.second);
      std::printf("}\n");
    }
    for (const std::string& name : f.Names()) {
      const Info* info = f.Find(name);
      std::printf("{\"name\": ");
      jstr(name);
      std::printf(", \"dtype\": \"%s\", \"shape\": [", info->dtype.c_str());
      for (size_t i = 0; i < info->shape.size(); i++) std::printf("%s%lld", i ? ", " : "", (long long)info->shape[i]);
      std::printf("]");
      if (info->dtype == "F32" || info->dtype == "BF16" || info->dtype == "F16" || info->dtype == "F64") {
        std::printf(", \"bits\": [");  // the fp32 values' bit patterns, exactly
        const auto v = f.Float32s(name);
        for (size_t i = 0; i < v.size(); i++) {
          uint32_t b;
          std::memcpy(&b, &v[i], 4);
          std::printf("%s%u", i ? ", " : "", b);
        }
        std::printf("]");
      }
      std::printf("}\n");
    }
  } catch (const Error& e) {
    std::printf("{\"error\": ");
    jstr(e.what());
    std::printf("}\n");
  }
  return 0;
}
