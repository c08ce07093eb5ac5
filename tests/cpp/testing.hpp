// Minimal Go-style test runner for the C++ host-mirror tests: TEST(Name)
// registers a function; t.Fatalf-like FATAL() stops that test; the binary
// prints "--- PASS: Name" / "--- FAIL: Name" and exits non-zero on failure.
#pragma once

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <exception>
#include <functional>
#include <string>
#include <vector>

namespace ctest {

struct Failure {
  std::string msg;
};

inline std::vector<std::pair<std::string, std::function<void()>>>& registry() {
  static std::vector<std::pair<std::string, std::function<void()>>> r;
  return r;
}

struct Reg {
  Reg(const char* n, std::function<void()> f) { registry().emplace_back(n, std::move(f)); }
};

inline std::string fmt(const char* f, ...) __attribute__((format(printf, 1, 2)));
inline std::string fmt(const char* f, ...) {
  char buf[2048];
  va_list ap;
  va_start(ap, f);
  vsnprintf(buf, sizeof buf, f, ap);
  va_end(ap);
  return buf;
}

inline int run_all(int argc, char** argv) {
  int failed = 0, run = 0;
  for (auto& [name, fn] : registry()) {
    if (argc > 1 && name.find(argv[1]) == std::string::npos) continue;
    run++;
    try {
      fn();
      std::printf("--- PASS: %s\n", name.c_str());
    } catch (const Failure& f) {
      failed++;
      std::printf("--- FAIL: %s\n    %s\n", name.c_str(), f.msg.c_str());
    } catch (const std::exception& e) {
      failed++;
      std::printf("--- FAIL: %s\n    unexpected exception: %s\n", name.c_str(), e.what());
    }
    std::fflush(stdout);
  }
  std::printf("%s (%d tests, %d failed)\n", failed ? "FAIL" : "ok", run, failed);
  return failed ? 1 : 0;
}

}  // namespace ctest

#define TEST(Name)                                         \
  static void Name();                                      \
  static ctest::Reg reg_##Name(#Name, Name);               \
  static void Name()

#define FATAL(...) throw ctest::Failure{ctest::fmt(__VA_ARGS__)}
#define EXPECT(cond)                                                            \
  do {                                                                          \
    if (!(cond)) FATAL("%s:%d: expected %s", __FILE__, __LINE__, #cond);        \
  } while (0)
