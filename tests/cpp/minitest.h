// Minimal test harness for the C++ drop-in API tests (no gtest in this image).
#pragma once
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <string>
#include <vector>

namespace minitest {
struct Case {
  const char* name;
  std::function<void()> body;
};
inline std::vector<Case>& registry() {
  static std::vector<Case> cases;
  return cases;
}
inline int& failures() {
  static int n = 0;
  return n;
}
struct Registrar {
  Registrar(const char* name, std::function<void()> body) { registry().push_back({name, body}); }
};
inline int run_all(int argc, char** argv) {
  const char* filter = argc > 1 ? argv[1] : nullptr;
  int ran = 0, failed_cases = 0;
  for (auto& c : registry()) {
    if (filter && std::string(c.name).find(filter) == std::string::npos) continue;
    const int before = failures();
    std::printf("[ RUN  ] %s\n", c.name);
    std::fflush(stdout);
    c.body();
    ++ran;
    const bool ok = failures() == before;
    if (!ok) ++failed_cases;
    std::printf("[ %s ] %s\n", ok ? " OK " : "FAIL", c.name);
  }
  std::printf("%d cases, %d failed\n", ran, failed_cases);
  return failed_cases ? 1 : 0;
}
}  // namespace minitest

#define MT_CAT2(a, b) a##b
#define MT_CAT(a, b) MT_CAT2(a, b)
#define TEST_CASE(name)                                                           \
  static void MT_CAT(mt_body_, __LINE__)();                                       \
  static minitest::Registrar MT_CAT(mt_reg_, __LINE__)(name, MT_CAT(mt_body_, __LINE__)); \
  static void MT_CAT(mt_body_, __LINE__)()
#define CHECK(cond)                                                                   \
  do {                                                                                \
    if (!(cond)) {                                                                    \
      std::printf("  %s:%d: CHECK failed: %s\n", __FILE__, __LINE__, #cond);          \
      ++minitest::failures();                                                         \
    }                                                                                 \
  } while (0)
#define CHECK_EQ(a, b) CHECK((a) == (b))
#define REQUIRE(cond)                                                                 \
  do {                                                                                \
    if (!(cond)) {                                                                    \
      std::printf("  %s:%d: REQUIRE failed: %s\n", __FILE__, __LINE__, #cond);        \
      ++minitest::failures();                                                         \
      return;                                                                         \
    }                                                                                 \
  } while (0)
#define CHECK_THROWS_AS(expr, type)                                                   \
  do {                                                                                \
    bool caught_ = false;                                                             \
    try {                                                                             \
      (void)(expr);                                                                   \
    } catch (const type&) {                                                           \
      caught_ = true;                                                                 \
    } catch (...) {                                                                   \
    }                                                                                 \
    if (!caught_) {                                                                   \
      std::printf("  %s:%d: expected %s from %s\n", __FILE__, __LINE__, #type, #expr); \
      ++minitest::failures();                                                         \
    }                                                                                 \
  } while (0)
#define MINITEST_MAIN() \
  int main(int argc, char** argv) { return minitest::run_all(argc, argv); }
