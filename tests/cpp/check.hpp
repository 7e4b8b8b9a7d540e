// check.hpp -- a minimal CHECK suite for the C++ host tests.
#pragma once

#include <cstdio>
#include <cstdlib>
#include <functional>
#include <string>
#include <vector>

namespace check {
inline int& failures() { static int f = 0; return f; }
inline int& checks() { static int c = 0; return c; }
inline std::vector<std::pair<std::string, std::function<void()>>>& registry() {
  static std::vector<std::pair<std::string, std::function<void()>>> r;
  return r;
}
struct Reg {
  Reg(const char* name, std::function<void()> fn) { registry().emplace_back(name, std::move(fn)); }
};
inline int run_all(int argc, char** argv) {
  const char* filter = argc > 1 ? argv[1] : nullptr;
  for (auto& [name, fn] : registry()) {
    if (filter && name.find(filter) == std::string::npos) continue;
    const int before = failures();
    fn();
    std::printf("%s %s\n", failures() == before ? "PASS" : "FAIL", name.c_str());
  }
  std::printf("%d checks, %d failures\n", checks(), failures());
  return failures() == 0 ? 0 : 1;
}
}  // namespace check

#define TEST(name)                                              \
  static void name();                                           \
  static check::Reg reg_##name(#name, name);                    \
  static void name()

#define CHECK(cond)                                                                   \
  do {                                                                                \
    ++check::checks();                                                                \
    if (!(cond)) {                                                                    \
      ++check::failures();                                                            \
      std::printf("  CHECK failed %s:%d: %s\n", __FILE__, __LINE__, #cond);          \
    }                                                                                 \
  } while (0)

#define CHECK_EQ(a, b)                                                                \
  do {                                                                                \
    ++check::checks();                                                                \
    const auto _va = (a);                                                             \
    const auto _vb = (b);                                                             \
    if (!(_va == _vb)) {                                                              \
      ++check::failures();                                                            \
      std::printf("  CHECK_EQ failed %s:%d: %s = %s vs %s = %s\n", __FILE__, __LINE__, #a, \
                  std::to_string(_va).c_str(), #b, std::to_string(_vb).c_str());     \
    }                                                                                 \
  } while (0)

#define CHECK_OK(expr)                                                                \
  do {                                                                                \
    ++check::checks();                                                                \
    const auto _st = (expr);                                                          \
    if (!_st.ok()) {                                                                  \
      ++check::failures();                                                            \
      std::printf("  CHECK_OK failed %s:%d: %s\n", __FILE__, __LINE__, #expr);       \
    }                                                                                 \
  } while (0)
