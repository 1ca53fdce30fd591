#pragma once
// Minimal assertion harness for the C++ tests (Catch2 is not available offline).
#include <cstdio>
#include <cstdlib>
#include <exception>
#include <functional>
#include <string>
#include <vector>

namespace mini {

struct Case {
    const char* name;
    std::function<void()> body;
};

inline std::vector<Case>& registry() {
    static std::vector<Case> cases;
    return cases;
}

struct Register {
    Register(const char* name, std::function<void()> body) { registry().push_back({name, std::move(body)}); }
};

struct Failure : std::exception {
    std::string message;
    explicit Failure(std::string m) : message(std::move(m)) {}
    const char* what() const noexcept override { return message.c_str(); }
};

inline int run_all() {
    int failed = 0;
    for (const auto& c : registry()) {
        std::printf("[ RUN  ] %s\n", c.name);
        std::fflush(stdout);
        try {
            c.body();
            std::printf("[  OK  ] %s\n", c.name);
        } catch (const std::exception& e) {
            ++failed;
            std::printf("[ FAIL ] %s: %s\n", c.name, e.what());
        }
        std::fflush(stdout);
    }
    std::printf("%zu cases, %d failed\n", registry().size(), failed);
    return failed == 0 ? 0 : 1;
}

}  // namespace mini

#define MINI_CAT2(a, b) a##b
#define MINI_CAT(a, b) MINI_CAT2(a, b)
#define TEST_CASE(name)                                                           \
    static void MINI_CAT(test_fn_, __LINE__)();                                   \
    static mini::Register MINI_CAT(test_reg_, __LINE__)(name, MINI_CAT(test_fn_, __LINE__)); \
    static void MINI_CAT(test_fn_, __LINE__)()

#define REQUIRE(cond)                                                             \
    do {                                                                          \
        if (!(cond))                                                              \
            throw mini::Failure(std::string(__FILE__) + ":" + std::to_string(__LINE__) + \
                                ": REQUIRE(" #cond ") failed");                   \
    } while (0)

#define REQUIRE_THROWS_AS(expr, type)                                             \
    do {                                                                          \
        bool caught_ = false;                                                     \
        try {                                                                     \
            expr;                                                                 \
        } catch (const type&) {                                                   \
            caught_ = true;                                                       \
        }                                                                         \
        if (!caught_)                                                             \
            throw mini::Failure(std::string(__FILE__) + ":" + std::to_string(__LINE__) + \
                                ": expected " #type " from " #expr);              \
    } while (0)

#define REQUIRE_NOTHROW(expr)                                                     \
    do {                                                                          \
        try {                                                                     \
            expr;                                                                 \
        } catch (const std::exception& e_) {                                      \
            throw mini::Failure(std::string(__FILE__) + ":" + std::to_string(__LINE__) + \
                                ": unexpected exception from " #expr ": " + e_.what()); \
        }                                                                         \
    } while (0)
