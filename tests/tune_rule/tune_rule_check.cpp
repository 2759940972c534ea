// Host-only checks of the tile search's adoption rule (acfun_amd/csrc/tune_rule.hpp).
#include <cstdio>

#include "../../acfun_amd/csrc/tune_rule.hpp"

int main() {
    int fails = 0;
    auto expect = [&](bool c, const char* what) {
        if (!c) { std::printf("FAIL: %s\n", what); ++fails; }
    };
    const float inf = 1e30f;
    {
        const float c[3] = {10.2f, 9.8f, 10.5f};      // best 2% faster: within noise, keep the default
        expect(acfun::tune_pick(10.0f, c, 3) == -1, "a 2% win keeps the built-in choice");
    }
    {
        const float c[3] = {10.2f, 9.5f, 9.6f};       // best 5% faster: adopted
        expect(acfun::tune_pick(10.0f, c, 3) == 1, "a 5% win is adopted");
    }
    {
        const float c[2] = {12.0f, 11.0f};            // every candidate slower: never adopted
        expect(acfun::tune_pick(10.0f, c, 2) == -1, "slower candidates never adopted");
    }
    {
        const float c[2] = {inf, inf};                // nothing ran
        expect(acfun::tune_pick(10.0f, c, 2) == -1, "candidates that cannot run never win");
    }
    {
        const float c[2] = {8.0f, 7.0f};              // the built-in choice could not run
        expect(acfun::tune_pick(inf, c, 2) == 1, "no built-in time: the fastest candidate");
    }
    {
        const float c[1] = {9.69f};                   // 3.1% faster
        expect(acfun::tune_pick(10.0f, c, 1) == 0, "just past the margin is adopted");
    }
    if (fails) return 1;
    std::printf("ok\n");
    return 0;
}
