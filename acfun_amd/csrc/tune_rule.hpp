// tune_rule.hpp -- the tile search's adoption rule, independent of HIP so that
// it can be exercised on the host.
//
// The reference adopts a tuned blocking only if no measured size regresses
// more than 3% against its heuristic (src/autotune.cpp:147,212).  Here every
// shape is timed with its built-in choice beside the candidates, in the same
// interleaved rounds, and a candidate replaces the built-in choice only when
// it is faster by more than kTuneMargin; otherwise the built-in choice stays
// (recorded as -1).  A candidate that could not run (+inf) never wins.
#pragma once

namespace acfun {

constexpr float kTuneMargin = 0.03f;

// default_ms: the built-in choice's time; cand_ms[0..n): the candidates'.
// Returns the adopted candidate, or -1 to keep the built-in choice.
inline int tune_pick(float default_ms, const float* cand_ms, int n) {
    int best = -1;
    float best_ms = default_ms;
    for (int c = 0; c < n; ++c)
        if (cand_ms[c] < best_ms) { best_ms = cand_ms[c]; best = c; }
    if (best < 0) return -1;
    // the built-in choice could not be timed: take the fastest candidate
    if (!(default_ms < 1e29f)) return best;
    return best_ms < (1.0f - kTuneMargin) * default_ms ? best : -1;
}

}  // namespace acfun
