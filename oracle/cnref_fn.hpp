// Elementary functions of the CPU oracle (test infrastructure): the C
// library's float functions, as the reference's float expressions call them;
// or, in the double-evaluation mode that cnref_set_accumulate_double selects
// (used only to measure how far a training trajectory moves under rounding),
// the double functions rounded once to float.
#pragma once
#include <cmath>

namespace cnref_detail {
extern int acc_double;
}

inline float ref_exp(float x) { return cnref_detail::acc_double ? (float)std::exp((double)x) : std::exp(x); }
inline float ref_log(float x) { return cnref_detail::acc_double ? (float)std::log((double)x) : std::log(x); }
inline float ref_tanh(float x) { return cnref_detail::acc_double ? (float)std::tanh((double)x) : std::tanh(x); }
