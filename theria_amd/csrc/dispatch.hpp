// Runtime (dtype, padded head dim, causal) -> template instantiation.
#pragma once

#include "sdpa_params.hpp"

namespace theria {

// L must provide: template <typename T, int DP, bool CAUSAL> static hipError_t run(const P&, hipStream_t).
template <typename L, typename T, int DP, typename P>
hipError_t dispatch_causal(const P& p, hipStream_t st) {
  return p.s.causal ? L::template run<T, DP, true>(p, st) : L::template run<T, DP, false>(p, st);
}

template <typename L, typename T, typename P>
hipError_t dispatch_dp(const P& p, hipStream_t st) {
  switch (p.s.dp) {
    case 32: return dispatch_causal<L, T, 32>(p, st);
    case 64: return dispatch_causal<L, T, 64>(p, st);
    case 128: return dispatch_causal<L, T, 128>(p, st);
    default: return hipErrorInvalidValue;
  }
}

template <typename L, typename P>
hipError_t dispatch_all(const P& p, hipStream_t st) {
  switch (p.s.dtype) {
    case 0: return dispatch_dp<L, float>(p, st);
    case 1: return dispatch_dp<L, _Float16>(p, st);
    case 2: return dispatch_dp<L, __bf16>(p, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace theria
