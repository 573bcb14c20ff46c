// Compile-time dispatch over (dtype, lanes per row) for the kernels.
#pragma once

#include <type_traits>

#include "kiv_common.h"
#include "kiv_internal.h"

namespace kiv {

template <int DT, typename F> static int with_lg(int lg, F &&f) {
  switch (lg) {
    case 1: return f(std::integral_constant<int, DT>{}, std::integral_constant<int, 1>{});
    case 2: return f(std::integral_constant<int, DT>{}, std::integral_constant<int, 2>{});
    case 4: return f(std::integral_constant<int, DT>{}, std::integral_constant<int, 4>{});
    case 8: return f(std::integral_constant<int, DT>{}, std::integral_constant<int, 8>{});
    case 16: return f(std::integral_constant<int, DT>{}, std::integral_constant<int, 16>{});
    case 32: return f(std::integral_constant<int, DT>{}, std::integral_constant<int, 32>{});
    case 64: return f(std::integral_constant<int, DT>{}, std::integral_constant<int, 64>{});
  }
  return fail(KIV_ERR_UNSUPPORTED, "no kernel for %d lanes per row", lg);
}

template <typename F> inline int with_dt_lg(int dt, int lg, F &&f) {
  if (dt == KIV_DTYPE_F32) return with_lg<DT_F32>(lg, f);
  if (dt == KIV_DTYPE_F16) return with_lg<DT_F16>(lg, f);
  return with_lg<DT_BF16>(lg, f);
}

template <typename F> inline int with_dt(int dt, F &&f) {
  if (dt == KIV_DTYPE_F32) return f(std::integral_constant<int, DT_F32>{});
  if (dt == KIV_DTYPE_F16) return f(std::integral_constant<int, DT_F16>{});
  return f(std::integral_constant<int, DT_BF16>{});
}

// Runs f(integral_constant<KT>) for head_dim = 32 * KT (KT in 1-4, 6, 8, 16).
template <typename F> static int with_kt(int kt, F &&f) {
  using std::integral_constant;
  switch (kt) {
    case 1: return f(integral_constant<int, 1>{});
    case 2: return f(integral_constant<int, 2>{});
    case 3: return f(integral_constant<int, 3>{});
    case 4: return f(integral_constant<int, 4>{});
    case 6: return f(integral_constant<int, 6>{});
    case 8: return f(integral_constant<int, 8>{});
    case 16: return f(integral_constant<int, 16>{});
  }
  return fail(KIV_ERR_UNSUPPORTED, "no MFMA kernel for head_dim %d", kt * 32);
}

}  // namespace kiv
