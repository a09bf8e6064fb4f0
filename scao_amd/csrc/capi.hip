// Library-level C ABI: version, thread-local error message, and the layout of
// the descriptor structs so the Python binding can verify its mirror of them.
#include <stdarg.h>
#include <stddef.h>
#include <stdio.h>

#include "scao_common.hpp"

static thread_local char g_err[512] = "";

void scao_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

extern "C" int scao_abi_version(void) { return SCAO_ABI_VERSION; }

extern "C" const char* scao_last_error(void) { return g_err; }

#define PUT(x)                        \
  do {                                \
    if (n < cap) out[n] = (int64_t)(x); \
    ++n;                              \
  } while (0)

extern "C" int scao_struct_layout(int which, int64_t* out, int cap) {
  int n = 0;
  if (!out || cap <= 0) return 0;
  switch (which) {
    case 0: {
      typedef scao_param_desc S;
      PUT(sizeof(S));
      PUT(offsetof(S, p)); PUT(offsetof(S, g)); PUT(offsetof(S, graw)); PUT(offsetof(S, exp_avg));
      PUT(offsetof(S, exp_avg_sq)); PUT(offsetof(S, exp_avg_diff)); PUT(offsetof(S, prev_grad));
      PUT(offsetof(S, upd)); PUT(offsetof(S, diag_ema)); PUT(offsetof(S, fema));
      PUT(offsetof(S, fthr)); PUT(offsetof(S, fseed)); PUT(offsetof(S, numel));
      PUT(offsetof(S, cols)); PUT(offsetof(S, lr)); PUT(offsetof(S, decay));
      PUT(offsetof(S, beta1)); PUT(offsetof(S, omb1)); PUT(offsetof(S, beta2));
      PUT(offsetof(S, omb2)); PUT(offsetof(S, beta3)); PUT(offsetof(S, omb3));
      PUT(offsetof(S, bc1)); PUT(offsetof(S, bc2)); PUT(offsetof(S, bc3));
      PUT(offsetof(S, blend)); PUT(offsetof(S, omblend)); PUT(offsetof(S, eps));
      PUT(offsetof(S, tau)); PUT(offsetof(S, lars)); PUT(offsetof(S, wd));
      PUT(offsetof(S, gsnr)); PUT(offsetof(S, diag_bias)); PUT(offsetof(S, adam_sqrt_bc2));
      PUT(offsetof(S, adam_alpha)); PUT(offsetof(S, dtype)); PUT(offsetof(S, flags));
      PUT(offsetof(S, pre_begin)); PUT(offsetof(S, pre_end)); PUT(offsetof(S, post_begin));
      PUT(offsetof(S, post_end)); PUT(offsetof(S, norm_index)); PUT(offsetof(S, fnoise));
      break;
    }
    case 1: {
      typedef scao_leaf_desc S;
      PUT(sizeof(S));
      PUT(offsetof(S, Ul)); PUT(offsetof(S, Ur)); PUT(offsetof(S, Sl)); PUT(offsetof(S, Sr));
      PUT(offsetof(S, T)); PUT(offsetof(S, Delta)); PUT(offsetof(S, W)); PUT(offsetof(S, off));
      PUT(offsetof(S, ld)); PUT(offsetof(S, param)); PUT(offsetof(S, m)); PUT(offsetof(S, n));
      PUT(offsetof(S, k)); PUT(offsetof(S, flags)); PUT(offsetof(S, dbias));
      PUT(offsetof(S, Wb));
      break;
    }
    case 2: {
      typedef scao_task S;
      PUT(sizeof(S));
      PUT(offsetof(S, idx)); PUT(offsetof(S, a)); PUT(offsetof(S, b)); PUT(offsetof(S, slot));
      break;
    }
    case 3: {
      typedef scao_param_stat S;
      PUT(sizeof(S));
      PUT(offsetof(S, g2)); PUT(offsetof(S, p2)); PUT(offsetof(S, nu2)); PUT(offsetof(S, u2));
      PUT(offsetof(S, gnorm)); PUT(offsetof(S, pnorm)); PUT(offsetof(S, nu));
      PUT(offsetof(S, clip)); PUT(offsetof(S, unorm)); PUT(offsetof(S, trust));
      PUT(offsetof(S, alpha));
      break;
    }
    case 4: {
      typedef scao_gram_desc S;
      PUT(sizeof(S));
      PUT(offsetof(S, g)); PUT(offsetof(S, off)); PUT(offsetof(S, ld)); PUT(offsetof(S, q));
      PUT(offsetof(S, scale)); PUT(offsetof(S, ema)); PUT(offsetof(S, amax));
      PUT(offsetof(S, rows)); PUT(offsetof(S, cols)); PUT(offsetof(S, side));
      PUT(offsetof(S, dtype)); PUT(offsetof(S, ntiles)); PUT(offsetof(S, flags));
      PUT(offsetof(S, rho)); PUT(offsetof(S, alpha));
      break;
    }
    case 5: {
      typedef scao_prep_desc S;
      PUT(sizeof(S));
      PUT(offsetof(S, q)); PUT(offsetof(S, scale)); PUT(offsetof(S, ema)); PUT(offsetof(S, out));
      PUT(offsetof(S, shift)); PUT(offsetof(S, dim)); PUT(offsetof(S, bias));
      break;
    }
    case 6: {
      typedef scao_filter_desc S;
      PUT(sizeof(S));
      PUT(offsetof(S, g)); PUT(offsetof(S, ema)); PUT(offsetof(S, out)); PUT(offsetof(S, work));
      PUT(offsetof(S, seed)); PUT(offsetof(S, numel)); PUT(offsetof(S, decay));
      PUT(offsetof(S, omd)); PUT(offsetof(S, q)); PUT(offsetof(S, noise));
      PUT(offsetof(S, dtype)); PUT(offsetof(S, flags)); PUT(offsetof(S, cand));
      PUT(offsetof(S, cap));
      break;
    }
    case 7: {
      typedef scao_lookahead_desc S;
      PUT(sizeof(S));
      PUT(offsetof(S, p)); PUT(offsetof(S, slow)); PUT(offsetof(S, numel)); PUT(offsetof(S, dtype));
      break;
    }
    default:
      return 0;
  }
  return n < cap ? n : cap;
}
