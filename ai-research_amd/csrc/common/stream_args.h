// stream_args.h -- host-side mirrors of the kernel argument blocks of the
// gemv.hip row streams (same member order and types as the device structs).
#pragma once
#include <stdint.h>

struct XPro {
  const float* x;
  const float* r;
  const float* wr;
  const float* w;
  float* xout;
  float s, eps;
  uint32_t mode;
  // mode 4 (a gated layer's input under quiescence, src/gpu/model_dispatch.zig:
  // 45-101): A' = (x + RMSNorm(r) * wr) * s when the previous layer ran
  // (pmode 1, or pmode 2 with *prun != 0), else A' = xa; the GEMV consumes
  // RMSNorm(A') * w; workgroup 0 writes A' to xout (when it differs from xa),
  // stores it as xprev and writes *run_out = mean((A' - xprev)^2) >= thr
  const float* xa;
  float* xprev;
  const uint32_t* prun;
  uint32_t* run_out;
  uint32_t pmode;
  float thr;
};

struct Q4Args {  // Q4Fmt::Args / Q8Fmt::Args
  const uint8_t* W;
  float* Y;
};

struct GateUpArgs {  // GateUpFmt::Args / GateUpQ8Fmt::Args
  const uint8_t* Wg;
  const uint8_t* Wu;
  float* Y;
};

struct ArgmaxArgs {  // Q8ArgmaxFmt::Args
  const uint8_t* W;
  float* Y;
  uint32_t* partial;
};
