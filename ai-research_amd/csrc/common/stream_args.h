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
