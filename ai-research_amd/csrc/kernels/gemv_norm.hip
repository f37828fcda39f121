// gemv_norm.hip -- the row streams of gemv.hip with the normed x prologue
// (RMSNorm / residual add + RMSNorm fused in), built as a separate code object.
#define GH_GEMV_NORMED 1
#include "gemv.hip"
