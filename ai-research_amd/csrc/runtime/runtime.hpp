// runtime.hpp -- internal C++ side of the C ABI (not installed).
#pragma once
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "gemma_hip.h"

struct gh_context {
  int device = 0;
  hipStream_t stream = nullptr;
  char name[256] = {0};
  int num_cus = 0;
  size_t max_lds = 0;
  std::vector<hipModule_t> modules;
  std::unordered_map<std::string, hipFunction_t> fns;
  std::mutex mu;

  gh_status load(const char* dir);
  hipFunction_t fn(const std::string& name);
  gh_status launch(const std::string& name, dim3 grid, dim3 block, unsigned lds, void** args);
  ~gh_context();
};

namespace gh {
using Context = gh_context;
gh_status fail(gh_status st, const std::string& msg);
gh_status hip_fail(hipError_t e, const char* what);
}  // namespace gh
