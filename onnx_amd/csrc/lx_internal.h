// lx_internal.h -- library-internal interface between the C ABI (lx_api.cpp)
// and the graph runtime (lx_graph.cpp, lx_onnx.cpp).
#pragma once

#include <hip/hip_runtime.h>

#include <string>

namespace lx {

int api_set_error(int code, const std::string &message);  // sets lx_last_error, returns code
bool api_initialized();
hipStream_t api_stream();
int64_t api_esize(int dtype);
const char *api_dtype_name(int dtype);

}  // namespace lx
