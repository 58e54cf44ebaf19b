// Shared host helpers of the library: the error slot behind fnkv_last_error() and the pool lookup.
#pragma once

#include "kv_pool.h"

#include <hip/hip_runtime.h>

#include <string>

struct fnkv_pool;

namespace fnkv {

void set_error(const std::string & e);
const char * last_error();
const kv_pool * pool_of(const fnkv_pool * p);
// an integer knob from the environment (dflt when unset), for measurement only; callers keep it in a function-local
// static so it is read once per process
int32_t env_int_once(const char * name, int32_t dflt);
// compute units of a device (cached)
int32_t device_cus(int32_t device);
// the append's launch (fnkv_q8_append after its checks); pos_dev set: the first position is that device word, and
// positions outside 0 .. max_cells - rows are not written
int append_enqueue(const kv_pool & p, int32_t slot, int32_t layer, int64_t pos0, const int32_t * pos_dev,
                   int64_t max_cells, int32_t rows, const void * k, const void * v, int32_t dtype, hipStream_t st);

} // namespace fnkv
