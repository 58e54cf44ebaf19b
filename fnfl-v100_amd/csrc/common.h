// Shared host helpers of the library: the error slot behind fnkv_last_error() and the pool lookup.
#pragma once

#include "kv_pool.h"

#include <string>

struct fnkv_pool;

namespace fnkv {

void set_error(const std::string & e);
const char * last_error();
const kv_pool * pool_of(const fnkv_pool * p);
// compute units of a device (cached)
int32_t device_cus(int32_t device);

} // namespace fnkv
