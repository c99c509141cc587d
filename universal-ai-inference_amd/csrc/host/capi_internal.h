// capi_internal.h — shared by the C entry points of libuaii_amd.so: sets the
// thread's uaii_last_error text and maps uaii::Error to uaii_status
// (libs/uaii-capi/src/capi.cpp:17-39).
#pragma once

#include "uaii/c_api/uaii.h"

#include "error.h"

uaii_status uaii_capi_status(const uaii::Error& err);
uaii_status uaii_capi_fail(uaii_status st, const char* msg);
