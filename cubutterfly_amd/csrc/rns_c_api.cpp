// RNS C ABI (include/cuntt/rns_c_api.h). Lowering added in a later milestone.
#include "../../include/cuntt/rns_c_api.h"

#include <string>

namespace {
thread_local std::string rns_error;
}

extern "C" {
const char* cubutterflyRnsLastError(void) { return rns_error.c_str(); }
int cubutterflyRnsCreate(const char*, cubutterflyRnsPlan* result) {
    if (result) *result = nullptr;
    rns_error = "RNS NTT is not yet lowered for gfx950";
    return 2;
}
int cubutterflyRnsPrepare(cubutterflyRnsPlan, int, const char*, int, unsigned, void*) {
    rns_error = "plan must be created";
    return 1;
}
int cubutterflyRnsExecute(cubutterflyRnsPlan, const uint64_t*, uint64_t*, void*) {
    rns_error = "plan must be prepared";
    return 1;
}
int cubutterflyRnsInfoJson(cubutterflyRnsPlan, char*, size_t*) {
    rns_error = "plan must be non-null";
    return 1;
}
int cubutterflyRnsDestroy(cubutterflyRnsPlan) { return 0; }
}
