// Thread-local error state of the C ABI (c_api.cpp:17-18).
#include "abi.hpp"

namespace tvara_amd::abi {
thread_local std::string error_message;
thread_local int error_status __attribute__((tls_model("initial-exec"))) = TVARA_OK;
}  // namespace tvara_amd::abi

extern "C" {

// c_api.h:17
const char* tvara_last_error(void) {
    return tvara_amd::abi::error_status == TVARA_OK ? "" : tvara_amd::abi::error_message.c_str();
}

int tvara_last_status(void) { return tvara_amd::abi::error_status; }

}  // extern "C"
