// The C ABI's error convention (core/src/c_api.cpp:17-18, 66-107): every
// call clears a thread-local message, catches every exception and returns a
// status naming its class.  Shared by the exports of every translation unit
// and free of device code.
#pragma once

#include <stdexcept>
#include <string>

#include "kv_ledger.hpp"
#include "tvara_capi.h"

namespace tvara_amd::abi {

// The message is meaningful only while the status says a call failed, so
// clearing (every call) touches the status alone: a trivially constructed
// thread-local, read without the wrapper a std::string needs, and in the
// initial-exec model (4 bytes of the static TLS block, a thread-pointer
// relative access instead of a __tls_get_addr call).
extern thread_local std::string error_message;
extern thread_local int error_status __attribute__((tls_model("initial-exec")));

inline int failed(int status, const char* what) {
    error_message = what;
    error_status = status;
    return status;
}

inline void clear() { error_status = TVARA_OK; }

template <class F>
int guard(F&& f) {
    clear();
    try {
        f();
        return TVARA_OK;
    } catch (const CacheExhausted& e) {
        return failed(TVARA_EXHAUSTED, e.what());
    } catch (const std::invalid_argument& e) {
        return failed(TVARA_INVALID, e.what());
    } catch (const std::logic_error& e) {
        return failed(TVARA_LOGIC, e.what());
    } catch (const std::exception& e) {
        return failed(TVARA_ERROR, e.what());
    } catch (...) {
        return failed(TVARA_ERROR, "unknown native error");
    }
}

inline Handle handle(tvara_kv_handle h) { return Handle{static_cast<size_t>(h.id), h.generation}; }
inline tvara_kv_handle exported(Handle h) { return tvara_kv_handle{h.id, h.generation}; }

// The bookkeeping behind a cache handle; throws invalid_argument("closed KV
// cache") for NULL.  Defined by the library that defines tvara_kv_cache.
KvLedger& ledger_of(tvara_kv_cache* cache);

}  // namespace tvara_amd::abi
