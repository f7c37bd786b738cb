// mugen_attn.hpp -- C++ adapter over the mugen_attn C ABI in the engine's
// error style.
//
// Mugen's host code reports failures as std::expected<T, std::string>
// (MetalCompute::dispatch_sync / dispatch_chain_sync, metal_compute.h:84-89;
// TransformerModel API, transformer.h:80-131) and never throws.  These inline
// wrappers turn the ABI's int status + thread-local message into that shape:
//
//     if (auto r = mugen_attn::mla_decode(args, ws, ws_bytes, stream); !r)
//         return std::unexpected(r.error());
//
// With a C++23 standard library mugen_attn::Status is std::expected<void,
// std::string>; older libraries (the engine itself requires C++23) get a
// minimal stand-in with the same members used above (operator bool,
// has_value, error).
#pragma once

#include <cstddef>
#include <string>

#include "mugen_attn.h"

#if __has_include(<expected>) && __cplusplus >= 202302L
#include <expected>
#endif

namespace mugen_attn {

#if defined(__cpp_lib_expected)
using Status = std::expected<void, std::string>;
inline Status fail(std::string msg) { return std::unexpected(std::move(msg)); }
#else
class Status {
public:
    Status() = default;
    static Status failure(std::string msg) {
        Status s;
        s.ok_ = false;
        s.err_ = std::move(msg);
        return s;
    }
    bool has_value() const noexcept { return ok_; }
    explicit operator bool() const noexcept { return ok_; }
    const std::string& error() const noexcept { return err_; }

private:
    bool ok_ = true;
    std::string err_;
};
inline Status fail(std::string msg) { return Status::failure(std::move(msg)); }
#endif

// status code + last error message -> Status
inline Status check(int rc) {
    if (rc == MUGEN_ATTN_OK) return Status{};
    std::string msg = mugen_attn_last_error();
    if (msg.empty()) msg = "mugen_attn error " + std::to_string(rc);
    return fail(std::move(msg));
}

inline size_t gqa_decode_workspace_size(const mugen_attn_gqa_decode_args& a) {
    return mugen_attn_gqa_decode_workspace_size(&a);
}
inline Status gqa_decode(const mugen_attn_gqa_decode_args& a, void* ws, size_t ws_bytes, void* stream) {
    return check(mugen_attn_gqa_decode(&a, ws, ws_bytes, stream));
}
inline Status gqa_prefill(const mugen_attn_gqa_prefill_args& a, void* stream) {
    return check(mugen_attn_gqa_prefill(&a, stream));
}
inline size_t mla_decode_workspace_size(const mugen_attn_mla_decode_args& a) {
    return mugen_attn_mla_decode_workspace_size(&a);
}
inline Status mla_decode(const mugen_attn_mla_decode_args& a, void* ws, size_t ws_bytes, void* stream) {
    return check(mugen_attn_mla_decode(&a, ws, ws_bytes, stream));
}
inline Status scatter_kv(const void* src, void* dst, uint64_t offset, uint64_t count, void* stream) {
    return check(mugen_attn_scatter_kv(src, dst, offset, count, stream));
}

}  // namespace mugen_attn
