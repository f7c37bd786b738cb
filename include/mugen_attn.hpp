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
inline Status mla_absorb(const mugen_attn_mla_absorb_args& a, void* stream) {
    return check(mugen_attn_mla_absorb(&a, stream));
}
inline Status mla_project(const mugen_attn_mla_project_args& a, void* stream) {
    return check(mugen_attn_mla_project(&a, stream));
}
inline Status mla_latent_write(const mugen_attn_mla_latent_write_args& a, void* stream) {
    return check(mugen_attn_mla_latent_write(&a, stream));
}
inline Status mla_prepare(const mugen_attn_mla_latent_write_args& lw, const mugen_attn_mla_absorb_args& ab,
                          void* stream) {
    return check(mugen_attn_mla_prepare(&lw, &ab, stream));
}
inline Status kv_q4_append(const mugen_attn_kv_q4_append_args& a, void* stream) {
    return check(mugen_attn_kv_q4_append(&a, stream));
}
inline size_t gqa_decode_q4_workspace_size(const mugen_attn_gqa_decode_q4_args& a) {
    return mugen_attn_gqa_decode_q4_workspace_size(&a);
}
inline Status gqa_decode_q4(const mugen_attn_gqa_decode_q4_args& a, void* ws, size_t ws_bytes, void* stream) {
    return check(mugen_attn_gqa_decode_q4(&a, ws, ws_bytes, stream));
}
inline Status kv_append(const mugen_attn_kv_append_args& a, void* stream) {
    return check(mugen_attn_kv_append(&a, stream));
}
inline Status seq_advance(int32_t* seq_lens, int32_t n, int32_t count, int32_t max_seq_len, void* stream,
                          int32_t* n_q4 = nullptr, const int32_t* n_q4_next = nullptr) {
    return check(mugen_attn_seq_advance(seq_lens, n, count, max_seq_len, n_q4, n_q4_next, stream));
}

}  // namespace mugen_attn
