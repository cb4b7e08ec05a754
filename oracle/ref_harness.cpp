// Test infrastructure, not product code: a C entry point over the
// reference's own CPU encoder, tans_encode_interleaved
// (csrc/tans_codec.cpp:69-196), which oracle/Makefile's `ref` target
// compiles unmodified from the reference tree together with this file into
// oracle/_ref/libref_codec.so.  The tests use it to check the oracle's C
// restatement of that encoder (oracle.c, ora_ref_encode_*) byte for byte.
#include <torch/torch.h>

#include <cstdint>
#include <cstring>
#include <exception>
#include <string>
#include <tuple>

// defined in csrc/tans_codec.cpp
std::tuple<torch::Tensor, torch::Tensor, torch::Tensor, torch::Tensor>
tans_encode_interleaved(torch::Tensor symbols, torch::Tensor freqs, torch::Tensor spread);

namespace {

struct Result {
    torch::Tensor comp, states, offsets, partial;
};

thread_local std::string g_error;

}  // namespace

extern "C" {

// Runs the reference encoder on symbols [K, N] (u8), freqs [nsym] (i32) and
// spread [4096] (i32).  Returns a handle holding the four output tensors
// (NULL on failure, message in ref_last_error) and their sizes.
void* ref_encode(const uint8_t* symbols, int64_t K, int64_t N, const int32_t* freqs,
                 int64_t nsym, const int32_t* spread, int64_t spread_len, int64_t* comp_bytes,
                 int64_t* n_offsets) {
    try {
        auto u8 = torch::TensorOptions().dtype(torch::kUInt8);
        auto i32 = torch::TensorOptions().dtype(torch::kInt32);
        auto sym = torch::from_blob(const_cast<uint8_t*>(symbols), {K, N}, u8);
        auto fr = torch::from_blob(const_cast<int32_t*>(freqs), {nsym}, i32);
        auto sp = torch::from_blob(const_cast<int32_t*>(spread), {spread_len}, i32);
        auto out = tans_encode_interleaved(sym, fr, sp);
        auto* r = new Result{std::get<0>(out).contiguous(), std::get<1>(out).contiguous(),
                             std::get<2>(out).contiguous(), std::get<3>(out).contiguous()};
        *comp_bytes = r->comp.numel();
        *n_offsets = r->offsets.numel();
        return r;
    } catch (const std::exception& e) {
        g_error = e.what();
        return nullptr;
    }
}

// Copies the outputs: comp [comp_bytes] u8, states [K] u16, offsets
// [n_offsets] i32, partial [K] u8.
void ref_encode_copy(void* handle, uint8_t* comp, uint16_t* states, int32_t* offsets,
                     uint8_t* partial) {
    auto* r = static_cast<Result*>(handle);
    std::memcpy(comp, r->comp.data_ptr(), (size_t)r->comp.numel());
    std::memcpy(states, r->states.data_ptr(), (size_t)r->states.numel() * 2);
    std::memcpy(offsets, r->offsets.data_ptr(), (size_t)r->offsets.numel() * 4);
    std::memcpy(partial, r->partial.data_ptr(), (size_t)r->partial.numel());
}

void ref_encode_free(void* handle) { delete static_cast<Result*>(handle); }

const char* ref_last_error(void) { return g_error.c_str(); }

}  // extern "C"
