// abi.cpp — ABI identity and the thread-local error message of libdsv41hip.so.
#include <string>

#include "common.h"

namespace dsv41 {
thread_local std::string g_last_error;
void set_error(const std::string& msg) { g_last_error = msg; }
int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}
}  // namespace dsv41

extern "C" int dsv41_abi_version(void) { return DSV41_ABI_VERSION; }
extern "C" size_t dsv41_sampler_desc_size(void) { return sizeof(dsv41_sampler_desc); }
extern "C" size_t dsv41_logprob_desc_size(void) { return sizeof(dsv41_logprob_desc); }
extern "C" size_t dsv41_logprob_grad_desc_size(void) { return sizeof(dsv41_logprob_grad_desc); }
extern "C" size_t dsv41_token_tis_desc_size(void) { return sizeof(dsv41_token_tis_desc); }
extern "C" size_t dsv41_grpo_desc_size(void) { return sizeof(dsv41_grpo_desc); }
extern "C" size_t dsv41_logprob_shard_desc_size(void) { return sizeof(dsv41_logprob_shard_desc); }
extern "C" size_t dsv41_logprob_combine_desc_size(void) { return sizeof(dsv41_logprob_combine_desc); }
extern "C" size_t dsv41_sampler_shard_desc_size(void) { return sizeof(dsv41_sampler_shard_desc); }
extern "C" size_t dsv41_sampler_merge_desc_size(void) { return sizeof(dsv41_sampler_merge_desc); }
extern "C" size_t dsv41_sampler_full_shard_desc_size(void) { return sizeof(dsv41_sampler_full_shard_desc); }
extern "C" size_t dsv41_sampler_full_finish_desc_size(void) { return sizeof(dsv41_sampler_full_finish_desc); }
extern "C" const char* dsv41_last_error(void) { return dsv41::g_last_error.c_str(); }
