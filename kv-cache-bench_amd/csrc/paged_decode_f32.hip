// paged_decode instantiations for f32 caches (head_dim 64/128, 1/2/4/8 query heads per workgroup,
// tile-aligned and any-page variants); one file per storage type so they compile in parallel.
#include "paged_decode_impl.hpp"

namespace kvbk {

hipError_t launch_paged_decode_f32(int head_dim, int qg, bool fast, const DecodeParams& p, int batch, hipStream_t s,
                                  const Marks& m) {
    return launch_for_kind<KV_F32>(head_dim, qg, fast, p, batch, s, m);
}

}  // namespace kvbk

#ifdef KVB_WG_TIMESTAMPS
// Measurement build only: copies n stamp words (kWgStampWords per workgroup) of this storage type's
// last launch.
extern "C" int kvb_wg_stamps_f32(void* dst, size_t n) {
    if (n > kvbk::kWgStampGroups * kvbk::kWgStampWords) return (int)hipErrorInvalidValue;
    return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(kvbk::g_wg_stamps), n * sizeof(unsigned long long), 0,
                                    hipMemcpyDeviceToHost);
}
#endif
