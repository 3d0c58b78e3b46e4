// Exposes the reference's own header-only codec and split-policy functions
// (uwp/rkva/rkva-kvarn-bulk.h:17-111, uwp/rkva/rkva-range-profile.h:82-147)
// through a C ABI so the tests can check the oracle's restatement against the
// compiled reference. Built by `make ref` with -I<reference>/uwp/rkva; the
// headers are read in place and nothing from them is copied here.
#include "rkva-kvarn-bulk.h"
#include "rkva-range-profile.h"

extern "C" {
uint16_t xr_f32_to_f16(float v) { return rkva_kvarn_bulk::f32_to_f16_bits(v); }
float xr_f16_to_f32(uint16_t h) { return rkva_kvarn_bulk::f16_bits_to_f32(h); }
uint8_t xr_f16_to_e5m2(uint16_t h) { return rkva_kvarn_bulk::f16_to_fp8_bits(h); }
uint16_t xr_e5m2_to_f16(uint8_t b) { return rkva_kvarn_bulk::fp8_to_f16_bits(b); }
uint32_t xr_reference_split_k(uint32_t active) { return rkva_rprof::reference_split_k(active); }
uint32_t xr_optimized_split_k(uint32_t active, uint32_t mode) {
    return rkva_rprof::optimized_split_k(active, mode);
}
uint32_t xr_split_rows(uint32_t active, uint32_t k) { return rkva_rprof::split_rows(active, k); }
void xr_q4_mq_split(uint32_t active, uint32_t mode, uint32_t* k, uint32_t* rows) {
    const rkva_rprof::Q4MqSplit s = rkva_rprof::q4_mq_split(active, mode);
    *k = s.split_k;
    *rows = s.split_rows;
}
}
