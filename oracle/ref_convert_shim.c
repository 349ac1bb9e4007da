/*
 * Exports the reference's header-only RNE converters (core/convert.h, all
 * static inline) so the checker can call them.  Built only by ref.mk, into
 * oracle/_ref/, from the header where it lies in the reference checkout.
 */
#include "core/convert.h"

uint16_t ref_f32_to_f16(float f) { return pg_f32_to_f16_scalar(f); }
float ref_f16_to_f32(uint16_t h) { return pg_f16_to_f32_scalar(h); }
uint16_t ref_f32_to_bf16(float f) { return pg_f32_to_bf16_scalar(f); }
float ref_bf16_to_f32(uint16_t h) { return pg_bf16_to_f32_scalar(h); }
