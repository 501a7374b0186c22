/* CPU oracle for the streaming sparse INT4 MLP -- TEST INFRASTRUCTURE ONLY (see oracle.c). */
#ifndef LS_ORACLE_H
#define LS_ORACLE_H
#include <stdint.h>
#include <stddef.h>

typedef struct ora_desc {
    uint32_t logical_group, physical_group, source_slot, dest_slot, source_kind;
} ora_desc;

float ora_f16_to_f32(uint16_t h);
uint16_t ora_f32_to_f16(float f);
uint16_t ora_f64_to_f16(double d);
uint64_t ora_stream(uint64_t seed, uint64_t i);
double ora_normal(uint64_t seed, uint64_t i);
void ora_fill_bytes(uint8_t* dst, uint64_t n, uint64_t seed);
void ora_fill_uniform_f16(uint16_t* dst, uint64_t n, uint64_t seed, double lo, double hi);
void ora_fill_normal_f16(uint16_t* dst, uint64_t n, uint64_t seed);
float ora_weight(const uint8_t* row, const uint16_t* scale_row, uint32_t c);
int ora_compute(const ora_desc* d, const uint8_t* cache, const uint8_t* staging, const uint16_t* scales,
                const uint16_t* x, uint32_t width, uint32_t G, float* partial_row, float* h_out);
void ora_reduce(const float* partial, uint32_t rows, uint32_t width, float* y32, uint16_t* y16);
int ora_layer(const ora_desc* descs, uint32_t count, uint32_t rows, const uint8_t* cache, const uint8_t* staging,
              const uint16_t* scales, const uint16_t* x, uint32_t width, uint32_t G, int threads, float* y32,
              uint16_t* y16, float* h_rows, float* partial);
int ora_rank(const float* scores, uint32_t n, uint32_t k, int32_t* out);
void ora_publish_hidden(const uint16_t* residual, const uint16_t* y16, uint32_t n, uint16_t* hidden);
int ora_rmsnorm(const uint16_t* x, const uint16_t* weight, float eps, uint32_t width, uint16_t* out);
#endif
