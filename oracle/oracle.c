/*
 * CPU oracle for the lgml ragged decode/prefill path.
 *
 * TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke()
 * and the cpu_baseline leg of bench.py, as the checker. The shipped
 * library never links or calls it.
 *
 * Everything here restates the reference's behaviour in plain C:
 * fp32 values, f64 reductions, f16 KV storage (round to nearest even),
 * closed-form Q4_K / Q6_K / Q8_0 dequantization. Reference citations are
 * paths under the lgml tree; [ggml] marks the semantics of the
 * un-vendored ggml op that the lgml wrapper calls (its public format or
 * algorithm, restated here in our own code).
 *
 * Pinning (what checks each part):
 *   orc_lcg_*, orc_fill_*        tests/test_oracle_golden.py regenerates the
 *                                tiny models; REF logits then pin them.
 *   f16 conversion               numpy astype(float16) on 2^32-sampled bits.
 *   dequantize Q4_K/Q6_K/Q8_0    hand-built blocks with known values,
 *                                quantize->dequantize error bounds
 *                                (test_convert.lua:287-310 rmse bounds).
 *   forward / attention          REF.llama / REF.qwen3 golden rows
 *                                (test_qwen_moe.lua:210-241), TOL 2e-3 + argmax;
 *                                attention also against numpy softmax on
 *                                tiny cases; batched == lone equality.
 *   mul_mat                      numpy matmul of the dequantized rows.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- random numbers ---------------------------------------------------- */

/* test/tiny.lua:16-22, test/test_qwen_moe.lua:32-38 (Lua 5.4 integers wrap
 * modulo 2^64 and >> is a logical shift). */
double
orc_lcg_next(uint64_t *state)
{
	*state = *state * 6364136223846793005ULL + 1442695040888963407ULL;
	return (double)(*state >> 11) / 9007199254740992.0;
}

/* test/test_qwen_moe.lua:77-86: lo + (hi - lo) * r(), in double, then the
 * f32 store of test/gguf.lua:41-50 (string.pack "<f"). */
void
orc_lcg_fill(uint64_t *state, float *out, int64_t n, double lo, double hi)
{
	for (int64_t i = 0; i < n; i++)
		out[i] = (float)(lo + (hi - lo) * orc_lcg_next(state));
}

/* src/lgml.c:3064-3079 */
static uint64_t
splitmix64(uint64_t *x)
{
	uint64_t z = (*x += 0x9e3779b97f4a7c15ULL);

	z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
	z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
	return z ^ (z >> 31);
}

/* One raw draw, for tests against splitmix64's published outputs. */
uint64_t
orc_splitmix64(uint64_t *state)
{
	return splitmix64(state);
}

static double
unit01(uint64_t *x)
{
	return (double)(splitmix64(x) >> 11) * (1.0 / 9007199254740992.0);
}

/* src/lgml.c:3130-3136 ("normal": two draws, cos branch). */
void
orc_fill_normal(uint64_t *seed, float *out, int64_t n, double mean, double sd)
{
	for (int64_t i = 0; i < n; i++) {
		double u1 = unit01(seed), u2 = unit01(seed);
		out[i] = (float)(mean + sd * sqrt(-2.0 * log(u1 > 0 ? u1 : 1e-300)) *
		    cos(6.283185307179586 * u2));
	}
}

/* The same values as orc_fill_normal(seed, out, n, ...), computed in
 * parallel: splitmix64's state after j draws is seed + j * gamma, so value
 * i (draws 2i+1, 2i+2) needs no sequential pass. */
static float
normal_at(uint64_t seed, int64_t i, double mean, double sd)
{
	uint64_t a = seed + (uint64_t)(2 * i) * 0x9e3779b97f4a7c15ULL;
	uint64_t b = a + 0x9e3779b97f4a7c15ULL;
	double u1 = unit01(&a), u2 = unit01(&b);
	return (float)(mean + sd * sqrt(-2.0 * log(u1 > 0 ? u1 : 1e-300)) *
	    cos(6.283185307179586 * u2));
}

void
orc_gen_normal(uint64_t seed, float *out, int64_t n, double mean, double sd, int n_threads)
{
#pragma omp parallel for schedule(static) num_threads(n_threads > 0 ? n_threads : 1)
	for (int64_t i = 0; i < n; i++)
		out[i] = normal_at(seed, i, mean, sd);
}

/* rows x cols normal values (as orc_gen_normal) quantized row by row into
 * type. Returns the bytes written or -1. */
int64_t
orc_gen_normal_quant(uint64_t seed, int type, int64_t rows, int64_t cols, double mean, double sd,
    void *out, int n_threads)
{
	int64_t rs = orc_row_size(type, cols);
	int bad = 0;

	if (rs <= 0)
		return -1;
#pragma omp parallel num_threads(n_threads > 0 ? n_threads : 1)
	{
		float *row = malloc(sizeof(float) * (size_t)cols);
		if (!row) {
#pragma omp atomic write
			bad = 1;
		}
#pragma omp for schedule(static)
		for (int64_t r = 0; r < rows; r++) {
			if (!row)
				continue;
			for (int64_t c = 0; c < cols; c++)
				row[c] = normal_at(seed, r * cols + c, mean, sd);
			if (orc_quantize_row(type, row, (uint8_t *)out + r * rs, cols) != rs) {
#pragma omp atomic write
				bad = 1;
			}
		}
		free(row);
	}
	return bad ? -1 : rows * rs;
}

/* src/lgml.c:3128-3129 ("uniform"). */
void
orc_fill_uniform(uint64_t *seed, float *out, int64_t n, double a, double b)
{
	for (int64_t i = 0; i < n; i++)
		out[i] = (float)(a + (b - a) * unit01(seed));
}

/* ---- f16 (IEEE binary16, round to nearest even) ---------------------------- */

uint16_t
orc_f32_to_f16(float f)
{
	uint32_t x;
	memcpy(&x, &f, 4);
	uint32_t sign = (x >> 16) & 0x8000u;
	uint32_t ex = (x >> 23) & 0xffu;
	uint32_t man = x & 0x7fffffu;

	if (ex == 0xffu)
		return (uint16_t)(sign | (man ? 0x7e00u : 0x7c00u));
	int e = (int)ex - 127 + 15;
	if (e >= 31)
		return (uint16_t)(sign | 0x7c00u);
	if (e <= 0) {
		/* f16 subnormal: value = m * 2^-24, m = mant24 >> (14 - e). */
		int shift = 14 - e;
		if (ex == 0 || shift > 24)
			return (uint16_t)sign;
		uint32_t m24 = man | 0x800000u;
		uint32_t h = m24 >> shift;
		uint32_t rem = m24 & ((1u << shift) - 1u);
		uint32_t half = 1u << (shift - 1);
		if (rem > half || (rem == half && (h & 1u)))
			h++;
		return (uint16_t)(sign | h);
	}
	uint32_t h = ((uint32_t)e << 10) | (man >> 13);
	uint32_t rem = man & 0x1fffu;
	if (rem > 0x1000u || (rem == 0x1000u && (h & 1u)))
		h++; /* a carry into the exponent is the correct rounding */
	return (uint16_t)(sign | h);
}

float
orc_f16_to_f32(uint16_t h)
{
	uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
	uint32_t ex = (h >> 10) & 0x1fu;
	uint32_t man = h & 0x3ffu;
	uint32_t x;

	if (ex == 0) {
		if (man == 0) {
			x = sign;
		} else {
			/* subnormal: normalise */
			int e = -1;
			do {
				man <<= 1;
				e++;
			} while (!(man & 0x400u));
			man &= 0x3ffu;
			x = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
		}
	} else if (ex == 0x1fu) {
		x = sign | 0x7f800000u | (man << 13);
	} else {
		x = sign | ((ex - 15 + 127) << 23) | (man << 13);
	}
	float f;
	memcpy(&f, &x, 4);
	return f;
}

/* orc_f16_to_f32 of every f16 bit pattern, for the attention loops (the
 * same values, read from a table). Filled once, before parallel regions. */
static float f16_lut[65536];
static int f16_lut_ready;

static void
f16_lut_init(void)
{
	if (__atomic_load_n(&f16_lut_ready, __ATOMIC_ACQUIRE))
		return;
#pragma omp critical(orc_f16_lut)
	{
		if (!f16_lut_ready) {
			for (uint32_t i = 0; i < 65536; i++)
				f16_lut[i] = orc_f16_to_f32((uint16_t)i);
			__atomic_store_n(&f16_lut_ready, 1, __ATOMIC_RELEASE);
		}
	}
}

void
orc_f32_to_f16_row(const float *x, uint16_t *y, int64_t n)
{
	for (int64_t i = 0; i < n; i++)
		y[i] = orc_f32_to_f16(x[i]);
}

void
orc_f16_to_f32_row(const uint16_t *x, float *y, int64_t n)
{
	for (int64_t i = 0; i < n; i++)
		y[i] = orc_f16_to_f32(x[i]);
}

/* ---- quantized block formats [ggml, public] --------------------------------
 * Q4_K: 256 values, 144 B {f16 d; f16 dmin; u8 scales[12]; u8 qs[128]}
 * Q6_K: 256 values, 210 B {u8 ql[128]; u8 qh[64]; i8 scales[16]; f16 d}
 * Q8_0:  32 values,  34 B {f16 d; i8 qs[32]}
 */
#define QK_K 256
#define Q4K_BYTES 144
#define Q6K_BYTES 210
#define Q8_0_BYTES 34

int64_t
orc_row_size(int type, int64_t n)
{
	switch (type) {
	case ORC_F32:
		return n * 4;
	case ORC_F16:
		return n * 2;
	case ORC_Q8_0:
		return n / 32 * Q8_0_BYTES;
	case ORC_Q4_K:
		return n / QK_K * Q4K_BYTES;
	case ORC_Q6_K:
		return n / QK_K * Q6K_BYTES;
	}
	return -1;
}

static uint16_t
rd16(const uint8_t *p)
{
	return (uint16_t)(p[0] | (p[1] << 8));
}

static void
wr16(uint8_t *p, uint16_t v)
{
	p[0] = (uint8_t)v;
	p[1] = (uint8_t)(v >> 8);
}

/* 6-bit scale and min j (0..7) of a Q4_K super-block's 12 scale bytes. */
static void
q4k_scale_min(int j, const uint8_t *s, int *sc, int *mn)
{
	if (j < 4) {
		*sc = s[j] & 63;
		*mn = s[j + 4] & 63;
	} else {
		*sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
		*mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
	}
}

/* Value v of a Q4_K super-block: group g = v / 32 has scale d * sc_g and
 * min dmin * m_g; the 4-bit q of v sits in byte 32 * (v / 64) + v % 32,
 * low nibble for v % 64 < 32, high nibble otherwise. The product d1 * q
 * is exact in f32 (11 + 6 + 4 bits), so y is one rounding of the exact
 * d1 * q - m1 with or without FMA contraction. */
static void
deq_q4k(const uint8_t *b, float *y)
{
	float d = orc_f16_to_f32(rd16(b));
	float dmin = orc_f16_to_f32(rd16(b + 2));
	const uint8_t *sc = b + 4, *qs = b + 16;

	for (int g = 0; g < 8; g++) {
		int s, m;
		q4k_scale_min(g, sc, &s, &m);
		float d1 = d * (float)s, m1 = dmin * (float)m;
		const uint8_t *q = qs + 32 * (g / 2);
		int hi = g & 1;
		for (int l = 0; l < 32; l++) {
			int qv = hi ? (q[l] >> 4) : (q[l] & 0xF);
			y[32 * g + l] = d1 * (float)qv - m1;
		}
	}
}

/* Value v of a Q6_K super-block: half h = v / 128, r = v % 128, quarter
 * t = r / 32, l = r % 32. Low 4 bits from ql[64h + l + 32 * (t & 1)]
 * (low nibble for t < 2, high for t >= 2); high 2 bits from
 * qh[32h + l] >> (2t). q = bits - 32; scale index v / 16.
 * y = (d * sc) * q, evaluated left to right as the reference does. */
static void
deq_q6k(const uint8_t *b, float *y)
{
	const uint8_t *ql = b, *qh = b + 128;
	const int8_t *sc = (const int8_t *)(b + 192);
	float d = orc_f16_to_f32(rd16(b + 208));

	for (int v = 0; v < QK_K; v++) {
		int h = v / 128, r = v % 128, t = r / 32, l = r % 32;
		int lo = ql[64 * h + l + 32 * (t & 1)];
		lo = t < 2 ? (lo & 0xF) : (lo >> 4);
		int hb = (qh[32 * h + l] >> (2 * t)) & 3;
		int q = (lo | (hb << 4)) - 32;
		y[v] = d * (float)sc[v / 16] * (float)q;
	}
}

static void
deq_q8_0(const uint8_t *b, float *y)
{
	float d = orc_f16_to_f32(rd16(b));
	const int8_t *q = (const int8_t *)(b + 2);

	for (int l = 0; l < 32; l++)
		y[l] = d * (float)q[l];
}

int
orc_dequantize_row(int type, const void *src, float *dst, int64_t n)
{
	const uint8_t *p = (const uint8_t *)src;

	switch (type) {
	case ORC_F32:
		memcpy(dst, src, (size_t)n * 4);
		return 0;
	case ORC_F16:
		orc_f16_to_f32_row((const uint16_t *)src, dst, n);
		return 0;
	case ORC_Q4_K:
		if (n % QK_K)
			return -1;
		for (int64_t i = 0; i < n / QK_K; i++)
			deq_q4k(p + i * Q4K_BYTES, dst + i * QK_K);
		return 0;
	case ORC_Q6_K:
		if (n % QK_K)
			return -1;
		for (int64_t i = 0; i < n / QK_K; i++)
			deq_q6k(p + i * Q6K_BYTES, dst + i * QK_K);
		return 0;
	case ORC_Q8_0:
		if (n % 32)
			return -1;
		for (int64_t i = 0; i < n / 32; i++)
			deq_q8_0(p + i * Q8_0_BYTES, dst + i * 32);
		return 0;
	}
	return -1;
}

static int
clampi(int v, int lo, int hi)
{
	return v < lo ? lo : v > hi ? hi : v;
}

/* Own Q4_K quantizer: per 32-group affine range [min(0, lo), hi], 6-bit
 * scales and mins relative to the super-block maxima. */
static void
quant_q4k(const float *x, uint8_t *b)
{
	float scale[8], mins[8], ms = 0, mm = 0;

	for (int g = 0; g < 8; g++) {
		float lo = x[32 * g], hi = x[32 * g];
		for (int l = 1; l < 32; l++) {
			lo = fminf(lo, x[32 * g + l]);
			hi = fmaxf(hi, x[32 * g + l]);
		}
		if (lo > 0)
			lo = 0;
		scale[g] = (hi - lo) / 15.0f;
		mins[g] = -lo;
		ms = fmaxf(ms, scale[g]);
		mm = fmaxf(mm, mins[g]);
	}
	uint16_t hd = orc_f32_to_f16(ms / 63.0f), hm = orc_f32_to_f16(mm / 63.0f);
	float d = orc_f16_to_f32(hd), dmin = orc_f16_to_f32(hm);
	int sc[8], mn[8];
	for (int g = 0; g < 8; g++) {
		sc[g] = d > 0 ? clampi((int)lrintf(scale[g] / d), 0, 63) : 0;
		mn[g] = dmin > 0 ? clampi((int)lrintf(mins[g] / dmin), 0, 63) : 0;
	}
	memset(b, 0, Q4K_BYTES);
	wr16(b, hd);
	wr16(b + 2, hm);
	uint8_t *s = b + 4, *qs = b + 16;
	for (int j = 0; j < 8; j++) {
		if (j < 4) {
			s[j] |= (uint8_t)sc[j];
			s[j + 4] |= (uint8_t)mn[j];
		} else {
			s[j + 4] = (uint8_t)((sc[j] & 0xF) | ((mn[j] & 0xF) << 4));
			s[j - 4] |= (uint8_t)((sc[j] >> 4) << 6);
			s[j] |= (uint8_t)((mn[j] >> 4) << 6);
		}
	}
	for (int g = 0; g < 8; g++) {
		float d1 = d * (float)sc[g], m1 = dmin * (float)mn[g];
		for (int l = 0; l < 32; l++) {
			int q = d1 > 0 ? clampi((int)lrintf((x[32 * g + l] + m1) / d1), 0, 15) : 0;
			int byte = 32 * (g / 2) + l;
			qs[byte] |= (uint8_t)(g & 1 ? q << 4 : q);
		}
	}
}

/* Own Q6_K quantizer: symmetric 16-groups, 8-bit signed scales. */
static void
quant_q6k(const float *x, uint8_t *b)
{
	float gs[16], ms = 0;

	for (int g = 0; g < 16; g++) {
		float a = 0;
		for (int l = 0; l < 16; l++)
			a = fmaxf(a, fabsf(x[16 * g + l]));
		gs[g] = a / 31.0f;
		ms = fmaxf(ms, gs[g]);
	}
	uint16_t hd = orc_f32_to_f16(ms / 127.0f);
	float d = orc_f16_to_f32(hd);
	memset(b, 0, Q6K_BYTES);
	int8_t *sc = (int8_t *)(b + 192);
	for (int g = 0; g < 16; g++)
		sc[g] = (int8_t)(d > 0 ? clampi((int)lrintf(gs[g] / d), -128, 127) : 0);
	uint8_t *ql = b, *qh = b + 128;
	for (int v = 0; v < QK_K; v++) {
		float s = d * (float)sc[v / 16];
		int q = s > 0 ? clampi((int)lrintf(x[v] / s), -32, 31) : 0;
		int u = q + 32;
		int h = v / 128, r = v % 128, t = r / 32, l = r % 32;
		int idx = 64 * h + l + 32 * (t & 1);
		ql[idx] |= (uint8_t)(t < 2 ? (u & 0xF) : ((u & 0xF) << 4));
		qh[32 * h + l] |= (uint8_t)(((u >> 4) & 3) << (2 * t));
	}
	wr16(b + 208, hd);
}

static void
quant_q8_0(const float *x, uint8_t *b)
{
	float a = 0;

	for (int l = 0; l < 32; l++)
		a = fmaxf(a, fabsf(x[l]));
	float d = a / 127.0f;
	uint16_t hd = orc_f32_to_f16(d);
	float id = d > 0 ? 1.0f / d : 0.0f;
	wr16(b, hd);
	for (int l = 0; l < 32; l++)
		((int8_t *)(b + 2))[l] = (int8_t)clampi((int)lrintf(x[l] * id), -127, 127);
}

int64_t
orc_quantize_row(int type, const float *src, void *dst, int64_t n)
{
	uint8_t *p = (uint8_t *)dst;

	switch (type) {
	case ORC_F32:
		memcpy(dst, src, (size_t)n * 4);
		return n * 4;
	case ORC_F16:
		orc_f32_to_f16_row(src, (uint16_t *)dst, n);
		return n * 2;
	case ORC_Q4_K:
		if (n % QK_K)
			return -1;
		for (int64_t i = 0; i < n / QK_K; i++)
			quant_q4k(src + i * QK_K, p + i * Q4K_BYTES);
		return n / QK_K * Q4K_BYTES;
	case ORC_Q6_K:
		if (n % QK_K)
			return -1;
		for (int64_t i = 0; i < n / QK_K; i++)
			quant_q6k(src + i * QK_K, p + i * Q6K_BYTES);
		return n / QK_K * Q6K_BYTES;
	case ORC_Q8_0:
		if (n % 32)
			return -1;
		for (int64_t i = 0; i < n / 32; i++)
			quant_q8_0(src + i * 32, p + i * Q8_0_BYTES);
		return n / 32 * Q8_0_BYTES;
	}
	return -1;
}

/* ---- ops ----------------------------------------------------------------- */

static int
nthreads(int n)
{
	return n > 0 ? n : 1;
}

/* sum_k a[k] b[k] in f64: eight f64 lanes (k mod 8) added pairwise at the
 * end, then the tail in order. */
typedef double orc_v4d __attribute__((vector_size(32)));
typedef float orc_v4f __attribute__((vector_size(16)));

static double
dot_f64(const float *a, const float *b, int64_t K)
{
	orc_v4d s0 = {0, 0, 0, 0}, s1 = {0, 0, 0, 0};
	int64_t k = 0;
	for (; k + 8 <= K; k += 8) {
		orc_v4f a0, b0, a1, b1;
		memcpy(&a0, a + k, 16);
		memcpy(&b0, b + k, 16);
		memcpy(&a1, a + k + 4, 16);
		memcpy(&b1, b + k + 4, 16);
		s0 += __builtin_convertvector(a0, orc_v4d) * __builtin_convertvector(b0, orc_v4d);
		s1 += __builtin_convertvector(a1, orc_v4d) * __builtin_convertvector(b1, orc_v4d);
	}
	double r = ((s0[0] + s1[0]) + (s0[1] + s1[1])) + ((s0[2] + s1[2]) + (s0[3] + s1[3]));
	for (; k < K; k++)
		r += (double)a[k] * (double)b[k];
	return r;
}

/* ggml_mul_mat via graph:mul_mat (src/lgml.c:1811-1839): y[n][m] =
 * sum_k w[m][k] * x[n][k]. Each weight row is dequantized once. */
int
orc_mul_mat(int type, const void *w, int64_t M, int64_t K, const float *x, int64_t N,
    float *y, int n_threads)
{
	/* rows in blocks of RB, dequantized together, so that each X row is
	 * read once per block (the per-output sums are unchanged) */
	enum { RB = 8 };
	int64_t rs = orc_row_size(type, K);
	int bad = 0;

	if (rs <= 0)
		return -1;
#pragma omp parallel num_threads(nthreads(n_threads))
	{
		float *rows = malloc((size_t)K * RB * sizeof(float));
		if (!rows) {
#pragma omp atomic write
			bad = 1;
		}
#pragma omp for schedule(static)
		for (int64_t m0 = 0; m0 < M; m0 += RB) {
			if (!rows)
				continue;
			int64_t nr = M - m0 < RB ? M - m0 : RB;
			for (int64_t r = 0; r < nr; r++)
				orc_dequantize_row(type, (const uint8_t *)w + (m0 + r) * rs, rows + r * K, K);
			for (int64_t n = 0; n < N; n++)
				for (int64_t r = 0; r < nr; r++)
					y[n * M + m0 + r] = (float)dot_f64(rows + r * K, x + n * K, K);
		}
		free(rows);
	}
	return bad ? -1 : 0;
}

/* ---- ggml's CPU arithmetic for quantized weights ---------------------------
 * [ggml] mul_mat on the CPU backend (what graph:mul_mat, src/lgml.c:1811-1839,
 * runs there) first converts each X row to the weight type's vec_dot_type and
 * then takes integer dot products block by block:
 *   Q4_K, Q6_K -> Q8_K: 256-value blocks {f32 d; int8 q[256]; int16 bsums[16]}
 *                 (quantize_row_q8_K_ref): amax = largest |x| (its first
 *                 occurrence gives the signed max), iscale = -127 / max,
 *                 q = min(127, nearest(iscale * x)) (round half to even),
 *                 bsums = sums of 16 q, d = 1 / iscale; an all-zero block
 *                 has d = 0 and q = 0.
 *   Q8_0       -> Q8_0: 32-value blocks {f16 d; int8 q[32]}
 *                 (quantize_row_q8_0_ref): d = amax / 127, id = d ? 1/d : 0,
 *                 q = roundf(x * id), d stored as f16.
 * The block dots (ggml_vec_dot_q4_K_q8_K, _q6_K_q8_K, _q8_0_q8_0):
 *   Q4_K: d_w d_x * sum_g sc_g sum(q x8) - dmin_w d_x * sum_g m_g (bsum_2g + bsum_2g+1)
 *   Q6_K: d_w d_x * sum_j sc_j sum_16 ((u - 32) x8)
 *   Q8_0: f16(d_w) f16(d_x) * sum(q_w q_x)
 * Integer parts are exact (int64 here); the scale products are f32 as in
 * ggml, and the blocks add in f64. ggml's SIMD variants add the per-block
 * f32 terms in other orders, so this matches them to f32 rounding, not bit
 * for bit; parity against ggml itself is unpinned (no fixture holds its
 * quantized-weight outputs). */

/* nearest(v) = round half to even, as ggml's nearest_int (|v| < 2^22). */
static int
nearest_even(float v)
{
	return (int)lrintf(v);
}

void
orc_quantize_q8_K(const float *x, int64_t K, int8_t *q, float *d, int16_t *bsums)
{
	for (int64_t b = 0; b < K / QK_K; b++) {
		const float *xb = x + b * QK_K;
		int8_t *qb = q + b * QK_K;
		float amax = 0, max = 0;
		for (int j = 0; j < QK_K; j++) {
			float ax = fabsf(xb[j]);
			if (ax > amax) {
				amax = ax;
				max = xb[j];
			}
		}
		if (amax == 0) {
			d[b] = 0;
			memset(qb, 0, QK_K);
			for (int j = 0; j < 16; j++)
				bsums[b * 16 + j] = 0;
			continue;
		}
		const float iscale = -127.0f / max;
		for (int j = 0; j < QK_K; j++) {
			int v = nearest_even(iscale * xb[j]);
			qb[j] = (int8_t)(v < 127 ? v : 127);
		}
		for (int j = 0; j < 16; j++) {
			int s = 0;
			for (int l = 0; l < 16; l++)
				s += qb[16 * j + l];
			bsums[b * 16 + j] = (int16_t)s;
		}
		d[b] = 1.0f / iscale;
	}
}

void
orc_quantize_q8_0_act(const float *x, int64_t K, int8_t *q, uint16_t *d)
{
	for (int64_t b = 0; b < K / 32; b++) {
		const float *xb = x + b * 32;
		float amax = 0;
		for (int j = 0; j < 32; j++)
			amax = fmaxf(amax, fabsf(xb[j]));
		const float dd = amax / 127.0f;
		const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
		d[b] = orc_f32_to_f16(dd);
		for (int j = 0; j < 32; j++)
			q[b * 32 + j] = (int8_t)roundf(xb[j] * id);
	}
}

/* One X row quantized for weight `type`. */
typedef struct {
	int8_t *q;
	float *d;       /* Q8_K: K/256 d; Q8_0: K/32 f16 d as f32 */
	int16_t *bsums; /* Q8_K: K/16 */
} xq_row;

static void
xq_quantize(int type, const float *x, int64_t K, xq_row *r)
{
	if (type == ORC_Q8_0) {
		uint16_t *h = malloc(sizeof(uint16_t) * (size_t)(K / 32));
		orc_quantize_q8_0_act(x, K, r->q, h);
		for (int64_t b = 0; b < K / 32; b++)
			r->d[b] = orc_f16_to_f32(h[b]);
		free(h);
	} else {
		orc_quantize_q8_K(x, K, r->q, r->d, r->bsums);
	}
}

/* sum over K of one weight row (raw blocks) with one quantized X row. */
static double
dot_q8(int type, const uint8_t *w, int64_t K, const xq_row *x)
{
	double acc = 0;

	if (type == ORC_Q8_0) {
		for (int64_t b = 0; b < K / 32; b++) {
			const uint8_t *blk = w + b * Q8_0_BYTES;
			const int8_t *qw = (const int8_t *)(blk + 2), *qx = x->q + b * 32;
			int64_t s = 0;
			for (int l = 0; l < 32; l++)
				s += (int64_t)qw[l] * qx[l];
			const float dd = orc_f16_to_f32(rd16(blk)) * x->d[b];
			acc += (double)dd * (double)s;
		}
		return acc;
	}
	for (int64_t b = 0; b < K / QK_K; b++) {
		const int8_t *qx = x->q + b * QK_K;
		if (type == ORC_Q4_K) {
			const uint8_t *blk = w + b * Q4K_BYTES, *qs = blk + 16;
			int64_t I = 0, Mn = 0;
			for (int g = 0; g < 8; g++) {
				int sc, mn;
				q4k_scale_min(g, blk + 4, &sc, &mn);
				const uint8_t *qq = qs + 32 * (g / 2);
				int64_t s = 0;
				for (int l = 0; l < 32; l++) {
					int qv = (g & 1) ? (qq[l] >> 4) : (qq[l] & 0xF);
					s += (int64_t)qv * qx[32 * g + l];
				}
				I += sc * s;
				Mn += (int64_t)mn * (x->bsums[b * 16 + 2 * g] + x->bsums[b * 16 + 2 * g + 1]);
			}
			const float d = orc_f16_to_f32(rd16(blk)) * x->d[b];
			const float dm = orc_f16_to_f32(rd16(blk + 2)) * x->d[b];
			acc += (double)d * (double)I - (double)dm * (double)Mn;
		} else { /* Q6_K */
			const uint8_t *blk = w + b * Q6K_BYTES, *ql = blk, *qh = blk + 128;
			const int8_t *sc = (const int8_t *)(blk + 192);
			int64_t I = 0;
			for (int j = 0; j < 16; j++) {
				int64_t s = 0;
				for (int l = 0; l < 16; l++) {
					int v = 16 * j + l, h = v / 128, r = v % 128, t = r / 32, ll = r % 32;
					int lo = ql[64 * h + ll + 32 * (t & 1)];
					lo = t < 2 ? (lo & 0xF) : (lo >> 4);
					int hb = (qh[32 * h + ll] >> (2 * t)) & 3;
					s += (int64_t)((lo | (hb << 4)) - 32) * qx[v];
				}
				I += sc[j] * s;
			}
			const float d = orc_f16_to_f32(rd16(blk + 208)) * x->d[b];
			acc += (double)d * (double)I;
		}
	}
	return acc;
}

int
orc_mul_mat_q8(int type, const void *w, int64_t M, int64_t K, const float *x, int64_t N,
    float *y, int n_threads)
{
	int64_t rs = orc_row_size(type, K);
	int64_t bs = type == ORC_Q8_0 ? 32 : QK_K;

	if (type == ORC_F32)
		return orc_mul_mat(type, w, M, K, x, N, y, n_threads);
	if (rs <= 0 || (type != ORC_Q4_K && type != ORC_Q6_K && type != ORC_Q8_0) || K % bs)
		return -1;
	int8_t *q = malloc((size_t)(N * K + 1));
	float *d = malloc(sizeof(float) * (size_t)(N * (K / bs) + 1));
	int16_t *bsum = malloc(sizeof(int16_t) * (size_t)(N * (K / 16) + 1));
	if (!q || !d || !bsum) {
		free(q);
		free(d);
		free(bsum);
		return -1;
	}
	for (int64_t n = 0; n < N; n++) {
		xq_row r = {q + n * K, d + n * (K / bs), bsum + n * (K / 16)};
		xq_quantize(type, x + n * K, K, &r);
	}
#pragma omp parallel for schedule(static) num_threads(nthreads(n_threads))
	for (int64_t m = 0; m < M; m++) {
		const uint8_t *wr = (const uint8_t *)w + m * rs;
		for (int64_t n = 0; n < N; n++) {
			xq_row r = {q + n * K, d + n * (K / bs), bsum + n * (K / 16)};
			y[n * M + m] = (float)dot_q8(type, wr, K, &r);
		}
	}
	free(q);
	free(d);
	free(bsum);
	return 0;
}

/* ggml_rms_norm [ggml] via graph:rms_norm (src/lgml.c:1633): sum of
 * squares in f64, mean rounded to f32, scale = 1/sqrtf(mean + eps). */
static void
rms_norm_row(const float *x, float *y, int64_t n, float eps, const float *w)
{
	double s = 0;
	for (int64_t i = 0; i < n; i++)
		s += (double)x[i] * (double)x[i];
	float mean = (float)(s / (double)n);
	float scale = 1.0f / sqrtf(mean + eps);
	for (int64_t i = 0; i < n; i++) {
		float v = x[i] * scale;
		y[i] = w ? v * w[i] : v;
	}
}

/* ggml_rope_ext [ggml] as graph:rope calls it (src/lgml.c:2004-2081),
 * ext_factor 0, freq_scale 1, attn_factor 1: theta_0 = pos, theta_{i+1} =
 * theta_i * base^(-2/n_rot) in f32; pair i rotates by theta_i / ff_i.
 * normal mode pairs (2i, 2i+1); neox pairs (i, i + n_rot/2). */
static void
rope_row(float *x, int n_heads, int D, int n_rot, int neox, float base, const float *ff,
    int pos)
{
	float theta_scale = powf(base, -2.0f / (float)n_rot);
	float cs[512], sn[512];
	float theta = (float)pos;

	for (int i = 0; i < n_rot / 2; i++) {
		float t = theta / (ff ? ff[i] : 1.0f);
		cs[i] = cosf(t);
		sn[i] = sinf(t);
		theta *= theta_scale;
	}
	for (int h = 0; h < n_heads; h++) {
		float *v = x + (int64_t)h * D;
		for (int i = 0; i < n_rot / 2; i++) {
			int a = neox ? i : 2 * i, b = neox ? i + n_rot / 2 : 2 * i + 1;
			double x0 = v[a], x1 = v[b];
			v[a] = (float)(x0 * cs[i] - x1 * sn[i]);
			v[b] = (float)(x0 * sn[i] + x1 * cs[i]);
		}
	}
}

static int64_t
cell_of(const orc_batch *b, int s, int p)
{
	return (int64_t)b->block_tab[(int64_t)s * b->max_blocks + p / b->block] * b->block +
	    p % b->block;
}

/* The ring cell of position p (rows_swa = p % ring, transformer.lua:
 * 2469-2476, ring = ring_blocks * block). */
static int64_t
ring_cell_of(const orc_batch *b, int s, int p)
{
	return (int64_t)b->ring_tab[(int64_t)s * b->ring_blocks + (p / b->block) % b->ring_blocks] *
	    b->block + p % b->block;
}

int
orc_set_rows_f16(uint16_t *dst, int64_t dst_rows, int64_t row, const float *src,
    const int64_t *ids, int64_t n)
{
	for (int64_t j = 0; j < n; j++) {
		if (ids[j] < 0 || ids[j] >= dst_rows)
			return -1;
		orc_f32_to_f16_row(src + j * row, dst + ids[j] * row, row);
	}
	return 0;
}

/* The per-sequence softmax(q k^T * scale + mask) v of
 * transformer.lua:1803-1817 (M.attend) under the fill_blocks mask of
 * src/lgml.c:2936-3017: query j of sequence s (position npast + j) sees
 * the cells of positions 0..npast+j; other cells are -inf and drop out.
 * GQA: query head h reads kv head h / (H / Hkv) (src/lgml.c:1805-1809).
 * Scores and sums in f64, K and V read from f16 storage. */
static int attend(const float *q, const uint16_t *kpool, const uint16_t *vpool, int H, int Hkv,
    int D, float scale, int window, int ring, const orc_batch *b, float *out, int n_threads);

int
orc_paged_attention(const float *q, const uint16_t *kpool, const uint16_t *vpool, int H,
    int Hkv, int D, float scale, const orc_batch *b, float *out, int n_threads)
{
	return attend(q, kpool, vpool, H, Hkv, D, scale, 0, 0, b, out, n_threads);
}

int
orc_paged_attention_swa(const float *q, const uint16_t *kpool, const uint16_t *vpool, int H,
    int Hkv, int D, float scale, int window, const orc_batch *b, float *out, int n_threads)
{
	if (window < 1 || b->ring_blocks < 1 || !b->ring_tab)
		return -1;
	return attend(q, kpool, vpool, H, Hkv, D, scale, window, 1, b, out, n_threads);
}

/* With window > 0, query j (position p) sees positions max(0, p - window
 * + 1)..p only (tensor_fill_mask's window, src/lgml.c:2920-2923); with
 * ring, they are read from the sequence's ring cells. */
static int
attend(const float *q, const uint16_t *kpool, const uint16_t *vpool, int H, int Hkv, int D,
    float scale, int window, int ring, const orc_batch *b, float *out, int n_threads)
{
	int64_t N = 0;
	int64_t *off = malloc(sizeof(int64_t) * (size_t)(b->n_seq + 1));
	if (!off)
		return -1;
	for (int s = 0; s < b->n_seq; s++) {
		off[s] = N;
		N += b->seq_n[s];
	}
	off[b->n_seq] = N;
	int64_t row = (int64_t)Hkv * D;
	int G = H / Hkv;
	int bad = 0;

	f16_lut_init();
#pragma omp parallel num_threads(nthreads(n_threads))
	{
		int maxp = 0;
		for (int s = 0; s < b->n_seq; s++)
			if (b->seq_npast[s] + b->seq_n[s] > maxp)
				maxp = b->seq_npast[s] + b->seq_n[s];
		double *sc = malloc(sizeof(double) * (size_t)(maxp + 1));
		double *acc = malloc(sizeof(double) * (size_t)D);
		if (!sc || !acc) {
#pragma omp atomic write
			bad = 1;
		}
#pragma omp for schedule(dynamic, 1) collapse(2)
		for (int64_t t = 0; t < N; t++) {
			for (int h = 0; h < H; h++) {
				if (!sc || !acc)
					continue;
				int s = 0;
				while (off[s + 1] <= t)
					s++;
				int p = b->seq_npast[s] + (int)(t - off[s]);
				int kh = h / G;
				const float *qh = q + (t * H + h) * D;
				double mx = -INFINITY;
				int j0 = window > 0 && p - window + 1 > 0 ? p - window + 1 : 0;
				for (int j = j0; j <= p; j++) {
					int64_t cell = ring ? ring_cell_of(b, s, j) : cell_of(b, s, j);
					const uint16_t *kr = kpool + cell * row + (int64_t)kh * D;
					double a = 0;
					for (int d = 0; d < D; d++)
						a += (double)qh[d] * (double)f16_lut[kr[d]];
					sc[j] = a * scale;
					if (sc[j] > mx)
						mx = sc[j];
				}
				double sum = 0;
				for (int j = j0; j <= p; j++) {
					sc[j] = exp(sc[j] - mx);
					sum += sc[j];
				}
				for (int d = 0; d < D; d++)
					acc[d] = 0;
				for (int j = j0; j <= p; j++) {
					int64_t cell = ring ? ring_cell_of(b, s, j) : cell_of(b, s, j);
					const uint16_t *vr = vpool + cell * row + (int64_t)kh * D;
					double w = sc[j] / sum;
					for (int d = 0; d < D; d++)
						acc[d] += w * (double)f16_lut[vr[d]];
				}
				float *o = out + (t * H + h) * D;
				for (int d = 0; d < D; d++)
					o[d] = (float)acc[d];
			}
		}
		free(sc);
		free(acc);
	}
	free(off);
	return bad ? -1 : 0;
}

/* ALiBi slope of head h (ggml_flash_attn_ext / soft_max_ext): with
 * n = the largest power of two <= H, m0 = 2^(-max_bias / n), m1 =
 * 2^(-max_bias / 2 / n); heads below n take m0^(h + 1), the rest
 * m1^(2 (h - n) + 1). 1 when max_bias is 0. */
static float
alibi_slope(int h, int H, float max_bias)
{
	if (max_bias <= 0.0f)
		return 1.0f;
	int n = 1;
	while (n * 2 <= H)
		n *= 2;
	const float m0 = powf(2.0f, -max_bias / (float)n);
	const float m1 = powf(2.0f, -(max_bias / 2.0f) / (float)n);
	return h < n ? powf(m0, (float)(h + 1)) : powf(m1, (float)(2 * (h - n) + 1));
}

int
orc_flash_attn(const float *q, int H, int T, int D, const uint16_t *k, const uint16_t *v,
    int Hkv, int n_kv, int64_t k_rs, int64_t k_hs, int64_t v_rs, int64_t v_hs,
    const uint16_t *mask, int mask_heads, int mask_rows, float scale, float max_bias,
    float softcap, float *out, int n_threads)
{
	if (H <= 0 || Hkv <= 0 || H % Hkv || T < 0 || D <= 0 || n_kv < 0 ||
	    (mask && (mask_heads <= 0 || H % mask_heads || mask_rows < T)) ||
	    (!mask && max_bias > 0.0f))
		return -1;
	const int G = H / Hkv;
	int bad = 0;

	f16_lut_init();
#pragma omp parallel num_threads(nthreads(n_threads))
	{
		double *sc = malloc(sizeof(double) * (size_t)(n_kv + 1));
		double *acc = malloc(sizeof(double) * (size_t)D);
		if (!sc || !acc) {
#pragma omp atomic write
			bad = 1;
		}
#pragma omp for schedule(dynamic, 1) collapse(2)
		for (int t = 0; t < T; t++) {
			for (int h = 0; h < H; h++) {
				if (!sc || !acc)
					continue;
				const int kh = h / G;
				const float *qh = q + ((int64_t)h * T + t) * D;
				const uint16_t *mr = mask ? mask + ((int64_t)(h % mask_heads) * mask_rows +
				    t) * n_kv : NULL;
				const float slope = alibi_slope(h, H, max_bias);
				double mx = -INFINITY;
				for (int j = 0; j < n_kv; j++) {
					const float mv = mr ? orc_f16_to_f32(mr[j]) : 0.0f;
					if (mv == -INFINITY) {
						sc[j] = -INFINITY;
						continue;
					}
					const uint16_t *kr = k + (int64_t)kh * k_hs + (int64_t)j * k_rs;
					double a = 0;
					for (int d = 0; d < D; d++)
						a += (double)qh[d] * (double)f16_lut[kr[d]];
					a *= scale;
					if (softcap > 0.0f)
						a = (double)softcap * tanh(a / softcap);
					sc[j] = a + (double)slope * mv;
					if (sc[j] > mx)
						mx = sc[j];
				}
				double sum = 0;
				for (int j = 0; j < n_kv; j++) {
					sc[j] = sc[j] == -INFINITY ? 0.0 : exp(sc[j] - mx);
					sum += sc[j];
				}
				for (int d = 0; d < D; d++)
					acc[d] = 0;
				for (int j = 0; j < n_kv && sum > 0; j++) {
					if (sc[j] == 0.0)
						continue;
					const uint16_t *vr = v + (int64_t)kh * v_hs + (int64_t)j * v_rs;
					const double w = sc[j] / sum;
					for (int d = 0; d < D; d++)
						acc[d] += w * (double)f16_lut[vr[d]];
				}
				float *o = out + ((int64_t)t * H + h) * D;
				for (int d = 0; d < D; d++)
					o[d] = (float)acc[d];
			}
		}
		free(sc);
		free(acc);
	}
	return bad ? -1 : 0;
}

int
orc_moe_route(const float *logits, int64_t n, int n_expert, int n_used, int gating,
    int norm_topk, float scale, int32_t *ids, float *w)
{
	if (n_expert <= 0 || n_used < 1 || n_used > n_expert ||
	    (gating != ORC_GATING_SOFTMAX && gating != ORC_GATING_SIGMOID))
		return -1;
	float *p = malloc(sizeof(float) * (size_t)n_expert);
	char *taken = malloc((size_t)n_expert);
	if (!p || !taken) {
		free(p);
		free(taken);
		return -1;
	}
	for (int64_t t = 0; t < n; t++) {
		const float *l = logits + t * n_expert;
		/* probs: ggml soft_max / sigmoid of the row */
		if (gating == ORC_GATING_SOFTMAX) {
			double mx = -INFINITY, sum = 0;
			for (int e = 0; e < n_expert; e++)
				if (l[e] > mx)
					mx = l[e];
			for (int e = 0; e < n_expert; e++)
				sum += exp((double)l[e] - mx);
			for (int e = 0; e < n_expert; e++)
				p[e] = (float)(exp((double)l[e] - mx) / sum);
		} else {
			for (int e = 0; e < n_expert; e++)
				p[e] = (float)(1.0 / (1.0 + exp(-(double)l[e])));
		}
		/* argsort_top_k: the n_used largest, largest first */
		memset(taken, 0, (size_t)n_expert);
		for (int j = 0; j < n_used; j++) {
			int best = -1;
			for (int e = 0; e < n_expert; e++)
				if (!taken[e] && (best < 0 || l[e] > l[best]))
					best = e;
			taken[best] = 1;
			ids[t * n_used + j] = best;
			w[t * n_used + j] = p[best];
		}
		/* w / clamp(sum_rows(w), 6.103515625e-5, inf) (:2003-2005) */
		if (norm_topk) {
			double s = 0;
			for (int j = 0; j < n_used; j++)
				s += w[t * n_used + j];
			float sf = (float)s;
			if (sf < 6.103515625e-5f)
				sf = 6.103515625e-5f;
			for (int j = 0; j < n_used; j++)
				w[t * n_used + j] = w[t * n_used + j] / sf;
		}
		if (scale != 1.0f)
			for (int j = 0; j < n_used; j++)
				w[t * n_used + j] = w[t * n_used + j] * scale;
	}
	free(p);
	free(taken);
	return 0;
}

/* The picks of each expert gathered into one orc_mul_mat call, so each
 * expert row is dequantized once per call. */
static int
mul_mat_id_mode(int type, const void *w, int64_t n_expert, int64_t M, int64_t K,
    const float *x, int64_t U, const int32_t *ids, int64_t T, int n_used, float *y,
    int n_threads, int act)
{
	int64_t rs = orc_row_size(type, K), P = T * n_used;
	int rc = 0;

	if (rs <= 0 || U < 1 || n_used % U)
		return -1;
	for (int64_t p = 0; p < P; p++)
		if (ids[p] < 0 || ids[p] >= n_expert)
			return -1;
	float *xg = malloc(sizeof(float) * (size_t)(P * K + 1));
	float *yg = malloc(sizeof(float) * (size_t)(P * M + 1));
	int64_t *which = malloc(sizeof(int64_t) * (size_t)(P + 1));
	if (!xg || !yg || !which) {
		rc = -1;
		goto done;
	}
	for (int64_t e = 0; e < n_expert; e++) {
		int64_t c = 0;
		for (int64_t p = 0; p < P; p++) {
			if (ids[p] != e)
				continue;
			int64_t t = p / n_used, j = p % n_used;
			memcpy(xg + c * K, x + (t * U + j % U) * K, sizeof(float) * (size_t)K);
			which[c++] = p;
		}
		if (!c)
			continue;
		if ((act ? orc_mul_mat_q8 : orc_mul_mat)(type, (const uint8_t *)w + e * M * rs, M, K,
		    xg, c, yg, n_threads)) {
			rc = -1;
			goto done;
		}
		for (int64_t i = 0; i < c; i++)
			memcpy(y + which[i] * M, yg + i * M, sizeof(float) * (size_t)M);
	}
done:
	free(xg);
	free(yg);
	free(which);
	return rc;
}

int
orc_mul_mat_id(int type, const void *w, int64_t n_expert, int64_t M, int64_t K,
    const float *x, int64_t U, const int32_t *ids, int64_t T, int n_used, float *y,
    int n_threads)
{
	return mul_mat_id_mode(type, w, n_expert, M, K, x, U, ids, T, n_used, y, n_threads, 0);
}

int
orc_mul_mat_id_q8(int type, const void *w, int64_t n_expert, int64_t M, int64_t K,
    const float *x, int64_t U, const int32_t *ids, int64_t T, int n_used, float *y,
    int n_threads)
{
	return mul_mat_id_mode(type, w, n_expert, M, K, x, U, ids, T, n_used, y, n_threads, 1);
}

int32_t
orc_argmax(const float *v, int64_t n)
{
	int64_t best = 0;
	float m = v[0];

	for (int64_t i = 1; i < n; i++) {
		if (v[i] > m) {
			m = v[i];
			best = i;
		}
	}
	return (int32_t)best;
}

static void
embed_rows(const orc_tensor *t, int64_t E, const int32_t *ids, int64_t N, float *x)
{
	int64_t rs = orc_row_size(t->type, E);
	for (int64_t i = 0; i < N; i++)
		orc_dequantize_row(t->type, (const uint8_t *)t->data + ids[i] * rs, x + i * E, E);
}

/* A weight product of the forward: with act_quant set, a quantized weight
 * takes ggml's CPU arithmetic (X in the weight's vec_dot_type, integer
 * block dots; orc_mul_mat_q8), f32 weights stay exact either way. */
static int
mm(const orc_model *m, const orc_tensor *w, int64_t M, int64_t K, const float *x, int64_t N,
    float *y, int nt)
{
	if (m->act_quant && w->type != ORC_F32)
		return orc_mul_mat_q8(w->type, w->data, M, K, x, N, y, nt);
	return orc_mul_mat(w->type, w->data, M, K, x, N, y, nt);
}

static int
mm_id(const orc_model *m, int type, const void *w, int64_t NE, int64_t M, int64_t K, const float *x, int64_t U,
    const int32_t *ids, int64_t T, int n_used, float *y, int nt)
{
	return mul_mat_id_mode(type, w, NE, M, K, x, U, ids, T, n_used, y, nt,
	    m->act_quant && type != ORC_F32);
}

/* The routed-expert FFN (transformer.lua:2054-2068 with M.moe :1989-2027,
 * experts :1875-1889, sum_picks :1894-1910) on the normed rows h; adds
 * the weighted sum of the picks to x (the residual add of :2079). */
static int
moe_ffn(const orc_model *m, const orc_layer *L, const float *h, int64_t N, float *x, int nt)
{
	const int64_t E = m->n_embd, NE = m->n_expert, K = m->n_used, F = m->n_ff_exp;
	const int64_t P = N * K;
	int rc = -1;
	float *lg = malloc(sizeof(float) * (size_t)(N * NE));
	int32_t *ids = malloc(sizeof(int32_t) * (size_t)P);
	float *w = malloc(sizeof(float) * (size_t)P);
	float *g = malloc(sizeof(float) * (size_t)(P * F));
	float *u = malloc(sizeof(float) * (size_t)(P * F));
	float *dn = malloc(sizeof(float) * (size_t)(P * E));

	if (!lg || !ids || !w || !g || !u || !dn)
		goto done;
	if (mm(m, &L->gate_inp, NE, E, h, N, lg, nt) ||
	    orc_moe_route(lg, N, (int)NE, (int)K, m->gating, m->norm_topk, m->expert_scale, ids, w) ||
	    mm_id(m, L->gate_exps.type, L->gate_exps.data, NE, F, E, h, 1, ids, N, (int)K, g, nt) ||
	    mm_id(m, L->up_exps.type, L->up_exps.data, NE, F, E, h, 1, ids, N, (int)K, u, nt))
		goto done;
	/* swiglu_split: silu(gate) * up */
	for (int64_t i = 0; i < P * F; i++) {
		double gv = g[i];
		g[i] = (float)(gv / (1.0 + exp(-gv)) * (double)u[i]);
	}
	if (mm_id(m, L->down_exps.type, L->down_exps.data, NE, E, F, g, K, ids, N, (int)K, dn,
	    nt))
		goto done;
	/* mul by the weights, then the picks added in order, then x */
	for (int64_t t = 0; t < N; t++)
		for (int64_t e = 0; e < E; e++) {
			double s = 0;
			for (int64_t j = 0; j < K; j++)
				s += (double)(dn[(t * K + j) * E + e] * w[t * K + j]);
			x[t * E + e] = (float)s + x[t * E + e];
		}
	rc = 0;
done:
	free(lg);
	free(ids);
	free(w);
	free(g);
	free(u);
	free(dn);
	return rc;
}

/* ggml_gelu [ggml] (the tanh form): 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))),
 * as geglu_split applies it to the gate (src/ops_nn.c:165-172). */
static double
gelu(double x)
{
	return 0.5 * x * (1.0 + tanh(0.7978845608028654 * (x + 0.044715 * x * x * x)));
}

/* The ops of the forward exported one by one, for tests of the device's
 * standalone entry points: rms_norm_row over rows (graph:rms_norm,
 * src/lgml.c:1633), rope_row over rows of heads at positions (graph:rope,
 * src/lgml.c:2004-2081), and the GLU of ffn (transformer.lua:2048:
 * silu(g) u, or gemma's gelu(g) u) in f64, rounded once. */
void
orc_rms_norm(const float *x, float *y, int64_t rows, int64_t n, float eps, const float *w)
{
	for (int64_t r = 0; r < rows; r++)
		rms_norm_row(x + r * n, y + r * n, n, eps, w);
}

void
orc_rope(float *x, int64_t rows, int n_heads, int D, int n_rot, int neox, float base,
    const float *ff, const int32_t *pos)
{
	for (int64_t r = 0; r < rows; r++)
		rope_row(x + r * n_heads * D, n_heads, D, n_rot, neox, base, ff, pos[r]);
}

void
orc_glu(const float *g, const float *u, float *out, int64_t n, int use_gelu)
{
	for (int64_t i = 0; i < n; i++) {
		double gv = g[i];
		double a = use_gelu ? gelu(gv) : gv / (1.0 + exp(-gv));
		out[i] = (float)(a * (double)u[i]);
	}
}

/* transformer.lua:2285-2365 (forward) with qkv (:1754-1789), the batched
 * attention (:2389-2416: set_rows into the pool or, for sliding layers, the
 * ring, then attend per sequence), attn_out (:1859-1872), ffn (:2042-2080),
 * and head (:2094-2104) on the rows of logit_rows (:2349-2350). llama /
 * qwen3 layers with a dense FFN, qwen3moe layers with routed experts
 * (moe_ffn), gemma layers (embedding scale :2304-2306, V rms-normed
 * :1782-1784, post norms :1866-1868,2070-2072, GeGLU :2048, layer output
 * scale :2334-2336, logit softcap :2097-2099). Every matrix is an f32 or
 * quantized weight. */
int
orc_forward(const orc_model *m, uint16_t *const *kpool, uint16_t *const *vpool,
    int64_t cap, const orc_batch *b, float *logits, int nt)
{
	const int64_t E = m->n_embd, H = m->n_head, F = m->n_ff, V = m->n_vocab;
	int64_t N = 0, Dmax = m->head_dim, HKmax = m->n_head_kv;
	int rc = 0;

	for (int s = 0; s < b->n_seq; s++)
		N += b->seq_n[s];
	if (N == 0)
		return 0;
	for (int il = 0; il < m->n_layer; il++) {
		const orc_layer *L = &m->layers[il];
		if (L->head_dim > Dmax)
			Dmax = L->head_dim;
		if (L->n_head_kv > HKmax)
			HKmax = L->n_head_kv;
	}
	const int64_t QW = H * Dmax > E ? H * Dmax : E;
	float *x = malloc(sizeof(float) * (size_t)(N * E));
	float *cur = malloc(sizeof(float) * (size_t)(N * E));
	float *q = malloc(sizeof(float) * (size_t)(N * H * Dmax));
	float *k = malloc(sizeof(float) * (size_t)(N * HKmax * Dmax));
	float *v = malloc(sizeof(float) * (size_t)(N * HKmax * Dmax));
	float *o = malloc(sizeof(float) * (size_t)(N * H * Dmax));
	float *tmp = malloc(sizeof(float) * (size_t)(N * QW));
	float *g = malloc(sizeof(float) * (size_t)(N * F));
	float *u = malloc(sizeof(float) * (size_t)(N * F));
	int32_t *pos = malloc(sizeof(int32_t) * (size_t)N);
	int64_t *cells = malloc(sizeof(int64_t) * (size_t)N);
	int64_t *rcells = malloc(sizeof(int64_t) * (size_t)N);
	if (!x || !cur || !q || !k || !v || !o || !tmp || !g || !u || !pos || !cells || !rcells) {
		rc = -1;
		goto done;
	}
	for (int s = 0, t = 0; s < b->n_seq; s++) {
		for (int j = 0; j < b->seq_n[s]; j++, t++) {
			pos[t] = b->seq_npast[s] + j;
			cells[t] = cell_of(b, s, pos[t]);
			rcells[t] = b->ring_blocks > 0 ? ring_cell_of(b, s, pos[t]) : -1;
			if (cells[t] < 0 || cells[t] >= cap || (b->ring_blocks > 0 && rcells[t] >= cap)) {
				rc = -2;
				goto done;
			}
		}
	}
	embed_rows(&m->tok_embd, E, b->ids, N, x);
	if (m->embd_scale > 0)
		for (int64_t i = 0; i < N * E; i++)
			x[i] = x[i] * m->embd_scale;
	for (int il = 0; il < m->n_layer; il++) {
		const orc_layer *L = &m->layers[il];
		const int64_t D = L->head_dim ? L->head_dim : m->head_dim;
		const int64_t Hkv = L->n_head_kv ? L->n_head_kv : m->n_head_kv;
		const int n_rot = L->n_rot ? L->n_rot : m->n_rot;
		const float base = L->rope_base > 0 ? L->rope_base : m->rope_base;
		const float *ff = L->rope_freqs ? L->rope_freqs : (m->gemma ? NULL : m->rope_freqs);
		const float scale = m->attn_scale > 0 ? m->attn_scale : 1.0f / sqrtf((float)D);
		if (L->swa && (b->ring_blocks < 1 || m->n_swa < 1)) {
			rc = -7;
			goto done;
		}
		for (int64_t t = 0; t < N; t++)
			rms_norm_row(x + t * E, cur + t * E, E, m->eps, (const float *)L->attn_norm.data);
		if (mm(m, &L->wq, H * D, E, cur, N, q, nt) || mm(m, &L->wk, Hkv * D, E, cur, N, k, nt)) {
			rc = -3;
			goto done;
		}
		if (L->wv.data) {
			if (mm(m, &L->wv, Hkv * D, E, cur, N, v, nt)) {
				rc = -3;
				goto done;
			}
		} else {
			memcpy(v, k, sizeof(float) * (size_t)(N * Hkv * D));  /* V = raw K */
		}
		for (int64_t t = 0; t < N; t++) {
			if (L->q_norm.data)
				for (int h = 0; h < H; h++)
					rms_norm_row(q + (t * H + h) * D, q + (t * H + h) * D, D, m->eps,
					    (const float *)L->q_norm.data);
			if (L->k_norm.data)
				for (int h = 0; h < Hkv; h++)
					rms_norm_row(k + (t * Hkv + h) * D, k + (t * Hkv + h) * D, D, m->eps,
					    (const float *)L->k_norm.data);
			if (m->gemma)
				for (int h = 0; h < Hkv; h++)
					rms_norm_row(v + (t * Hkv + h) * D, v + (t * Hkv + h) * D, D, m->eps,
					    NULL);
			rope_row(q + t * H * D, (int)H, (int)D, n_rot, m->rope_neox, base, ff, pos[t]);
			rope_row(k + t * Hkv * D, (int)Hkv, (int)D, n_rot, m->rope_neox, base, ff, pos[t]);
		}
		const int64_t *wc = L->swa ? rcells : cells;
		orc_set_rows_f16(kpool[il], cap, Hkv * D, k, wc, N);
		orc_set_rows_f16(vpool[il], cap, Hkv * D, v, wc, N);
		if (attend(q, kpool[il], vpool[il], (int)H, (int)Hkv, (int)D, scale,
		    L->swa ? m->n_swa : 0, L->swa, b, o, nt)) {
			rc = -4;
			goto done;
		}
		if (mm(m, &L->wo, E, H * D, o, N, tmp, nt)) {
			rc = -3;
			goto done;
		}
		if (L->post_attn_norm.data)
			for (int64_t t = 0; t < N; t++)
				rms_norm_row(tmp + t * E, tmp + t * E, E, m->eps,
				    (const float *)L->post_attn_norm.data);
		for (int64_t i = 0; i < N * E; i++)
			x[i] = tmp[i] + x[i];
		for (int64_t t = 0; t < N; t++)
			rms_norm_row(x + t * E, cur + t * E, E, m->eps, (const float *)L->ffn_norm.data);
		if (L->gate_inp.data) {
			if (moe_ffn(m, L, cur, N, x, nt)) {
				rc = -6;
				goto done;
			}
		} else {
			if (mm(m, &L->gate, F, E, cur, N, g, nt) || mm(m, &L->up, F, E, cur, N, u, nt)) {
				rc = -3;
				goto done;
			}
			for (int64_t i = 0; i < N * F; i++) {
				double gv = g[i];
				double a = m->gemma ? gelu(gv) : gv / (1.0 + exp(-gv));
				g[i] = (float)(a * (double)u[i]);
			}
			if (mm(m, &L->down, E, F, g, N, tmp, nt)) {
				rc = -3;
				goto done;
			}
			if (L->post_ffn_norm.data)
				for (int64_t t = 0; t < N; t++)
					rms_norm_row(tmp + t * E, tmp + t * E, E, m->eps,
					    (const float *)L->post_ffn_norm.data);
			for (int64_t i = 0; i < N * E; i++)
				x[i] = tmp[i] + x[i];
		}
		if (L->out_scale != 0.0f)
			for (int64_t i = 0; i < N * E; i++)
				x[i] = x[i] * L->out_scale;
	}
	for (int r = 0; r < b->n_out; r++) {
		if (b->out_rows[r] < 0 || b->out_rows[r] >= N) {
			rc = -5;
			goto done;
		}
		rms_norm_row(x + (int64_t)b->out_rows[r] * E, cur + (int64_t)r * E, E, m->eps,
		    (const float *)m->output_norm.data);
	}
	if (mm(m, &m->output, V, E, cur, b->n_out, logits, nt)) {
		rc = -3;
		goto done;
	}
	if (m->softcap > 0)
		for (int64_t i = 0; i < (int64_t)b->n_out * V; i++)
			logits[i] = (float)((double)m->softcap * tanh((double)logits[i] / m->softcap));
done:
	free(x);
	free(cur);
	free(q);
	free(k);
	free(v);
	free(o);
	free(tmp);
	free(g);
	free(u);
	free(pos);
	free(cells);
	free(rcells);
	return rc;
}
