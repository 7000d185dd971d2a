/*
 * sumsq_walk_model.c -- TEST INFRASTRUCTURE: a CPU model of the binade walk
 * of vitni-tensor_amd/csrc/vtq_sumsq.h (sumsq_walk_helper and sumsq_walk),
 * statement for statement, with the wave's 64 lanes as loops: ballots are
 * bit masks of lane predicates, readlane / readfirstlane are array reads,
 * and the DPP scans are replayed in their row_shr / row_bcast order.  It lets
 * tests/test_sumsq_walk_model.py run the walk on many rows, including rows
 * built to reach its rare branches, and compare it with the serial chain of
 * rms_norm_slice (src/ops/rms_norm.rs:96-100: sumsq += v * v in order).
 *
 * Built by the test with gcc -O2 -ffp-contract=off (IEEE binary32, no FMA,
 * denormals kept, like the kernels).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define NB 5         /* kWalkBinades */
#define MAXT 1536    /* kWalkMaxTerms */
#define MAXSTOPS 48  /* kWalkMaxStops */
#define CAP (1u << 25)

/* path flags reported per row */
enum {
    P_HELPER_FB = 1,     /* helpers chose the plain chain (non-finite, zero or tiny sums) */
    P_START_FB = 2,      /* the head's sum was outside the window */
    P_NO_EVENT = 4,      /* finished by integer arithmetic */
    P_CROSS = 8,         /* a binade crossing event */
    P_TIE = 16,          /* a tie event */
    P_NEXT_BIN = 32,     /* moved to the next binade */
    P_JUMP_BIN = 64,     /* moved two or more binades at once */
    P_LEFT_WINDOW = 128, /* left the window: chain from there */
    P_STOP_LIMIT = 256,  /* kWalkMaxStops reached */
    P_CAPPED = 512,      /* a helper total reached kWalkCap */
    P_GUARD = 1024,      /* the empty-ballot guard fired */
};

static inline uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static inline float u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

int walk_pass_index(int i) { return 4096 * (i >> 12) + 256 * ((i & 63) >> 2) + 4 * ((i >> 6) & 63) + (i & 3); }
int walk_head(int n) { return (n % 64 == 0 && n >= 1024 && n <= 4096) ? (n - MAXT > 640 ? n - MAXT : 640) : 0; }

typedef struct {
    uint32_t Q[NB][MAXT];
    uint32_t TM[NB][64];
    uint32_t WT[NB][4];
    float part[2][16];
    int elo, nb, fb;
} walk_t;

/* inclusive scans of wave_total_f32 / wave_scan_u32: row_shr 1, 2, 4, 8 inside
 * 16-lane rows (a lane without a source keeps its value), then row_bcast:15
 * into rows 1 and 3, then row_bcast:31 into rows 2 and 3 */
static void scan_f32(float v[64]) {
    float o[64];
    for (int sh = 1; sh <= 8; sh <<= 1) {
        memcpy(o, v, sizeof o);
        for (int l = 0; l < 64; l++)
            if ((l & 15) >= sh) v[l] = o[l - sh] + o[l];
    }
    memcpy(o, v, sizeof o);
    for (int l = 16; l < 64; l++)
        if ((l >> 4) == 1 || (l >> 4) == 3) v[l] = o[16 * (l >> 4) - 1] + o[l];
    memcpy(o, v, sizeof o);
    for (int l = 32; l < 64; l++) v[l] = o[31] + o[l];
}
static void scan_u32(uint32_t v[64]) {
    uint32_t o[64];
    for (int sh = 1; sh <= 8; sh <<= 1) {
        memcpy(o, v, sizeof o);
        for (int l = 0; l < 64; l++)
            if ((l & 15) >= sh) v[l] = o[l - sh] + o[l];
    }
    memcpy(o, v, sizeof o);
    for (int l = 16; l < 64; l++)
        if ((l >> 4) == 1 || (l >> 4) == 3) v[l] = o[16 * (l >> 4) - 1] + o[l];
    memcpy(o, v, sizeof o);
    for (int l = 32; l < 64; l++) v[l] = o[31] + o[l];
}

static float wave_total(const float in[64]) {
    float v[64];
    memcpy(v, in, sizeof v);
    scan_f32(v);
    return v[63];
}

/* sumsq_walk_helper for helper wave h */
static void helper(int h, const float* prod, int n, int H, walk_t* w, int* flags) {
    const int NQ = (n - H) >> 3;
    float t1[64], t2[64];
    for (int l = 0; l < 64; l++) {
        const float pp = l < 32 ? w->part[l >> 4][l & 15] : 0.0f;
        t1[l] = l < 16 ? pp : 0.0f;
        t2[l] = l >= 16 ? pp : 0.0f;
    }
    const float ah = wave_total(t1), a = wave_total(t2);
    const float lo = ah * (1.0f - 1.0f / 4096.0f), hi = a * (1.0f + 1.0f / 1024.0f);
    int elo = 0, nb = 0, fb = 0;
    const int flo = (int)(f2u(lo) >> 23) & 255, fhi = (int)(f2u(hi) >> 23) & 255;
    if (!(a < INFINITY) || !(lo > 0.0f) || flo < 30) {
        fb = 1;
    } else {
        elo = flo - 127;
        nb = fhi - flo + 1 < NB ? fhi - flo + 1 : NB;
    }
    if (h == 0) {
        w->elo = elo;
        w->nb = nb;
        w->fb = fb;
        if (fb) *flags |= P_HELPER_FB;
    }
    if (fb) return;
    uint32_t rr[64][8], loc[64][8], acc[64], tm[64], tot[64], incl[64];
    int tzm[64][8];
    for (int l = 0; l < 64; l++) {
        const int q = 64 * h + l, qc = q < NQ - 1 ? q : NQ - 1;
        const int g = H + 8 * qc, kk = g & 63, Lc = g >> 6;
        float pj[8];
        for (int c = 0; c < 4; c++) {
            pj[c] = prod[256 * (kk >> 2) + 4 * Lc + c];
            pj[4 + c] = prod[256 * ((kk >> 2) + 1) + 4 * Lc + c];
        }
        const int efb0 = elo + 127;
        for (int j = 0; j < 8; j++) {
            const uint32_t pb = f2u(pj[j]);
            const int ep = (int)(pb >> 23);
            const uint32_t mp = (pb & 0x7FFFFFu) | (ep ? 0x800000u : 0u);
            const int dm1 = efb0 - 1 - (ep > 1 ? ep : 1);
            if (dm1 >= 0) {
                rr[l][j] = mp >> (dm1 < 31 ? dm1 : 31);
            } else {
                const uint32_t sh = mp << (-dm1 < 5 ? -dm1 : 5), c = 1u << 28;
                rr[l][j] = sh < c ? sh : c;
            }
            const int tz = __builtin_ctz(mp | 0x80000000u);
            tzm[l][j] = tz <= 23 ? tz - dm1 : -1000;
        }
    }
    for (int b = 0; b < NB; b++) {
        if (b >= nb) continue;
        for (int l = 0; l < 64; l++) {
            const int q = 64 * h + l;
            acc[l] = 0;
            tm[l] = 0;
            for (int j = 0; j < 8; j++) {
                if (b > 0) rr[l][j] >>= 1;
                const int tie = tzm[l][j] == b;
                acc[l] += (rr[l][j] + (tie ? 0u : 1u)) >> 1;
                loc[l][j] = acc[l];
                tm[l] |= tie ? 1u << j : 0u;
            }
            tot[l] = q < NQ ? (acc[l] < CAP ? acc[l] : CAP) : 0u;
            if (q < NQ && acc[l] >= CAP) *flags |= P_CAPPED;
            incl[l] = tot[l];
        }
        scan_u32(incl);
        for (int l = 0; l < 64; l++) {
            const int q = 64 * h + l;
            const uint32_t ex = incl[l] - tot[l];
            if (q < NQ) {
                for (int j = 0; j < 8; j++) w->Q[b][8 * q + j] = ex + loc[l][j];
                ((uint8_t*)&w->TM[b][0])[q] = (uint8_t)tm[l];
            }
        }
        w->WT[b][h] = incl[63] < CAP ? incl[63] : CAP;
    }
}

static float chain(const float* prod, int from, int n, float run) {
    for (int i = from; i < n; i++) run = run + prod[walk_pass_index(i)];
    return run;
}

static void load_bin(const walk_t* w, int b, int NS, uint32_t v1o[64], uint32_t two[64], uint32_t* a1,
                     uint32_t* a2) {
    *a1 = w->WT[b][0];
    *a2 = *a1 + w->WT[b][1];
    for (int l = 0; l < 64; l++) {
        const uint32_t st = l < NS ? w->Q[b][32 * l + 31] : 0u;
        v1o[l] = l < NS ? st + (l >= 32 ? *a2 : l >= 16 ? *a1 : 0u) : 0u;
        two[l] = l < NS ? w->TM[b][l] : 0u;
    }
}

/* sumsq_walk from the head's sum s */
static float walk(float s, const float* prod, int n, int H, const walk_t* w, int* flags) {
    const int M = n - H, NS = M >> 5;
    const int elo = w->elo, nb = w->nb;
    int fb = w->fb != 0;
    int k = 0, stops = 0;
    uint32_t sb = f2u(s);
    int bi = (int)(sb >> 23) - 127 - elo;
    uint32_t base = 0, v1[64] = {0}, tw[64] = {0}, o1 = 0, o2 = 0;
    if (!fb) {
        if (bi < 0 || bi >= nb || (sb >> 23) < 30) {
            fb = 1;
            *flags |= P_START_FB;
        } else {
            load_bin(w, bi, NS, v1, tw, &o1, &o2);
        }
    }
    while (!fb && k < M) {
        if (stops >= MAXSTOPS) {
            fb = 1;
            *flags |= P_STOP_LIMIT;
            break;
        }
        const int ef = (int)(sb >> 23);
        const uint32_t m = (sb & 0x7FFFFFu) | 0x800000u;
        const uint32_t T = (1u << 24) - m + base;
        const float u = u2f((uint32_t)(ef - 23) << 23);
        uint32_t twm[64];
        uint64_t b1 = 0, bt = 0;
        for (int l = 0; l < 64; l++) {
            int sh = k - 32 * l;
            sh = sh < 0 ? 0 : sh > 32 ? 32 : sh;
            twm[l] = tw[l] & (uint32_t)(~0ull << sh);
            if (v1[l] >= T) b1 |= 1ull << l;
            if (twm[l] != 0u) bt |= 1ull << l;
        }
        const uint32_t c1 = b1 ? (uint32_t)__builtin_ctzll(b1) : 64u, c2 = bt ? (uint32_t)__builtin_ctzll(bt) : 64u;
        const uint32_t seg = c1 < c2 ? c1 : c2;
        if (seg >= 64) {
            sb = f2u(u2f(sb) + u * (float)(v1[NS - 1] - base));
            k = M;
            *flags |= P_NO_EVENT;
            break;
        }
        const int bn = bi + 1 < NB - 1 ? bi + 1 : NB - 1;
        uint32_t qv[64], v1n[64], twn[64], n1, n2, qt[64];
        float pv[64];
        for (int l = 0; l < 64; l++) {
            qv[l] = w->Q[l < 32 ? bi : bn][32 * seg + (l & 31)];
            const int pl = 256 * ((l & 31) >> 2) + (l & 3);
            pv[l] = prod[pl + 2048 * (seg & 1) + 4 * (H / 64 + (seg >> 1))];
        }
        load_bin(w, bn, NS, v1n, twn, &n1, &n2);
        const uint32_t wt = twm[seg];
        const int hs = (int)seg >> 4;
        for (int l = 0; l < 64; l++)
            qt[l] = qv[l] + (l < 32 ? (hs == 2 ? o2 : hs == 1 ? o1 : 0u) : (hs == 2 ? n2 : hs == 1 ? n1 : 0u));
        const int kr = k - 32 * (int)seg;
        uint64_t b2 = 0;
        for (int l = 0; l < 64; l++)
            if (l < 32 && l >= kr && (qt[l] >= T || ((wt >> (l & 31)) & 1u))) b2 |= 1ull << l;
        if (b2 == 0) {
            fb = 1;
            *flags |= P_GUARD;
            break;
        }
        const int el = __builtin_ctzll(b2);
        const int ev = 32 * (int)seg + el;
        const uint32_t qa = qt[el - 1 > 0 ? el - 1 : 0], qb = v1[(int)seg - 1 > 0 ? (int)seg - 1 : 0];
        const uint32_t qprev = el > 0 ? qa : (seg > 0 ? qb : 0u);
        const float pe = pv[el];
        *flags |= (qt[el] >= T) ? P_CROSS : P_TIE;
        const float snew = (u2f(sb) + u * (float)(qprev - base)) + pe;
        sb = f2u(snew);
        k = ev + 1;
        stops++;
        const int bi2 = (int)(sb >> 23) - 127 - elo;
        if (bi2 == bi) {
            base = qt[el];
        } else if (bi2 == bi + 1 && bi2 < nb) {
            base = qt[32 + el];
            memcpy(v1, v1n, sizeof v1);
            memcpy(tw, twn, sizeof tw);
            o1 = n1;
            o2 = n2;
            *flags |= P_NEXT_BIN;
        } else if (bi2 > bi && bi2 < nb && (sb >> 23) < 255) {
            load_bin(w, bi2, NS, v1, tw, &o1, &o2);
            const int hv = ev >> 9;
            base = w->Q[bi2][ev] + (hv == 2 ? o2 : hv == 1 ? o1 : 0u);
            *flags |= P_JUMP_BIN;
        } else {
            fb = 1;
            *flags |= P_LEFT_WINDOW;
        }
        bi = bi2;
    }
    s = u2f(sb);
    if (fb) s = chain(prod, H + k, n, s);
    return s;
}

/* The sum of squares of x[0..n) as the walk forms it (n a multiple of 64 in
 * 1024..4096), with the partial estimates of the standalone RMSNorm kernel
 * (four waves, lane-strided), the walk tables first filled with the byte
 * `stale`; flags receives the P_* bits of the path. */
float walk_sumsq(const float* x, int n, int stale, int* flags) {
    static float prod[4096];
    static walk_t w;
    const int H = walk_head(n);
    *flags = 0;
    /* the tables start as whatever the LDS held before: only what the helpers
     * write may be used */
    memset(&w, stale, sizeof w);
    for (int wv = 4; wv < 16; wv++) w.part[0][wv] = w.part[1][wv] = 0.0f;  /* no waves 4-15 */
    float hpart[256] = {0}, apart[256] = {0};
    for (int i = 0; i < n; i++) {
        const float p = x[i] * x[i];
        prod[walk_pass_index(i)] = p;
        const int t = i & 255;
        apart[t] += p;
        if (i < H) hpart[t] += p;
    }
    for (int wv = 0; wv < 4; wv++) {
        w.part[0][wv] = wave_total(hpart + 64 * wv);
        w.part[1][wv] = wave_total(apart + 64 * wv);
    }
    float s = chain(prod, 0, H, 0.0f);
    for (int h = 0; h < 3; h++) helper(h, prod, n, H, &w, flags);
    return walk(s, prod, n, H, &w, flags);
}

/* rms_norm_slice's serial sum of squares (src/ops/rms_norm.rs:96-100) */
float serial_sumsq(const float* x, int n) {
    float s = 0.0f;
    for (int i = 0; i < n; i++) s = s + x[i] * x[i];
    return s;
}
