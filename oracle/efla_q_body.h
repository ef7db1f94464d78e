/*
 * Mode Q EFLA recurrence, included twice by efla_oracle.c with REAL = double
 * (the parity reference) and REAL = float (the timed CPU baseline).
 * TEST INFRASTRUCTURE ONLY (see efla_oracle.c).
 *
 * Per (sequence, head), token-sequential (generalises efla.cu:154-233):
 *   lambda_t = ||k_t||^2, c_t = (1 - exp(-beta_t lambda_t)) / lambda_t
 *   u_t = S^T k_t,  S <- S + c_t k_t (v_t - u_t)^T,  o_t = S^T q_t
 * Backward (generalises the BPTT of efla.cu:315-454 to the q readout and a
 * per-token beta; states recomputed from checkpoints every OR_CKPT tokens):
 *   g   = G + q_t dO_t^T          (gradient w.r.t. the post-update state)
 *   dq  = S_t dO_t
 *   dr  = c g^T k                 (= dv; r = v - u)
 *   dc  = k^T g r
 *   dk  = c g r - S_{t-1} dr + 2 dc (dc/dlambda) k
 *   dbeta = dc * exp(-beta lambda)
 *   G  <- g - k dr^T
 * Layouts: q,k (tokens,H,K); v,o (tokens,H,V); beta (tokens,H); states
 * (N,H,K,V) row-major.  cu_seqlens == NULL means N sequences of length T laid
 * out back to back (batch-major); otherwise sequence n spans tokens
 * [cu_seqlens[n], cu_seqlens[n+1]).
 */
#define OR_CAT2(a, b) a##_##b
#define OR_CAT(a, b) OR_CAT2(a, b)
#define FN(name) OR_CAT(name, SFX)

#ifndef OR_CKPT
#define OR_CKPT 64
#endif

static void FN(q_coeff)(REAL lambda, REAL beta, REAL* c, REAL* dcl, REAL* dcb) {
    if (sizeof(REAL) == sizeof(double)) {
        double cc, dl, db;
        or_efla_coeff_f64((double)lambda, (double)beta, &cc, &dl, &db);
        *c = (REAL)cc;
        *dcl = (REAL)dl;
        *dcb = (REAL)db;
    } else {
        float cc, dl;
        or_efla_coeff_f32((float)lambda, (float)beta, &cc, &dl);
        *c = (REAL)cc;
        *dcl = (REAL)dl;
        *dcb = (REAL)expf(-(float)beta * (float)lambda);
    }
}

static void FN(q_bounds)(const int32_t* cu, int64_t n, int64_t T, int64_t* bos, int64_t* len) {
    if (cu) {
        *bos = cu[n];
        *len = (int64_t)cu[n + 1] - (int64_t)cu[n];
    } else {
        *bos = n * T;
        *len = T;
    }
}

/* One forward token on state S (K x V): returns c, writes r = v - u. */
static REAL FN(q_step)(REAL* S, const REAL* kt, const REAL* vt, REAL bt, REAL* r, int64_t K,
                       int64_t V, REAL* dcl, REAL* dcb) {
    REAL lam = 0;
    for (int64_t i = 0; i < K; ++i) lam += kt[i] * kt[i];
    REAL c, dl, db;
    FN(q_coeff)(lam, bt, &c, &dl, &db);
    for (int64_t j = 0; j < V; ++j) r[j] = vt[j];
    for (int64_t i = 0; i < K; ++i) {
        const REAL ki = kt[i];
        const REAL* Si = S + i * V;
        for (int64_t j = 0; j < V; ++j) r[j] -= ki * Si[j];
    }
    for (int64_t i = 0; i < K; ++i) {
        const REAL cki = c * kt[i];
        REAL* Si = S + i * V;
        for (int64_t j = 0; j < V; ++j) Si[j] += cki * r[j];
    }
    if (dcl) *dcl = dl;
    if (dcb) *dcb = db;
    return c;
}

void FN(or_efla_q_forward)(const REAL* q, const REAL* k, const REAL* v, const REAL* beta,
                           const int32_t* cu_seqlens, int64_t N, int64_t T, int64_t H,
                           int64_t K, int64_t V, const REAL* S0, REAL* O, REAL* ST) {
#pragma omp parallel for schedule(dynamic)
    for (int64_t nh = 0; nh < N * H; ++nh) {
        const int64_t n = nh / H, h = nh % H;
        int64_t bos, len;
        FN(q_bounds)(cu_seqlens, n, T, &bos, &len);
        REAL* S = (REAL*)malloc((size_t)(K * V + V) * sizeof(REAL));
        REAL* r = S + K * V;
        if (S0)
            memcpy(S, S0 + nh * K * V, (size_t)(K * V) * sizeof(REAL));
        else
            memset(S, 0, (size_t)(K * V) * sizeof(REAL));
        for (int64_t t = 0; t < len; ++t) {
            const int64_t tok = bos + t;
            const REAL* qt = q + (tok * H + h) * K;
            const REAL* kt = k + (tok * H + h) * K;
            const REAL* vt = v + (tok * H + h) * V;
            FN(q_step)(S, kt, vt, beta[tok * H + h], r, K, V, NULL, NULL);
            REAL* ot = O + (tok * H + h) * V;
            for (int64_t j = 0; j < V; ++j) ot[j] = 0;
            for (int64_t i = 0; i < K; ++i) {
                const REAL qi = qt[i];
                const REAL* Si = S + i * V;
                for (int64_t j = 0; j < V; ++j) ot[j] += qi * Si[j];
            }
        }
        if (ST) memcpy(ST + nh * K * V, S, (size_t)(K * V) * sizeof(REAL));
        free(S);
    }
}

void FN(or_efla_q_backward)(const REAL* q, const REAL* k, const REAL* v, const REAL* beta,
                            const REAL* dO, const int32_t* cu_seqlens, int64_t N, int64_t T,
                            int64_t H, int64_t K, int64_t V, const REAL* S0, const REAL* dST,
                            REAL* dq, REAL* dk, REAL* dv, REAL* dbeta, REAL* dS0) {
#pragma omp parallel for schedule(dynamic)
    for (int64_t nh = 0; nh < N * H; ++nh) {
        const int64_t n = nh / H, h = nh % H;
        int64_t bos, len;
        FN(q_bounds)(cu_seqlens, n, T, &bos, &len);
        const int64_t KV = K * V;
        const int64_t nck = (len + OR_CKPT - 1) / OR_CKPT;
        /* checkpoints: state before token j*OR_CKPT, plus a segment buffer of
         * the pre-update states of one segment */
        REAL* ck = (REAL*)malloc((size_t)((nck > 0 ? nck : 1) * KV) * sizeof(REAL));
        REAL* seg = (REAL*)malloc((size_t)((OR_CKPT + 1) * KV) * sizeof(REAL));
        REAL* G = (REAL*)malloc((size_t)KV * sizeof(REAL));
        REAL* vec = (REAL*)malloc((size_t)(3 * V + 2 * K) * sizeof(REAL));
        REAL *r = vec, *dr = vec + V, *gr = vec + 2 * V, *tmpk = vec + 3 * V, *gk = tmpk + K;
        REAL* S = seg;
        if (S0)
            memcpy(S, S0 + nh * KV, (size_t)KV * sizeof(REAL));
        else
            memset(S, 0, (size_t)KV * sizeof(REAL));
        for (int64_t t = 0; t < len; ++t) {
            if (t % OR_CKPT == 0) memcpy(ck + (t / OR_CKPT) * KV, S, (size_t)KV * sizeof(REAL));
            const int64_t tok = bos + t;
            FN(q_step)(S, k + (tok * H + h) * K, v + (tok * H + h) * V, beta[tok * H + h], r, K,
                       V, NULL, NULL);
        }
        if (dST)
            memcpy(G, dST + nh * KV, (size_t)KV * sizeof(REAL));
        else
            memset(G, 0, (size_t)KV * sizeof(REAL));
        for (int64_t j = nck - 1; j >= 0; --j) {
            const int64_t t0 = j * OR_CKPT;
            const int64_t t1 = (t0 + OR_CKPT < len) ? t0 + OR_CKPT : len;
            /* seg[i] = state before token t0+i, i = 0..t1-t0 */
            memcpy(seg, ck + j * KV, (size_t)KV * sizeof(REAL));
            for (int64_t t = t0; t < t1; ++t) {
                const int64_t tok = bos + t;
                REAL* nxt = seg + (t - t0 + 1) * KV;
                memcpy(nxt, seg + (t - t0) * KV, (size_t)KV * sizeof(REAL));
                FN(q_step)(nxt, k + (tok * H + h) * K, v + (tok * H + h) * V,
                           beta[tok * H + h], r, K, V, NULL, NULL);
            }
            for (int64_t t = t1 - 1; t >= t0; --t) {
                const int64_t tok = bos + t;
                const REAL* Sp = seg + (t - t0) * KV;
                const REAL* Sn = seg + (t - t0 + 1) * KV;
                const REAL* qt = q + (tok * H + h) * K;
                const REAL* kt = k + (tok * H + h) * K;
                const REAL* vt = v + (tok * H + h) * V;
                const REAL* dot = dO + (tok * H + h) * V;
                REAL lam = 0;
                for (int64_t i = 0; i < K; ++i) lam += kt[i] * kt[i];
                REAL c, dcl, dcb;
                FN(q_coeff)(lam, beta[tok * H + h], &c, &dcl, &dcb);
                /* r = v - Sp^T k */
                for (int64_t jj = 0; jj < V; ++jj) r[jj] = vt[jj];
                for (int64_t i = 0; i < K; ++i)
                    for (int64_t jj = 0; jj < V; ++jj) r[jj] -= kt[i] * Sp[i * V + jj];
                /* dq = Sn dO */
                REAL* dqt = dq + (tok * H + h) * K;
                for (int64_t i = 0; i < K; ++i) {
                    REAL s = 0;
                    for (int64_t jj = 0; jj < V; ++jj) s += Sn[i * V + jj] * dot[jj];
                    dqt[i] = s;
                }
                /* g = G + q dO^T (in place in G) */
                for (int64_t i = 0; i < K; ++i)
                    for (int64_t jj = 0; jj < V; ++jj) G[i * V + jj] += qt[i] * dot[jj];
                /* dr = c g^T k ; gr = g r */
                for (int64_t jj = 0; jj < V; ++jj) dr[jj] = 0;
                for (int64_t i = 0; i < K; ++i) {
                    REAL s = 0;
                    for (int64_t jj = 0; jj < V; ++jj) {
                        dr[jj] += G[i * V + jj] * kt[i];
                        s += G[i * V + jj] * r[jj];
                    }
                    tmpk[i] = s;
                }
                for (int64_t jj = 0; jj < V; ++jj) dr[jj] *= c;
                REAL dc = 0;
                for (int64_t i = 0; i < K; ++i) dc += kt[i] * tmpk[i];
                for (int64_t i = 0; i < K; ++i) {
                    REAL s = 0;
                    for (int64_t jj = 0; jj < V; ++jj) s += Sp[i * V + jj] * dr[jj];
                    gk[i] = c * tmpk[i] - s + (REAL)2 * dc * dcl * kt[i];
                }
                REAL* dkt = dk + (tok * H + h) * K;
                REAL* dvt = dv + (tok * H + h) * V;
                for (int64_t i = 0; i < K; ++i) dkt[i] = gk[i];
                for (int64_t jj = 0; jj < V; ++jj) dvt[jj] = dr[jj];
                dbeta[tok * H + h] = dc * dcb;
                /* G <- g - k dr^T */
                for (int64_t i = 0; i < K; ++i)
                    for (int64_t jj = 0; jj < V; ++jj) G[i * V + jj] -= kt[i] * dr[jj];
                (void)gr;
            }
        }
        if (dS0) memcpy(dS0 + nh * KV, G, (size_t)KV * sizeof(REAL));
        free(vec);
        free(G);
        free(seg);
        free(ck);
    }
}

#undef FN
#undef OR_CAT
#undef OR_CAT2
