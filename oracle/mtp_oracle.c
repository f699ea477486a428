/*
 * mtp_oracle.c -- CPU restatement of IMR-MLP's MTP E/F/S and training
 * loss-gradient path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP product.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * Build: gcc -O2 -std=c11 -ffp-contract=off -fopenmp (oracle/Makefile).
 * Floating-point contraction is off so that wrap, image translations and
 * displacements are reproducible bit for bit; the product compiles its
 * neighbour kernels the same way.
 *
 * Pinning (what each part is checked against, see tests/):
 *   loader ............ reference fixtures (unitest/test-data, .mtp files) and
 *                        the loader's documented defaults (scaling 0.01,
 *                        default radial/linear coefficients)
 *   wrap + neighbours .. oracle/_ref/nbh_ref (base/neighborhood.cpp compiled
 *                        from the reference sources), bit for bit, and a
 *                        brute-force periodic enumeration (set + count)
 *   RBChebyshev ........ closed form cos(k acos xi) and finite differences
 *   site E/F, getEFS ... oracle/_ref/mlip_ref (runtime/mtp/mlip.cpp
 *                        compiled from the reference sources), the
 *                        closed-form two-moment model of
 *                        unitest/ut_mtp_cuda.cpp:110-173, FD of E,
 *                        sum F = 0, strain FD of the virial, invariance
 *   gradient ........... coefficient finite differences of the loss
 *                        (unitest/ut_mtp_cpu_training.cpp:12-70 style)
 *   design rows/Gram ... E/F/S = rows . coefficients (linearity), and a
 *                        long-double textbook Gram
 */
#define _GNU_SOURCE
#include "mtp_oracle.h"

#include <ctype.h>
#include <float.h>
#include <limits.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static void set_err(char *err, int errlen, const char *msg)
{
    if (err && errlen > 0) {
        strncpy(err, msg, (size_t)errlen - 1);
        err[errlen - 1] = 0;
    }
}

/* ======================================================================
 * .mtp reader: restates PotMTP::Load (potentials/potential_mtp.cpp:119-571)
 * for the non-split RBChebyshev grammar, using istream >> semantics.
 * ====================================================================== */
typedef struct {
    const char *p;
    int fail;
} rd_t;

static void rd_skipws(rd_t *r)
{
    while (*r->p && isspace((unsigned char)*r->p))
        r->p++;
}
static int rd_word(rd_t *r, char *buf, int n)
{
    rd_skipws(r);
    int k = 0;
    while (*r->p && !isspace((unsigned char)*r->p)) {
        if (k < n - 1)
            buf[k++] = *r->p;
        r->p++;
    }
    buf[k] = 0;
    if (k == 0)
        r->fail = 1;
    return k;
}
static void rd_ignore(rd_t *r, int n)
{
    while (n-- > 0 && *r->p)
        r->p++;
}
static void rd_ignore_until(rd_t *r, int n, char delim)
{
    while (n-- > 0 && *r->p) {
        char c = *r->p++;
        if (c == delim)
            return;
    }
}
static double rd_double(rd_t *r)
{
    rd_skipws(r);
    char *end = NULL;
    double v = strtod(r->p, &end);
    if (end == r->p) {
        r->fail = 1;
        return 0;
    }
    r->p = end;
    return v;
}
static int rd_int(rd_t *r)
{
    rd_skipws(r);
    char *end = NULL;
    long v = strtol(r->p, &end, 10);
    if (end == r->p) {
        r->fail = 1;
        return 0;
    }
    r->p = end;
    return (int)v;
}
static char rd_char(rd_t *r)
{
    rd_skipws(r);
    if (!*r->p) {
        r->fail = 1;
        return 0;
    }
    return *r->p++;
}
static void rd_line(rd_t *r, char *buf, int n)
{
    int k = 0;
    while (*r->p && *r->p != '\n') {
        if (k < n - 1)
            buf[k++] = *r->p;
        r->p++;
    }
    if (*r->p == '\n')
        r->p++;
    if (k > 0 && buf[k - 1] == '\r')
        k--;
    buf[k] = 0;
}

void orc_model_free(orc_model *m)
{
    if (!m)
        return;
    free(m->basic);
    free(m->times);
    free(m->map);
    free(m->nu);
    free(m->coef);
    free(m->bases);
    free(m->tag);
    free(m);
}

/* basis_name_to_code (basis/basis.cpp:10-27), the four types restated here */
static int basis_code(const char *name)
{
    if (strcmp(name, "RBChebyshev") == 0)
        return 0;
    if (strcmp(name, "RBChebyCos") == 0)
        return 1;
    if (strcmp(name, "RBChebyshevPoly4") == 0)
        return 2;
    if (strcmp(name, "RBChebyshevPoly5") == 0)
        return 3;
    if (strcmp(name, "RBChebyshevConfigurable") == 0)
        return 4;
    return -1;
}
static const char *basis_name(int code)
{
    static const char *names[] = {"RBChebyshev", "RBChebyCos", "RBChebyshevPoly4",
                                  "RBChebyshevPoly5", "RBChebyshevConfigurable"};
    return names[code];
}

/* Cutoff::cutoff_type_name / XTransForm::shift_type_name (basis/cutoff.cpp,
 * basis/xtrans.cpp), in the order of their enums. */
static const char *cut_names[] = {"quadratic",    "normalized_quadratic", "cosine",
                                  "cosine_left",  "cosine_unscaled",      "cosine_squared",
                                  "sine_squared", "poly3",                "poly4",
                                  "poly5",        "smoothstep5",          "smoothstep7"};
static const char *shift_names[] = {"linear", "exponential", "exponential_left", "i2",
                                    "exponential_tanh"};
enum { CUT_QUAD, CUT_NQUAD, CUT_COS, CUT_COSL, CUT_COSU, CUT_COS2, CUT_SIN2, CUT_P3, CUT_P4,
       CUT_P5, CUT_SS5, CUT_SS7 };
enum { SH_LIN, SH_EXP, SH_EXPL, SH_I2, SH_EXPT };

/* "key = value" (cutoff.cpp / xtrans.cpp read_value, read_double) */
static int rd_keyval(rd_t *r, const char *key, char *val, int n)
{
    char tok[256];
    rd_word(r, tok, sizeof tok);
    if (strcmp(tok, key) != 0)
        return 0;
    rd_word(r, tok, sizeof tok);
    if (strcmp(tok, "=") != 0)
        return 0;
    return rd_word(r, val, n) > 0;
}
static int rd_keydouble(rd_t *r, const char *key, double *v)
{
    char val[256], *end = NULL;
    if (!rd_keyval(r, key, val, sizeof val))
        return 0;
    *v = strtod(val, &end);
    return end && *end == 0 && end != val && isfinite(*v);
}
static int find_name(const char **names, int n, const char *s)
{
    for (int i = 0; i < n; ++i)
        if (strcmp(names[i], s) == 0)
            return i;
    return -1;
}

/* RBasis_ChebyshevConfigurable::LoadFromStream (basis.cpp:893-911) after
 * the common lines: an optional basis_function_type, then
 * Cutoff::load_cutoff (cutoff.cpp:441-454) and XTransForm::load_shift
 * (xtrans.cpp:360-371), with the constructors' checks (setup :875-891,
 * FormulaCutoff :187-206, FormulaShift, ExponentialShift). */
static const char *load_configurable(rd_t *r, orc_basis *b)
{
    char val[256];
    b->one_minus = 0;
    rd_skipws(r);
    if (*r->p == 'b') {
        if (!rd_keyval(r, "basis_function_type", val, sizeof val))
            return "Error loading configurable radial basis: expected basis_function_type = <value>";
        if (strcmp(val, "one_minus_chebyshev") == 0)
            b->one_minus = 1;
        else if (strcmp(val, "chebyshev") != 0)
            return "Unknown configurable radial basis function type";
    }
    if (!rd_keyval(r, "cutoff_type", val, sizeof val))
        return "Error loading configurable radial basis: expected cutoff_type = <value>";
    b->cut = find_name(cut_names, 12, val);
    if (b->cut < 0)
        return "Unknown configurable radial cutoff type";
    b->cut_b = b->cut_r1 = b->cut_r2 = 0;
    if (b->cut == CUT_P3 || b->cut == CUT_P4 || b->cut == CUT_P5)
        if (!rd_keydouble(r, "cutoff_b", &b->cut_b))
            return "Error loading configurable radial basis: invalid cutoff_b";
    if (b->cut == CUT_SS7)
        if (!rd_keydouble(r, "cutoff_r1", &b->cut_r1) || !rd_keydouble(r, "cutoff_r2", &b->cut_r2))
            return "Error loading configurable radial basis: invalid cutoff_r1/cutoff_r2";
    if (!rd_keyval(r, "shift_type", val, sizeof val))
        return "Error loading configurable radial basis: expected shift_type = <value>";
    b->shift = find_name(shift_names, 5, val);
    if (b->shift < 0)
        return "Unknown configurable radial shift type";
    b->lambda = b->scale_lambda = 0;
    if (b->shift == SH_EXP || b->shift == SH_EXPL || b->shift == SH_EXPT)
        if (!rd_keydouble(r, "shift_lambda", &b->lambda))
            return "Error loading configurable radial basis: invalid shift_lambda";
    if (b->shift == SH_EXPT)
        if (!rd_keydouble(r, "shift_scale_lambda", &b->scale_lambda))
            return "Error loading configurable radial basis: invalid shift_scale_lambda";
    const double lo = b->rmin, hi = b->rmax;
    if (!isfinite(lo) || !isfinite(hi) || !(lo < hi))
        return "RBChebyshevConfigurable requires finite min_dist < max_dist";
    if (b->cut == CUT_COSL && hi == 0.0)
        return "cosine_left cutoff requires nonzero max_dist";
    if (b->cut == CUT_SS7 && !(lo < b->cut_r1 && b->cut_r1 <= b->cut_r2 && b->cut_r2 < hi))
        return "smoothstep7 cutoff requires min_dist < cutoff_r1 <= cutoff_r2 < max_dist";
    if (b->shift == SH_EXPL && hi == 0.0)
        return "exponential_left shift requires nonzero max_dist";
    if ((b->shift == SH_EXP || b->shift == SH_EXPL || b->shift == SH_EXPT) && b->lambda != 0.0) {
        const double den = expm1(b->lambda);
        if (!isfinite(den) || den == 0.0)
            return "shift_lambda produces a non-finite exponential normalization";
    }
    if (b->shift == SH_EXPT && b->scale_lambda != 0.0 && tanh(b->scale_lambda) == 0.0)
        return "shift_scale_lambda produces an invalid normalization";
    return 0;
}

/* AnyBasis::LoadFromStream (basis/basis.cpp:73-117) and, for Poly4/Poly5,
 * the rb_b line of their LoadFromStream (:543-558, :716-731).  0 on success,
 * else an error message. */
static const char *load_basis(rd_t *r, int code, double scaling, orc_basis *b)
{
    char tok[256];
    b->type = code;
    b->scaling = scaling;
    b->b = 0;
    rd_word(r, tok, sizeof tok);
    if (strcmp(tok, "min_dist") != 0)
        return "Error in loading basis: min_dist";
    rd_ignore(r, 2);
    b->rmin = rd_double(r);
    rd_word(r, tok, sizeof tok);
    if (strcmp(tok, "max_dist") != 0)
        return "Error in loading basis: max_dist";
    rd_ignore(r, 2);
    b->rmax = rd_double(r);
    return 0;
}
static const char *load_basis_tail(rd_t *r, orc_basis *b)
{
    char tok[256];
    if (b->type == 4)
        return load_configurable(r, b);
    if (b->type == 2 || b->type == 3) {
        rd_word(r, tok, sizeof tok);
        if (strcmp(tok, "rb_b") != 0)
            return "Error in loading basis: rb_b";
        rd_ignore(r, 2);
        b->b = rd_double(r);
        if (r->fail)
            return "Error in loading basis: rb_b";
    }
    return 0;
}

/* ---- MTP-M metadata (runtime/mtp/mlip.cpp:70-296 read_mtp_gpu_metadata,
 * tools/mtp_metadata.h:374-398 legacy_model_fields) ------------------------
 * The fields come from a structured potential_tag (model, q,
 * model_coeffs_count, nn.activation, nn.hidden_layers) and from
 * "mtp_<key> = value" lines (a leading '#' allowed) before any "#MVS_v1.1"
 * payload; a key given twice with different values is an error. */
typedef struct {
    char model[32], activation[32];
    long q, mcc, h1, h2;  /* -1: absent */
} mtpm_fields;

/* A JSON string or integer member of the tag text (the tag is this
 * library's own canonical JSON: "key":value with no spaces). */
static int json_str(const char *js, const char *key, char *out, int n)
{
    char pat[64];
    snprintf(pat, sizeof pat, "\"%s\":\"", key);
    const char *p = strstr(js, pat);
    if (!p)
        return 0;
    p += strlen(pat);
    int k = 0;
    while (*p && *p != '"' && k < n - 1)
        out[k++] = *p++;
    out[k] = 0;
    return 1;
}
static long json_int(const char *js, const char *key)
{
    char pat[64];
    snprintf(pat, sizeof pat, "\"%s\":", key);
    const char *p = strstr(js, pat);
    if (!p)
        return -1;
    return strtol(p + strlen(pat), NULL, 10);
}
static const char *set_field_l(long *f, long v)
{
    if (*f >= 0 && *f != v)
        return "conflicting MTP-M metadata";
    *f = v;
    return 0;
}
static const char *set_field_s(char *f, int n, const char *v)
{
    if (f[0] && strcmp(f, v) != 0)
        return "conflicting MTP-M metadata";
    snprintf(f, (size_t)n, "%s", v);
    return 0;
}
static const char *mtpm_read_fields(const char *text, const char *tag, mtpm_fields *F)
{
    memset(F, 0, sizeof *F);
    F->q = F->mcc = F->h1 = F->h2 = -1;
    const char *e;
    if (tag[0] == '{') {
        char v[32];
        if (json_str(tag, "model", v, sizeof v) && (e = set_field_s(F->model, 32, v)))
            return e;
        if ((e = set_field_l(&F->q, json_int(tag, "q"))))
            return e;
        F->mcc = json_int(tag, "model_coeffs_count");
        const char *nn = strstr(tag, "\"nn\":");
        if (nn) {
            if (json_str(nn, "activation", v, sizeof v))
                snprintf(F->activation, sizeof F->activation, "%s", v);
            const char *hl = strstr(nn, "\"hidden_layers\":[");
            if (hl) {
                char *end = NULL;
                F->h1 = strtol(hl + 17, &end, 10);
                F->h2 = (end && *end == ',') ? strtol(end + 1, NULL, 10) : 0;
            }
        }
    }
    if (strcmp(F->model, "mtp_m_nn2") == 0)
        snprintf(F->model, sizeof F->model, "mtp_m_n2");
    for (const char *line = text; line && *line;) {
        const char *eol = strchr(line, '\n');
        size_t len = eol ? (size_t)(eol - line) : strlen(line);
        char buf[256];
        if (len >= sizeof buf)
            len = sizeof buf - 1;
        memcpy(buf, line, len);
        buf[len] = 0;
        line = eol ? eol + 1 : NULL;
        char *s = buf;
        while (*s == ' ' || *s == '\t')
            ++s;
        if (strncmp(s, "#MVS_v1.1", 9) == 0)
            break;
        if (*s == '#')
            ++s;
        while (*s == ' ' || *s == '\t')
            ++s;
        if (strncmp(s, "mtp_", 4) != 0 || !strchr(s, '='))
            continue;
        char *eq = strchr(s, '=');
        char *ke = eq;
        while (ke > s && (ke[-1] == ' ' || ke[-1] == '\t'))
            --ke;
        *ke = 0;
        char *v = eq + 1;
        while (*v == ' ' || *v == '\t')
            ++v;
        char *ve = v + strlen(v);
        while (ve > v && (ve[-1] == ' ' || ve[-1] == '\t' || ve[-1] == '\r'))
            *--ve = 0;
        if (strcmp(s, "mtp_model") == 0) {
            const char *name = strcmp(v, "mtp_m_nn2") == 0 ? "mtp_m_n2"
                               : strcmp(v, "mtp") == 0     ? "linear"
                                                           : v;
            if ((e = set_field_s(F->model, 32, name)))
                return e;
        } else if (strcmp(s, "mtp_descriptor_count") == 0) {
            if ((e = set_field_l(&F->q, strtol(v, NULL, 10))))
                return e;
        } else if (strcmp(s, "mtp_model_coeffs_count") == 0) {
            if ((e = set_field_l(&F->mcc, strtol(v, NULL, 10))))
                return e;
        } else if (strcmp(s, "mtp_hidden1") == 0) {
            if ((e = set_field_l(&F->h1, strtol(v, NULL, 10))))
                return e;
        } else if (strcmp(s, "mtp_hidden2") == 0) {
            if ((e = set_field_l(&F->h2, strtol(v, NULL, 10))))
                return e;
        } else if (strcmp(s, "mtp_activation") == 0) {
            char up[32];
            int k = 0;
            for (; v[k] && k < 31; ++k)
                up[k] = (char)toupper((unsigned char)v[k]);
            up[k] = 0;
            if ((e = set_field_s(F->activation, 32, up)))
                return e;
        }
    }
    for (char *c = F->activation; *c; ++c)
        *c = (char)toupper((unsigned char)*c);
    return 0;
}

/* the head, its dimensions and coefficient count (mlip.cpp:226-296) */
static const char *mtpm_configure(orc_model *m, const mtpm_fields *F)
{
    static const char *names[] = {"linear", "mtp_m_li", "mtp_m_q2", "mtp_m_fs", "mtp_m_n1",
                                  "mtp_m_n2"};
    m->head = 0;
    m->P = 1;
    m->h1 = m->h2 = m->Mc = 0;
    m->act = 0;
    if (!F->model[0])
        return 0;
    int h = -1;
    for (int k = 0; k < 6; ++k)
        if (strcmp(F->model, names[k]) == 0)
            h = k;
    if (h < 0)
        return "unknown mtp_model";
    const long q = F->q < 0 ? 0 : F->q, mcc = F->mcc < 0 ? 0 : F->mcc;
    const long h1 = F->h1 < 0 ? 0 : F->h1, h2 = F->h2 < 0 ? 0 : F->h2;
    if (h != 4 && h != 5 && (h1 != 0 || h2 != 0))
        return "non-neural models require zero hidden dimensions";
    if (h == 4 && h2 != 0)
        return "NN1 requires zero hidden2";
    if (h == 0)
        return 0;
    m->head = h;
    if (h == 1) {
        m->P = q == 0 ? 1 : (int)q;
        if (m->P != 1 || mcc != 0)
            return "linear MTP-M requires one descriptor and no head coefficients";
    } else if (h == 2 || h == 3) {
        m->P = q == 0 ? 2 : (int)q;
        if (m->P != 2)
            return "analytic q2/fs models require descriptor_count 2";
        const long want = h == 2 ? 5 : 1;
        if (mcc != 0 && mcc != want)
            return "analytic model coefficient count does not match model type";
        m->Mc = (int)want;
    } else {
        if (q <= 0 || h1 <= 0)
            return "neural model requires positive descriptor_count and hidden1";
        if (h == 5 && h2 <= 0)
            return "NN2 model requires positive hidden2";
        m->P = (int)q;
        m->h1 = (int)h1;
        m->h2 = (int)h2;
        const long want = h == 4 ? h1 * (q + 2) : q * h1 + h1 + h1 * h2 + 2 * h2;
        if (mcc != 0 && mcc != want)
            return "neural model coefficient count does not match dimensions";
        m->Mc = (int)want;
        const char *a = F->activation;
        m->act = strcmp(a, "TANH") == 0      ? 0
                 : strcmp(a, "RELU") == 0    ? 1
                 : strcmp(a, "SIGMOID") == 0 ? 2
                 : strcmp(a, "LINEAR") == 0  ? 3
                                             : -1;
        if (m->act < 0)
            return "unknown mtp_activation";
        if (h == 5 && m->act == 3)
            return "NN2 does not support LINEAR activation";
    }
    return 0;
}

#define LOAD_FAIL(msg)                                                                     \
    do {                                                                                   \
        set_err(err, errlen, msg);                                                         \
        orc_model_free(m);                                                                 \
        return NULL;                                                                       \
    } while (0)

orc_model *orc_model_load_text(const char *text, char *err, int errlen)
{
    orc_model *m = (orc_model *)calloc(1, sizeof(orc_model));
    rd_t r = {text, 0};
    char line[1024], tok[256];

    rd_line(&r, line, sizeof line); /* :127-136 */
    if (strcmp(line, "MTP") != 0)
        LOAD_FAIL("Can only read MTP format potentials");
    rd_line(&r, line, sizeof line); /* :138-145 */
    if (strcmp(line, "version = 1.1.0") != 0)
        LOAD_FAIL("MTP file must have version \"1.1.0\"");

    rd_word(&r, tok, sizeof tok); /* :148-154 */
    if (strcmp(tok, "potential_name") == 0) {
        rd_ignore(&r, 2);
        rd_word(&r, tok, sizeof tok);
        rd_word(&r, tok, sizeof tok);
    }
    double scaling = 0.01; /* :155 -- the loader's default is 0.01 */
    if (strcmp(tok, "scaling") == 0) {
        rd_ignore(&r, 2);
        scaling = rd_double(&r);
        rd_word(&r, tok, sizeof tok);
    }
    if (strcmp(tok, "species_count") != 0)
        LOAD_FAIL("Error reading .mtp file, no species_count tag found");
    rd_ignore(&r, 2);
    m->Z = rd_int(&r);
    if (r.fail || m->Z <= 0)
        LOAD_FAIL("Error reading .mtp file, invalid species_count");

    rd_word(&r, tok, sizeof tok); /* :171-187 */
    m->tag = (char *)calloc(1, 1);
    if (strcmp(tok, "potential_tag") == 0) {
        const char *nl = strchr(r.p, '\n');
        size_t len = nl ? (size_t)(nl - r.p) : strlen(r.p);
        char *raw = (char *)malloc(len + 1);
        memcpy(raw, r.p, len);
        raw[len] = 0;
        r.p += len + (nl ? 1 : 0);
        char *eq = strchr(raw, '=');
        if (!eq) {
            free(raw);
            LOAD_FAIL("Invalid potential_tag assignment");
        }
        /* MTPMetadata::Tag::parse trims the text after '=' (tools/mtp_metadata.h:208-212) */
        char *b0 = eq + 1, *e0 = raw + len;
        while (*b0 && strchr(" \t\r\n", *b0))
            ++b0;
        while (e0 > b0 && strchr(" \t\r\n", e0[-1]))
            --e0;
        free(m->tag);
        m->tag = (char *)malloc((size_t)(e0 - b0) + 1);
        memcpy(m->tag, b0, (size_t)(e0 - b0));
        m->tag[e0 - b0] = 0;
        free(raw);
        if (m->tag[0] != '{' && strstr(m->tag, "imrmlp_meta_v"))
            LOAD_FAIL("imrmlp_meta_v1 potential tags are not supported");
        rd_word(&r, tok, sizeof tok);
    }
    m->split = 0;
    if (strcmp(tok, "radial_split") == 0 || strcmp(tok, "radial_basis_split") == 0) {
        rd_ignore(&r, 2); /* :190-204 */
        m->split = rd_int(&r) != 0;
        if (!m->split)
            rd_word(&r, tok, sizeof tok);
    }
    const char *berr = 0;
    if (m->split) { /* :206-265: one basis per ordered species pair */
        const int P = m->Z * m->Z;
        m->bases = (orc_basis *)calloc((size_t)P, sizeof(orc_basis));
        char *seen = (char *)calloc((size_t)P, 1);
        int rb_last = 0;
        m->cutoff = 0;
        for (int q = 0; q < P; ++q) {
            rd_word(&r, tok, sizeof tok);
            if (strcmp(tok, "pair") != 0) {
                free(seen);
                LOAD_FAIL("Error reading .mtp file, incorrect pair setting");
            }
            int ci = rd_int(&r), cj = rd_int(&r);
            if (r.fail || ci < 0 || ci >= m->Z || cj < 0 || cj >= m->Z) {
                free(seen);
                LOAD_FAIL("Error reading .mtp file, invalid radial basis pair");
            }
            if (seen[ci * m->Z + cj]) {
                free(seen);
                LOAD_FAIL("Error reading .mtp file, duplicate radial basis pair");
            }
            seen[ci * m->Z + cj] = 1;
            rd_word(&r, tok, sizeof tok);
            if (strcmp(tok, "radial_basis_type") != 0) {
                free(seen);
                LOAD_FAIL("Error reading .mtp file, incorrect pair setting");
            }
            rd_ignore(&r, 2);
            rd_word(&r, tok, sizeof tok);
            const int code = basis_code(tok);
            if (code < 0) {
                free(seen);
                LOAD_FAIL("unsupported radial basis type");
            }
            orc_basis *bb = &m->bases[ci * m->Z + cj];
            berr = load_basis(&r, code, scaling, bb);
            int size = 0;
            if (!berr) {
                rd_word(&r, tok, sizeof tok);
                if (strcmp(tok, "radial_basis_size") != 0)
                    berr = "Error in loading basis: radial_basis_size";
                rd_ignore(&r, 2);
                size = rd_int(&r);
                if (!berr && (r.fail || size <= 0))
                    berr = "Error in loading basis: radial_basis_size must be positive";
            }
            if (!berr)
                berr = load_basis_tail(&r, bb);
            if (berr) {
                free(seen);
                LOAD_FAIL(berr);
            }
            if (rb_last == 0)
                rb_last = size;
            else if (size != rb_last) {
                free(seen);
                LOAD_FAIL("Error reading .mtp file, split radial bases must have the same "
                          "radial_basis_size");
            }
            if (m->cutoff < bb->rmax)
                m->cutoff = bb->rmax;
        }
        free(seen);
        m->R = rb_last;
    } else {
        if (strcmp(tok, "radial_basis_type") != 0) /* :267-272 */
            LOAD_FAIL("Error reading .mtp file");
        rd_ignore(&r, 2);
        rd_word(&r, tok, sizeof tok);
        const int code = basis_code(tok);
        if (code < 0)
            LOAD_FAIL("unsupported radial basis type");
        m->bases = (orc_basis *)calloc(1, sizeof(orc_basis));
        berr = load_basis(&r, code, scaling, m->bases);
        if (berr)
            LOAD_FAIL(berr);
        rd_word(&r, tok, sizeof tok);
        if (strcmp(tok, "radial_basis_size") != 0)
            LOAD_FAIL("Error in loading basis: radial_basis_size");
        rd_ignore(&r, 2);
        m->R = rd_int(&r);
        if (r.fail || m->R <= 0)
            LOAD_FAIL("Error in loading basis: radial_basis_size must be positive");
        berr = load_basis_tail(&r, m->bases);
        if (berr)
            LOAD_FAIL(berr);
        m->cutoff = m->bases[0].rmax;
    }
    for (int q = 0; q < (m->split ? m->Z * m->Z : 1); ++q)
        if (m->bases[q].type == 4 && m->R > 62)
            LOAD_FAIL("this restatement takes radial_basis_size <= 62 for RBChebyshevConfigurable");
    m->rmin = m->bases[0].rmin;
    m->rmax = m->cutoff;
    m->scaling = scaling;

    rd_word(&r, tok, sizeof tok); /* :291-297 */
    if (strcmp(tok, "radial_funcs_count") != 0)
        LOAD_FAIL("Error reading .mtp file");
    rd_ignore(&r, 2);
    m->M = rd_int(&r);
    if (r.fail || m->M < 0)
        LOAD_FAIL("Error reading .mtp file, invalid radial basis dimensions");

    const int Z = m->Z, M = m->M, R = m->R;
    m->nradial = Z * Z * M * R;
    double *radial = (double *)calloc((size_t)(m->nradial > 0 ? m->nradial : 1), sizeof(double));
    rd_word(&r, tok, sizeof tok);
    if (strcmp(tok, "radial_coeffs") == 0) { /* :309-334 */
        for (int s1 = 0; s1 < Z; s1++)
            for (int s2 = 0; s2 < Z; s2++) {
                int ts1 = rd_int(&r);
                rd_char(&r);
                int ts2 = rd_int(&r);
                if (r.fail || ts1 < 0 || ts1 >= Z || ts2 < 0 || ts2 >= Z) {
                    free(radial);
                    LOAD_FAIL("Error reading .mtp file, invalid radial coefficient pair");
                }
                for (int i = 0; i < M; ++i) {
                    rd_char(&r);
                    for (int j = 0; j < R; ++j) {
                        double t = rd_double(&r);
                        rd_char(&r);
                        if (r.fail) {
                            free(radial);
                            LOAD_FAIL("Error reading .mtp file, missing radial coefficient");
                        }
                        radial[(ts1 * Z + ts2) * M * R + i * R + j] = t;
                    }
                }
            }
        rd_word(&r, tok, sizeof tok);
    } else { /* :335-351 -- default radial coefficients */
        for (int i = 0; i < Z * Z; ++i)
            for (int k = 0; k < M; ++k) {
                for (int l = 0; l < R; ++l)
                    radial[i * M * R + k * R + l] = 1e-5;
                radial[i * M * R + k * R + (k < R - 1 ? k : R - 1)] = 1e-3 + k;
            }
    }

    if (strcmp(tok, "alpha_moments_count") != 0) { /* :353-363 */
        free(radial);
        LOAD_FAIL("Error reading .mtp file, except: alpha_moments_count");
    }
    rd_ignore(&r, 2);
    m->K = rd_int(&r);
    rd_word(&r, tok, sizeof tok);
    if (r.fail || strcmp(tok, "alpha_index_basic_count") != 0) {
        free(radial);
        LOAD_FAIL("Error reading .mtp file");
    }
    rd_ignore(&r, 2);
    m->B = rd_int(&r);
    rd_word(&r, tok, sizeof tok);
    if (r.fail || strcmp(tok, "alpha_index_basic") != 0 || m->B < 0 || m->K < m->B) {
        free(radial);
        LOAD_FAIL("Error reading .mtp file");
    }
    rd_ignore(&r, 4);
    m->basic = (int *)calloc((size_t)(m->B > 0 ? m->B : 1) * 4, sizeof(int));
    m->nu = (int *)calloc((size_t)(m->B > 0 ? m->B : 1), sizeof(int));
    int radial_func_max = -1;
    for (int i = 0; i < m->B; ++i) { /* :385-399 */
        rd_ignore_until(&r, 1000, '{');
        for (int q = 0; q < 4; ++q) {
            m->basic[4 * i + q] = rd_int(&r);
            if (q < 3)
                rd_char(&r);
        }
        if (r.fail || m->basic[4 * i] < 0 || m->basic[4 * i + 1] < 0 ||
            m->basic[4 * i + 2] < 0 || m->basic[4 * i + 3] < 0) {
            free(radial);
            LOAD_FAIL("Error reading .mtp file");
        }
        m->nu[i] = m->basic[4 * i + 1] + m->basic[4 * i + 2] + m->basic[4 * i + 3];
        if (m->basic[4 * i] > radial_func_max)
            radial_func_max = m->basic[4 * i];
    }
    if (radial_func_max != M - 1) {
        free(radial);
        LOAD_FAIL("Wrong number of radial functions specified");
    }
    rd_ignore_until(&r, 1000, '\n');

    rd_word(&r, tok, sizeof tok); /* :406-430 */
    if (strcmp(tok, "alpha_index_times_count") != 0) {
        free(radial);
        LOAD_FAIL("Error reading .mtp file");
    }
    rd_ignore(&r, 2);
    m->T = rd_int(&r);
    rd_word(&r, tok, sizeof tok);
    if (r.fail || strcmp(tok, "alpha_index_times") != 0 || m->T < 0) {
        free(radial);
        LOAD_FAIL("Error reading .mtp file");
    }
    rd_ignore(&r, 4);
    m->times = (int *)calloc((size_t)(m->T > 0 ? m->T : 1) * 4, sizeof(int));
    for (int i = 0; i < m->T; ++i) {
        rd_ignore_until(&r, 1000, '{');
        for (int q = 0; q < 4; ++q) {
            m->times[4 * i + q] = rd_int(&r);
            if (q < 3)
                rd_char(&r);
        }
        const int *t = m->times + 4 * i;
        if (r.fail || t[0] < 0 || t[0] >= m->K || t[1] < 0 || t[1] >= m->K || t[3] < 0 ||
            t[3] >= m->K) {
            free(radial);
            LOAD_FAIL("Error reading .mtp file");
        }
    }
    rd_ignore_until(&r, 1000, '\n');

    rd_word(&r, tok, sizeof tok); /* :432-451 */
    if (strcmp(tok, "alpha_scalar_moments") != 0) {
        free(radial);
        LOAD_FAIL("Error reading .mtp file");
    }
    rd_ignore(&r, 2);
    m->S = rd_int(&r);
    rd_word(&r, tok, sizeof tok);
    if (r.fail || strcmp(tok, "alpha_moment_mapping") != 0 || m->S < 0) {
        free(radial);
        LOAD_FAIL("Error reading .mtp file");
    }
    rd_ignore(&r, 4);
    m->map = (int *)calloc((size_t)(m->S > 0 ? m->S : 1), sizeof(int));
    for (int i = 0; i < m->S; ++i) {
        m->map[i] = rd_int(&r);
        rd_char(&r);
        if (r.fail || m->map[i] < 0 || m->map[i] >= m->K) {
            free(radial);
            LOAD_FAIL("Error reading .mtp file");
        }
    }
    rd_ignore_until(&r, 1000, '\n');

    {
        mtpm_fields F;
        const char *herr = mtpm_read_fields(text, m->tag, &F);
        if (!herr)
            herr = mtpm_configure(m, &F);
        if (herr) {
            free(radial);
            LOAD_FAIL(herr);
        }
    }
    /* PotMTP_M::Load (potential_mtp_m.h:2018-2124): Z (P + 1) species
     * coefficients, P S moment coefficients, then the head's */
    const int nsp = m->head ? Z * (m->P + 1) : Z, nmom = m->P * m->S;
    m->ncoef = m->nradial + nsp + nmom + m->Mc;
    m->coef = (double *)calloc((size_t)m->ncoef, sizeof(double));
    memcpy(m->coef, radial, sizeof(double) * (size_t)m->nradial);
    free(radial);
    double *lin = m->coef + m->nradial;
    for (int i = 0; i < nsp + nmom + m->Mc; ++i) /* :471-474 -- default linear coefficients */
        lin[i] = 1e-3;
    tok[0] = 0;
    rd_word(&r, tok, sizeof tok);
    r.fail = 0;
    if (strcmp(tok, "species_coeffs") == 0) { /* :479-489 */
        rd_ignore(&r, 4);
        for (int i = 0; i < nsp; ++i) {
            lin[i] = rd_double(&r);
            rd_char(&r);
            if (r.fail)
                LOAD_FAIL("Error reading .mtp file, missing species coefficient");
        }
        rd_ignore_until(&r, 1000, '\n');
        tok[0] = 0;
        rd_word(&r, tok, sizeof tok);
        r.fail = 0;
    }
    if (strcmp(tok, "moment_coeffs") == 0) { /* :490-502 */
        rd_ignore(&r, 2);
        rd_ignore_until(&r, 10, '{');
        for (int i = 0; i < nmom; ++i) {
            lin[nsp + i] = rd_double(&r);
            rd_char(&r);
            if (r.fail)
                LOAD_FAIL("Error reading .mtp file, missing moment coefficient");
        }
        rd_ignore_until(&r, 1000, '\n');
        tok[0] = 0;
        rd_word(&r, tok, sizeof tok);
        r.fail = 0;
    }
    if (m->head) { /* potential_mtp_m.h:2112-2124; mlip.cpp:201-207 asks for the section */
        if (strcmp(tok, "model_coeffs") != 0)
            LOAD_FAIL("nonlinear mtp_model requires a model_coeffs section");
        rd_ignore(&r, 2);
        rd_ignore_until(&r, 10, '{');
        for (int i = 0; i < m->Mc; ++i) {
            lin[nsp + nmom + i] = rd_double(&r);
            rd_char(&r);
            if (r.fail)
                LOAD_FAIL("Error reading .mtp file, missing model coefficient");
        }
    } else if (!m->head && strcmp(tok, "model_coeffs") == 0) {
        LOAD_FAIL("model_coeffs is present but mtp_model metadata is missing");
    }

    /* PotMTP::init_basic, potential_mtp.cpp:576-604 */
    m->max_nu1 = 0;
    m->max_mu = -1;
    for (int i = 0; i < m->B; ++i) {
        if (m->nu[i] > m->max_nu1)
            m->max_nu1 = m->nu[i];
        if (m->basic[4 * i] > m->max_mu)
            m->max_mu = m->basic[4 * i];
    }
    m->max_nu1++;
    m->max_mu++;
    return m;
}

int orc_model_head(const orc_model *m, int *o)
{
    o[0] = m->head;
    o[1] = m->P;
    o[2] = m->h1;
    o[3] = m->h2;
    o[4] = m->act;
    o[5] = m->Mc;
    return m->head;
}

int orc_model_info(const orc_model *m, int *o)
{
    o[0] = m->Z;
    o[1] = m->M;
    o[2] = m->R;
    o[3] = m->K;
    o[4] = m->B;
    o[5] = m->T;
    o[6] = m->S;
    o[7] = m->max_nu1;
    o[8] = m->max_mu;
    o[9] = m->nradial;
    o[10] = m->ncoef;
    return 0;
}

void orc_model_get_coeffs(const orc_model *m, double *x)
{
    memcpy(x, m->coef, sizeof(double) * (size_t)m->ncoef);
}
void orc_model_set_coeffs(orc_model *m, const double *x)
{
    memcpy(m->coef, x, sizeof(double) * (size_t)m->ncoef);
}
void orc_model_tables(const orc_model *m, int *basic, int *times, int *map, double *rb3)
{
    if (basic)
        memcpy(basic, m->basic, sizeof(int) * 4 * (size_t)m->B);
    if (times)
        memcpy(times, m->times, sizeof(int) * 4 * (size_t)m->T);
    if (map)
        memcpy(map, m->map, sizeof(int) * (size_t)m->S);
    if (rb3) {
        rb3[0] = m->rmin;
        rb3[1] = m->rmax;
        rb3[2] = m->scaling;
    }
}

/* PotMTP::write_header / write_radial_info / write_radial_coeff / write_rules /
 * write_linear_coeff (potentials/potential_mtp.cpp:647-785), scientific
 * notation with max_digits10 (17) significant digits. */
/* picojson's serialize_str (tools/picojson.h:484-519): the escapes of a JSON
 * string as the reference's metadata writer emits them. */
static size_t json_escape(const char *in, char *out)
{
    size_t k = 0;
    out[k++] = '"';
    for (const unsigned char *c = (const unsigned char *)in; *c; ++c) {
        const char *rep = 0;
        switch (*c) {
        case '"': rep = "\\\""; break;
        case '\\': rep = "\\\\"; break;
        case '/': rep = "\\/"; break;
        case '\b': rep = "\\b"; break;
        case '\f': rep = "\\f"; break;
        case '\n': rep = "\\n"; break;
        case '\r': rep = "\\r"; break;
        case '\t': rep = "\\t"; break;
        default: break;
        }
        if (rep) {
            memcpy(out + k, rep, strlen(rep));
            k += strlen(rep);
        } else if (*c < 0x20 || *c == 0x7f) {
            k += (size_t)sprintf(out + k, "\\u%04x", *c & 0xff);
        } else {
            out[k++] = (char)*c;
        }
    }
    out[k++] = '"';
    out[k] = 0;
    return k;
}

/* PotMTP::Save (potentials/potential_mtp.cpp:1052-1061): write_header
 * (:656-671), write_radial_info (:673-690, AnyBasis::SaveToStream
 * basis/basis.h:50-56 and the rb_b line of Poly4/Poly5, basis.cpp:560-564,
 * :733-737), write_radial_coeff (:692-714), write_rules (:716-752),
 * write_linear_coeff (:754-785), on a stream set to std::scientific with
 * max_digits10 = 17 digits (printf "%.17e").  The potential_tag line is
 * MTPMetadata::Tag::output(model_metadata()) serialised
 * (tools/mtp_metadata.h:353-370): this restatement covers an absent tag and
 * a plain-text (legacy) tag, kept as "legacy_tag"; it returns -1 for a tag
 * in JSON form and for a potential with an MTP-M head. */
int orc_model_save_text(const orc_model *m, char *buf, int buflen)
{
    if (m->tag[0] == '{' || m->head)
        return -1;
    size_t cap = 1 << 16, len = 0;
    char *out = (char *)malloc(cap);
#define EMIT(...)                                                                          \
    do {                                                                                   \
        int need_ = snprintf(NULL, 0, __VA_ARGS__);                                        \
        while (len + (size_t)need_ + 1 > cap) {                                            \
            cap *= 2;                                                                      \
            out = (char *)realloc(out, cap);                                               \
        }                                                                                  \
        snprintf(out + len, cap - len, __VA_ARGS__);                                       \
        len += (size_t)need_;                                                              \
    } while (0)
    EMIT("MTP\nversion = 1.1.0\npotential_name = MTP1m\n");
    EMIT("scaling = %.17e\n", m->scaling);
    EMIT("species_count = %d\n", m->Z);
    if (m->tag[0]) {
        char *esc = (char *)malloc(6 * strlen(m->tag) + 3);
        json_escape(m->tag, esc);
        EMIT("potential_tag = {\"legacy_tag\":%s,\"model\":\"linear\",\"schema\":\"gpml.mtp.metadata\","
             "\"type\":\"MTP\",\"version\":1}\n", esc);
        free(esc);
    } else {
        EMIT("potential_tag = {\"model\":\"linear\",\"schema\":\"gpml.mtp.metadata\","
             "\"type\":\"MTP\",\"version\":1}\n");
    }
    if (m->split)
        EMIT("radial_basis_split = 1\n");
    const int nb = m->split ? m->Z * m->Z : 1;
    for (int q = 0; q < nb; ++q) {
        const orc_basis *bb = &m->bases[q];
        if (m->split)
            EMIT("pair %d %d\n", q / m->Z, q % m->Z);
        EMIT("radial_basis_type = %s\n", basis_name(bb->type));
        EMIT("\tmin_dist = %.17e\n\tmax_dist = %.17e\n\tradial_basis_size = %d\n", bb->rmin,
             bb->rmax, m->R);
        if (bb->type == 2 || bb->type == 3)
            EMIT("\trb_b = %.17e\n", bb->b);
        if (bb->type == 4) {  /* RBasis_ChebyshevConfigurable::SaveToStream (basis.cpp:913-919) */
            EMIT("\tbasis_function_type = %s\n", bb->one_minus ? "one_minus_chebyshev" : "chebyshev");
            EMIT("\tcutoff_type = %s\n", cut_names[bb->cut]);
            if (bb->cut == CUT_P3 || bb->cut == CUT_P4 || bb->cut == CUT_P5)
                EMIT("\tcutoff_b = %.17e\n", bb->cut_b);
            if (bb->cut == CUT_SS7)
                EMIT("\tcutoff_r1 = %.17e\n\tcutoff_r2 = %.17e\n", bb->cut_r1, bb->cut_r2);
            EMIT("\tshift_type = %s\n", shift_names[bb->shift]);
            if (bb->shift == SH_EXP || bb->shift == SH_EXPL || bb->shift == SH_EXPT)
                EMIT("\tshift_lambda = %.17e\n", bb->lambda);
            if (bb->shift == SH_EXPT)
                EMIT("\tshift_scale_lambda = %.17e\n", bb->scale_lambda);
        }
    }
    EMIT("radial_funcs_count = %d\n", m->M);
    EMIT("radial_coeffs\n");
    int q = 0;
    for (int i = 0; i < m->Z; ++i)
        for (int j = 0; j < m->Z; ++j) {
            EMIT("\t%d-%d\n", i, j);
            for (int k = 0; k < m->M; ++k) {
                EMIT("\t\t{");
                for (int l = 0; l < m->R; ++l, ++q)  /* EMIT evaluates its arguments twice */
                    EMIT("%.17e%s", m->coef[q], l != m->R - 1 ? ", " : "}\n");
            }
        }
    EMIT("alpha_moments_count = %d\n", m->K);
    EMIT("alpha_index_basic_count = %d\n", m->B);
    EMIT("alpha_index_basic = {");
    for (int i = 0; i < m->B; ++i)
        EMIT("{%d, %d, %d, %d}%s", m->basic[4 * i], m->basic[4 * i + 1], m->basic[4 * i + 2],
             m->basic[4 * i + 3], i < m->B - 1 ? ", " : "");
    EMIT("}\n");
    EMIT("alpha_index_times_count = %d\n", m->T);
    EMIT("alpha_index_times = {");
    for (int i = 0; i < m->T; ++i)
        EMIT("{%d, %d, %d, %d}%s", m->times[4 * i], m->times[4 * i + 1], m->times[4 * i + 2],
             m->times[4 * i + 3], i < m->T - 1 ? ", " : "");
    EMIT("}\n");
    EMIT("alpha_scalar_moments = %d\n", m->S);
    EMIT("alpha_moment_mapping = {");
    for (int i = 0; i < m->S; ++i)
        EMIT("%s%d", i ? ", " : "", m->map[i]);
    EMIT("}\n");
    EMIT("species_coeffs = {");
    for (int i = 0; i < m->Z; ++i)
        EMIT("%s%.17e", i ? ", " : "", m->coef[m->nradial + i]);
    EMIT("}\n");
    EMIT("moment_coeffs = {");
    for (int i = 0; i < m->S; ++i)
        EMIT("%s%.17e", i ? ", " : "", m->coef[m->nradial + m->Z + i]);
    EMIT("}\n");
#undef EMIT
    int ret = (int)len;
    if (buf && (size_t)buflen > len) {
        memcpy(buf, out, len + 1);
    }
    free(out);
    return ret;
}

/* PotMTP::Orthogonalize (potentials/potential_mtp.cpp:3849-3930).  The
 * projection divides by the squared norm of c_k (the vector being projected),
 * not of c_k2, and the final norm adds 1e-10 per term; both kept. */
void orc_orthogonalize(orc_model *m)
{
    const int Z = m->Z, M = m->M, R = m->R;
    double *c = m->coef;
    for (int k = 0; k < M; ++k) {
        for (int k2 = 0; k2 < k; ++k2) {
            double norm = 0;
            for (int i = 0; i < Z; ++i)
                for (int j = 0; j < Z; ++j)
                    for (int l = 0; l < R; ++l) {
                        int idx = (i * Z + j) * M * R + k * R + l;
                        norm += c[idx] * c[idx];
                    }
            double scal = 0;
            for (int i = 0; i < Z; ++i)
                for (int j = 0; j < Z; ++j)
                    for (int l = 0; l < R; ++l) {
                        int i1 = (i * Z + j) * M * R + k * R + l;
                        int i2 = (i * Z + j) * M * R + k2 * R + l;
                        scal += c[i1] * c[i2];
                    }
            for (int i = 0; i < Z; ++i)
                for (int j = 0; j < Z; ++j)
                    for (int l = 0; l < R; ++l) {
                        int i1 = (i * Z + j) * M * R + k * R + l;
                        int i2 = (i * Z + j) * M * R + k2 * R + l;
                        c[i1] -= c[i2] * scal / norm;
                    }
        }
        double norm = 0;
        for (int i = 0; i < Z; i++)
            for (int j = 0; j < Z; j++)
                for (int l = 0; l < R; l++) {
                    int idx = (i * Z + j) * M * R + k * R + l;
                    norm += c[idx] * c[idx] + 1e-10;
                }
        norm = sqrt(norm);
        for (int i = 0; i < Z; i++)
            for (int j = 0; j < Z; j++)
                for (int l = 0; l < R; l++)
                    c[(i * Z + j) * M * R + k * R + l] /= norm;
    }
}

/* ======================================================================
 * Radial bases, calc_der of basis/basis.cpp: RBasis_Chebyshev (:119-164,
 * setup :119-125), RBasis_ChebyCos (:242-271, setup :228-235),
 * RBasis_ChebyshevPoly4 (:585-619, setup :533-540) and
 * RBasis_ChebyshevPoly5 (:776-805, setup :706-713).
 * ====================================================================== */
/* ksi = (2 r - (min + max)) / (max - min), the Chebyshev argument of all four */
static double ksi_of(const orc_basis *bs, double value)
{
    return (2 * value - (bs->rmax + bs->rmin)) / (bs->rmax - bs->rmin);
}

/* Value and first derivative (the first two members of the reference's
 * Jet2; the second derivative is not needed here). */
typedef struct {
    double v, d;
} jet;
static jet jc(double c) { jet r = {c, 0}; return r; }
static jet jadd(jet a, jet b) { jet r = {a.v + b.v, a.d + b.d}; return r; }
static jet jsub(jet a, jet b) { jet r = {a.v - b.v, a.d - b.d}; return r; }
static jet jmul(jet a, jet b) { jet r = {a.v * b.v, a.d * b.v + a.v * b.d}; return r; }
static jet jscale(double s, jet a) { jet r = {s * a.v, s * a.d}; return r; }
static jet jsin(jet a) { jet r = {sin(a.v), cos(a.v) * a.d}; return r; }
static jet jcos(jet a) { jet r = {cos(a.v), -sin(a.v) * a.d}; return r; }
static jet jexp(jet a) { double e = exp(a.v); jet r = {e, e * a.d}; return r; }
static jet jtanh(jet a) { double t = tanh(a.v); jet r = {t, (1.0 - t * t) * a.d}; return r; }
static jet jpow2(jet a) { return jmul(a, a); }
static jet jpow3(jet a) { return jmul(jmul(a, a), a); }
static jet jpow4(jet a) { return jpow2(jpow2(a)); }
static jet jpow5(jet a) { return jmul(jpow4(a), a); }
static jet jpow6(jet a) { return jmul(jpow3(a), jpow3(a)); }
static jet jpow7(jet a) { return jmul(jpow6(a), a); }

/* Cutoff value and derivative: QuadraticCutoff, CosineCutoff, Poly5Cutoff
 * (cutoff.cpp:325-421) and FormulaCutoff::evaluate (:147-185). */
static void cutoff_der(const orc_basis *b, double r, double *fc, double *dfc)
{
    const double lo = b->rmin, hi = b->rmax, inv = 1.0 / (hi - lo), pi = M_PI;
    if (b->cut == CUT_QUAD) {
        const double delta = r - hi;
        *fc = delta * delta;
        *dfc = 2.0 * delta;
        return;
    }
    if (b->cut == CUT_COS) {
        const double freq = pi / (hi - lo), phase = (r - lo) * freq;
        *fc = 0.5 * (1.0 + cos(phase));
        *dfc = -0.5 * freq * sin(phase);
        return;
    }
    if (b->cut == CUT_P5) {
        const double x = (r - lo) * inv, omx = 1.0 - x, sq = omx * omx, cube = sq * omx;
        *fc = sq * sq * (1.0 + (4.0 + b->cut_b) * x);
        *dfc = -cube * (20.0 * x + b->cut_b * (5.0 * x - 1.0)) * inv;
        return;
    }
    const jet radius = {r, 1.0}, one = jc(1.0);
    const jet t = jmul(jsub(radius, jc(lo)), jc(inv));
    const jet q = jsub(one, t);
    jet res = one;
    switch (b->cut) {
    case CUT_NQUAD: res = jpow2(q); break;
    case CUT_COSL: res = jscale(0.5, jadd(one, jcos(jscale(pi / hi, radius)))); break;
    case CUT_COSU: res = jadd(one, jcos(jscale(pi, t))); break;
    case CUT_COS2: res = jpow2(jadd(one, jcos(jscale(pi, t)))); break;
    case CUT_SIN2: res = jpow2(jsin(jscale(pi, t))); break;
    case CUT_P3: res = jmul(jpow2(q), jadd(one, jscale(b->cut_b + 2.0, t))); break;
    case CUT_P4: res = jmul(jpow3(q), jadd(one, jscale(b->cut_b + 3.0, t))); break;
    case CUT_SS5:
        res = jadd(jsub(jscale(6.0, jpow5(q)), jscale(15.0, jpow4(q))), jscale(10.0, jpow3(q)));
        break;
    case CUT_SS7:
        if (r <= b->cut_r1) {
            const jet p = jscale(1.0 / (b->cut_r1 - lo), jsub(radius, jc(lo)));
            res = jsub(jadd(jsub(jscale(35.0, jpow4(p)), jscale(84.0, jpow5(p))),
                            jscale(70.0, jpow6(p))),
                       jscale(20.0, jpow7(p)));
        } else if (r >= b->cut_r2) {
            const jet p = jscale(1.0 / (hi - b->cut_r2), jsub(radius, jc(b->cut_r2)));
            res = jadd(jsub(jadd(jsub(one, jscale(35.0, jpow4(p))), jscale(84.0, jpow5(p))),
                            jscale(70.0, jpow6(p))),
                       jscale(20.0, jpow7(p)));
        }
        break;
    }
    *fc = res.v;
    *dfc = res.d;
}

/* Shift value and derivative: LinearShift, ExponentialShift
 * (xtrans.cpp:240-330) and FormulaShift::evaluate (:104-141). */
static void shift_der(const orc_basis *b, double r, double *x, double *dx)
{
    const double lo = b->rmin, hi = b->rmax, inv = 1.0 / (hi - lo), lam = b->lambda;
    if (b->shift == SH_LIN) {
        const double slope = 2.0 / (hi - lo);
        *x = -1.0 + slope * (r - lo);
        *dx = slope;
        return;
    }
    if (b->shift == SH_EXP) {
        if (lam == 0.0) {
            *x = -1.0 + 2.0 * (r - lo) * inv;
            *dx = 2.0 * inv;
            return;
        }
        const double den = expm1(lam), e = lam * (hi - r) * inv;
        *x = 1.0 - 2.0 * expm1(e) / den;
        *dx = 2.0 * lam * inv * exp(e) / den;
        return;
    }
    const jet radius = {r, 1.0}, one = jc(1.0);
    const jet t = jmul(jsub(radius, jc(lo)), jc(inv));
    jet res = one;
    if (b->shift == SH_I2) {
        const jet k = jmul(jsub(radius, jc(hi)), jc(inv));
        res = jsub(jscale(2.0, jmul(k, k)), one);
    } else if (b->shift == SH_EXPL) {
        if (lam == 0.0) {
            res = jsub(jscale(2.0, jscale(1.0 / hi, radius)), one);
        } else {
            const double den = expm1(lam);
            const jet ex = jscale(lam, jsub(one, jscale(1.0 / hi, radius)));
            res = jsub(one, jscale(2.0 / den, jsub(jexp(ex), one)));
        }
    } else {  /* exponential_tanh */
        jet sh;
        if (lam == 0.0) {
            sh = jsub(jscale(2.0, t), one);
        } else {
            const double den = expm1(lam);
            sh = jsub(one, jscale(2.0 / den, jsub(jexp(jscale(lam, jsub(one, t))), one)));
        }
        res = b->scale_lambda == 0.0 ? sh
                                     : jscale(1.0 / tanh(b->scale_lambda),
                                              jtanh(jscale(b->scale_lambda, sh)));
    }
    *x = res.v;
    *dx = res.d;
}

/* RBasis_ChebyshevConfigurable::calculate (basis.cpp:931-1011): zero
 * outside [min, max]; otherwise the Chebyshev polynomials T_i of the shift
 * x(r) (or 1 - T_{i+1} for one_minus_chebyshev) times the cutoff, scaled. */
static void configurable_der(const orc_basis *b, int R, double value, double *val, double *der)
{
    if (value < b->rmin || value > b->rmax) {
        for (int i = 0; i < R; ++i)
            val[i] = der[i] = 0;
        return;
    }
    double x, dx, fc, dfc;
    shift_der(b, value, &x, &dx);
    cutoff_der(b, value, &fc, &dfc);
    const int np = R + (b->one_minus ? 1 : 0);
    double T[64], dT[64];
    T[0] = 1.0;
    dT[0] = 0.0;
    if (np > 1) {
        T[1] = x;
        dT[1] = dx;
    }
    for (int i = 2; i < np; ++i) {
        T[i] = 2.0 * x * T[i - 1] - T[i - 2];
        dT[i] = 2.0 * (dx * T[i - 1] + x * dT[i - 1]) - dT[i - 2];
    }
    for (int i = 0; i < R; ++i) {
        const int k = i + (b->one_minus ? 1 : 0);
        const double raw = b->one_minus ? 1.0 - T[k] : T[k];
        const double rawd = b->one_minus ? -dT[k] : dT[k];
        val[i] = b->scaling * raw * fc;
        der[i] = b->scaling * (rawd * fc + raw * dfc);
    }
}

static void basis_calc_der(const orc_basis *bs, int R, double value, double *val, double *der)
{
    if (bs->type == 4) {
        configurable_der(bs, R, value, val, der);
        return;
    }
    const double min_val = bs->rmin, max_val = bs->rmax, scaling = bs->scaling;
    const double mult = 2.0 / (max_val - min_val);
    const double su = max_val - min_val;
    const double pu = max_val + min_val;
    if (bs->type == 0) {
        double ksi = (2 * value - pu) / su;
        double ru = value - max_val;
        val[0] = scaling * (1 * ru * ru);
        der[0] = scaling * (0 * ru * ru + 2 * ru);
        if (R == 1)
            return;
        val[1] = scaling * (ksi * ru * ru);
        der[1] = scaling * (mult * ru * ru + 2 * ksi * ru);
    } else if (bs->type == 1) {
        const double irpi = M_PI / max_val;
        double ksi = (2 * value - pu) / su;
        double rc = 0.5 * (1.0 + cos(value * irpi));
        double drc = -0.5 * irpi * sin(value * irpi);
        val[0] = scaling * (1 * rc);
        der[0] = scaling * (0 * rc + drc);
        if (R == 1)
            return;
        val[1] = scaling * (ksi * rc);
        der[1] = scaling * (mult * rc + ksi * drc);
    } else {
        if (value < min_val || value > max_val) {
            for (int i = 0; i < R; i++)
                val[i] = der[i] = 0;
            return;
        }
        const double dxdr = 1.0 / su;
        double ksi = (2 * value - pu) / su;
        double x = (value - min_val) / su;
        double vx = 1.0 - x;
        double vxx = vx * vx;
        double vxxx = vxx * vx;
        double rc, drc;
        if (bs->type == 2) {
            rc = vxxx * (1 + (3 + bs->b) * x);
            drc = vxx * (bs->b * (1. - 4.0 * x) - 12.0 * x) * dxdr;
        } else {
            double vxxxx = vxx * vxx;
            rc = vxxxx * (1 + (4 + bs->b) * x);
            drc = -vxxx * (20 * x + bs->b * (5 * x - 1)) * dxdr;
        }
        val[0] = scaling * rc;
        der[0] = scaling * drc;
        if (R == 1)
            return;
        val[1] = scaling * (ksi * rc);
        der[1] = scaling * (mult * rc + ksi * drc);
    }
    for (int i = 2; i < R; i++) {
        val[i] = 2 * ksi_of(bs, value) * val[i - 1] - val[i - 2];
        der[i] = 2 * (mult * val[i - 1] + ksi_of(bs, value) * der[i - 1]) - der[i - 2];
    }
}

/* the shared basis, or the pair's own (PotMTP::rb_calcder(itype, jtype, r)) */
static const orc_basis *pair_basis(const orc_model *m, int ti, int tj)
{
    return m->split ? &m->bases[ti * m->Z + tj] : &m->bases[0];
}
/* cutoffs(itype, jtype) of the site loop (potential_mtp.cpp:2842) */
static double pair_cutoff(const orc_model *m, int ti, int tj)
{
    return pair_basis(m, ti, tj)->rmax;
}

void orc_rb_calc_der(const orc_model *m, double value, double *val, double *der)
{
    basis_calc_der(&m->bases[0], m->R, value, val, der);
}

void orc_rb_calc_der_pair(const orc_model *m, int ti, int tj, double value, double *val,
                          double *der)
{
    basis_calc_der(pair_basis(m, ti, tj), m->R, value, val, der);
}

/* ======================================================================
 * Atoms::wrap (base/structures.cpp:1282-1305) and the BOXED neighbour
 * builder (base/neighborhoods_base.h:31-266, base/neighborhood.cpp:77-146).
 *
 * Cell rows are lattice vectors.  Small fixed-size Eigen products are
 * restated with the evaluation order of the Eigen 5.0.1-dev snapshot the
 * reference vendors (SSE2 baseline, no contraction):
 *   RowVector3d * Matrix3d : ((p0*m0j + p1*m1j) + p2*m2j)         all j
 *   Matrix3d * Vector3d    : rows 0,1 ((b0 + b1) + b2), row 2 (b0 + (b1 + b2))
 *   Matrix3d::inverse      : cofactor expansion, det = (c00 m00 + c10 m10) + c20 m20
 * ====================================================================== */
static void rowvec_mat(const double p[3], const double *M, double out[3])
{
    for (int j = 0; j < 3; ++j) {
        double a0 = p[0] * M[0 * 3 + j], a1 = p[1] * M[1 * 3 + j], a2 = p[2] * M[2 * 3 + j];
        out[j] = (a0 + a1) + a2;
    }
}

static double cof3(const double *m, int i, int j)
{
    int i1 = (i + 1) % 3, i2 = (i + 2) % 3, j1 = (j + 1) % 3, j2 = (j + 2) % 3;
    return m[i1 * 3 + j1] * m[i2 * 3 + j2] - m[i1 * 3 + j2] * m[i2 * 3 + j1];
}

void orc_cell_inverse(const double *m, double *inv)
{
    double c0 = cof3(m, 0, 0), c1 = cof3(m, 1, 0), c2 = cof3(m, 2, 0);
    double det = (c0 * m[0] + c1 * m[3]) + c2 * m[6];
    double invdet = 1.0 / det;
    for (int i = 0; i < 3; ++i)
        for (int j = 0; j < 3; ++j)
            inv[j * 3 + i] = cof3(m, i, j) * invdet;
}

void orc_wrap(const double *cell, const int *pbc, int n, double *pos)
{
    if (!pbc[0] && !pbc[1] && !pbc[2])
        return;
    double inv[9];
    orc_cell_inverse(cell, inv);
    for (int i = 0; i < n; ++i) {
        double f[3];
        rowvec_mat(pos + 3 * i, inv, f);
        for (int j = 0; j < 3; ++j)
            if (pbc[j])
                f[j] -= floor(f[j]);
        rowvec_mat(f, cell, pos + 3 * i);
    }
}

void orc_nbh_free(orc_nbh *h)
{
    if (!h)
        return;
    free(h->offsets);
    free(h->idx);
    free(h->types);
    free(h->vec);
    free(h->dist);
    free(h->pt);
    free(h->center_types);
    free(h->pts);
    free(h->orig);
    free(h);
}

typedef struct {
    int *start; /* [nbox+1] */
    int *items; /* [npts] */
} boxes_t;

/* Invert a small symmetric positive-definite matrix (dims <= 3). */
static int small_inverse(int d, const double *a, double *inv)
{
    if (d == 1) {
        inv[0] = 1.0 / a[0];
        return 1;
    }
    if (d == 2) {
        double det = a[0] * a[3] - a[1] * a[2];
        if (det == 0)
            return 0;
        inv[0] = a[3] / det;
        inv[1] = -a[1] / det;
        inv[2] = -a[2] / det;
        inv[3] = a[0] / det;
        return 1;
    }
    double c0 = cof3(a, 0, 0), c1 = cof3(a, 1, 0), c2 = cof3(a, 2, 0);
    double det = c0 * a[0] + c1 * a[3] + c2 * a[6];
    if (det == 0)
        return 0;
    for (int i = 0; i < 3; ++i)
        for (int j = 0; j < 3; ++j)
            inv[j * 3 + i] = cof3(a, i, j) / det;
    return 1;
}

orc_nbh *orc_build_neighbors(const double *cell, const int *pbc, int n, const double *pos_in,
                             const int *types, double cutoff, char *err, int errlen)
{
    orc_nbh *h = (orc_nbh *)calloc(1, sizeof(orc_nbh));
    h->n = n;
    h->offsets = (int *)calloc((size_t)n + 1, sizeof(int));
    h->center_types = (int *)calloc((size_t)(n > 0 ? n : 1), sizeof(int));
    if (n == 0) /* init_single, neighborhoods_base.h:254-266 */
        return h;

    /* load_positions (neighborhoods_base.h:113-127): re-wrap only if fully periodic */
    int cap = n * 2 + 64, npts = n;
    double *pts = (double *)malloc(sizeof(double) * 3 * (size_t)cap);
    int *orig = (int *)malloc(sizeof(int) * (size_t)cap);
    memcpy(pts, pos_in, sizeof(double) * 3 * (size_t)n);
    for (int i = 0; i < n; ++i)
        orig[i] = i;
    const int fully = pbc[0] && pbc[1] && pbc[2];
    const int nonper = !pbc[0] && !pbc[1] && !pbc[2];
    if (fully) {
        double inv[9];
        orc_cell_inverse(cell, inv);
        for (int i = 0; i < n; ++i) {
            double f[3];
            rowvec_mat(pts + 3 * i, inv, f);
            for (int d = 0; d < 3; ++d)
                f[d] -= floor(f[d]);
            rowvec_mat(f, cell, pts + 3 * i);
        }
    }

    /* BOXED extent_impl (neighborhoods_base.h:130-143) */
    double lo[3], hi[3];
    for (int d = 0; d < 3; ++d)
        lo[d] = hi[d] = pts[d];
    for (int i = 0; i < n; ++i)
        for (int d = 0; d < 3; ++d) {
            double v = pts[3 * i + d];
            /* cwiseMin/cwiseMax */
            lo[d] = v < lo[d] ? v : lo[d];
            hi[d] = v > hi[d] ? v : hi[d];
        }
    for (int d = 0; d < 3; ++d)
        if (hi[d] - lo[d] < cutoff)
            hi[d] = lo[d] + cutoff;

    /* append_images (neighborhoods_base.h:31-99).  The periodic axes are
     * sorted by squared lattice-vector length (stable for ties, as
     * libstdc++'s insertion sort is for three elements); the outermost loop
     * runs over the longest axis.  The reference bounds each integer range
     * with a Householder QR back-substitution; any superset of that range,
     * walked in the same lexicographic order, appends the same images,
     * because the AABB test below decides membership.  The superset used
     * here comes from the pseudo-inverse of the periodic basis. */
    if (!nonper) {
        int axes[3] = {0, 1, 2};
        double nrm[3];
        for (int a = 0; a < 3; ++a)
            nrm[a] = cell[3 * a] * cell[3 * a] + cell[3 * a + 1] * cell[3 * a + 1] +
                     cell[3 * a + 2] * cell[3 * a + 2];
        for (int a = 1; a < 3; ++a) { /* insertion sort, stable */
            int v = axes[a], b = a - 1;
            while (b >= 0 && nrm[v] < nrm[axes[b]]) {
                axes[b + 1] = axes[b];
                b--;
            }
            axes[b + 1] = v;
        }
        double basis[9] = {0};
        int dims = 0;
        for (int q = 0; q < 3; ++q)
            if (pbc[axes[q]]) {
                for (int r = 0; r < 3; ++r)
                    basis[r * 3 + dims] = cell[axes[q] * 3 + r];
                dims++;
            }
        double ext[3];
        for (int d = 0; d < 3; ++d)
            ext[d] = hi[d] - lo[d] + cutoff;
        /* pinv = (B^T B)^-1 B^T, B = basis[:, :dims] */
        double btb[9] = {0}, btbi[9] = {0};
        for (int a = 0; a < dims; ++a)
            for (int b = 0; b < dims; ++b) {
                double s = 0;
                for (int r = 0; r < 3; ++r)
                    s += basis[r * 3 + a] * basis[r * 3 + b];
                btb[a * dims + b] = s;
            }
        if (!small_inverse(dims, btb, btbi)) {
            set_err(err, errlen, "singular periodic cell");
            free(pts);
            free(orig);
            orc_nbh_free(h);
            return NULL;
        }
        long rng[3] = {0, 0, 0};
        for (int k = 0; k < dims; ++k) {
            double bnd = 0;
            for (int r = 0; r < 3; ++r) {
                double pk = 0;
                for (int a = 0; a < dims; ++a)
                    pk += btbi[k * dims + a] * basis[r * 3 + a];
                bnd += fabs(pk) * ext[r];
            }
            if (!(bnd < 1e8)) {
                set_err(err, errlen, "Neighbor periodic image index exceeds integer range");
                free(pts);
                free(orig);
                orc_nbh_free(h);
                return NULL;
            }
            rng[k] = (long)ceil(bnd) + 1;
        }
        long img[3] = {0, 0, 0};
        long lo2 = dims > 2 ? -rng[2] : 0, hi2 = dims > 2 ? rng[2] : 0;
        long lo1 = dims > 1 ? -rng[1] : 0, hi1 = dims > 1 ? rng[1] : 0;
        long lo0 = -rng[0], hi0 = rng[0];
        for (img[2] = lo2; img[2] <= hi2; ++img[2])
            for (img[1] = lo1; img[1] <= hi1; ++img[1])
                for (img[0] = lo0; img[0] <= hi0; ++img[0]) {
                    if (img[0] == 0 && img[1] == 0 && img[2] == 0)
                        continue;
                    double iv[3] = {(double)img[0], (double)img[1], (double)img[2]};
                    double b[3][3];
                    for (int r = 0; r < 3; ++r)
                        for (int c = 0; c < 3; ++c)
                            b[r][c] = basis[r * 3 + c] * iv[c];
                    double t[3];
                    t[0] = (b[0][0] + b[0][1]) + b[0][2];
                    t[1] = (b[1][0] + b[1][1]) + b[1][2];
                    t[2] = b[2][0] + (b[2][1] + b[2][2]);
                    for (int i = 0; i < n; ++i) {
                        double p0 = pts[3 * i] + t[0], p1 = pts[3 * i + 1] + t[1],
                               p2 = pts[3 * i + 2] + t[2];
                        if (p0 < lo[0] - cutoff || p1 < lo[1] - cutoff || p2 < lo[2] - cutoff ||
                            p0 > hi[0] + cutoff || p1 > hi[1] + cutoff || p2 > hi[2] + cutoff)
                            continue;
                        if (npts == cap) {
                            cap *= 2;
                            pts = (double *)realloc(pts, sizeof(double) * 3 * (size_t)cap);
                            orig = (int *)realloc(orig, sizeof(int) * (size_t)cap);
                        }
                        pts[3 * npts] = p0;
                        pts[3 * npts + 1] = p1;
                        pts[3 * npts + 2] = p2;
                        orig[npts] = i;
                        npts++;
                    }
                }
    }

    /* boxes (neighborhoods_base.h:145-225) */
    double xd[3] = {hi[0] - lo[0], hi[1] - lo[1], hi[2] - lo[2]};
    int bl[3];
    for (int d = 0; d < 3; ++d) {
        double count = floor((hi[d] - lo[d]) / cutoff) + 2;
        if (!isfinite(count) || count >= (double)INT_MAX) {
            set_err(err, errlen, "Neighbor spatial box count exceeds integer range");
            free(pts);
            free(orig);
            orc_nbh_free(h);
            return NULL;
        }
        bl[d] = (int)count;
        if (bl[d] == 2)
            bl[d] = 3;
    }
    int64_t nbox = (int64_t)bl[0] * bl[1] * bl[2];
    int *pbox = (int *)malloc(sizeof(int) * (size_t)npts);
    for (int i = 0; i < npts; ++i) {
        double tp1 = pts[3 * i] - lo[0], tp2 = pts[3 * i + 1] - lo[1], tp3 = pts[3 * i + 2] - lo[2];
        int i1 = (int)ceil(tp1 * (bl[0] - 2) / xd[0]);
        int i2 = (int)ceil(tp2 * (bl[1] - 2) / xd[1]);
        int i3 = (int)ceil(tp3 * (bl[2] - 2) / xd[2]);
        if (i < n) {
            if (i1 == 0) i1 = 1;
            if (i2 == 0) i2 = 1;
            if (i3 == 0) i3 = 1;
            if (i1 == bl[0] - 1) --i1;
            if (i2 == bl[1] - 1) --i2;
            if (i3 == bl[2] - 1) --i3;
        } else {
            if (i1 < 0) i1 = 0;
            if (i2 < 0) i2 = 0;
            if (i3 < 0) i3 = 0;
            if (i1 >= bl[0]) i1 = bl[0] - 1;
            if (i2 >= bl[1]) i2 = bl[1] - 1;
            if (i3 >= bl[2]) i3 = bl[2] - 1;
        }
        pbox[i] = (i1 * bl[1] + i2) * bl[2] + i3;
    }
    boxes_t bx;
    bx.start = (int *)calloc((size_t)nbox + 1, sizeof(int));
    bx.items = (int *)malloc(sizeof(int) * (size_t)npts);
    for (int i = 0; i < npts; ++i)
        bx.start[pbox[i] + 1]++;
    for (int64_t b = 0; b < nbox; ++b)
        bx.start[b + 1] += bx.start[b];
    {
        int *cur = (int *)malloc(sizeof(int) * (size_t)nbox);
        for (int64_t b = 0; b < nbox; ++b)
            cur[b] = bx.start[b];
        for (int i = 0; i < npts; ++i) /* insertion order: originals, then images */
            bx.items[cur[pbox[i]]++] = i;
        free(cur);
    }

    /* construct (neighborhood.cpp:77-146): two passes, count then fill; the
     * fill repeats the traversal so each list keeps its append order. */
    const double cutoffsq = cutoff * cutoff;
    int *cnt = (int *)calloc((size_t)n, sizeof(int));
    int *cur = NULL;
    for (int pass = 0; pass < 2; ++pass) {
        if (pass == 1) {
            for (int i = 0; i < n; ++i)
                h->offsets[i + 1] = h->offsets[i] + cnt[i];
            h->P = h->offsets[n];
            size_t P = (size_t)(h->P > 0 ? h->P : 1);
            h->idx = (int *)malloc(sizeof(int) * P);
            h->types = (int *)malloc(sizeof(int) * P);
            h->vec = (double *)malloc(sizeof(double) * 3 * P);
            h->dist = (double *)malloc(sizeof(double) * P);
            h->pt = (int *)malloc(sizeof(int) * P);
            cur = (int *)malloc(sizeof(int) * (size_t)n);
            for (int i = 0; i < n; ++i)
                cur[i] = h->offsets[i];
        }
        for (int i = 1; i < bl[0] - 1; ++i)
            for (int j = 1; j < bl[1] - 1; ++j)
                for (int k = 1; k < bl[2] - 1; ++k) {
                    int bidx = (i * bl[1] + j) * bl[2] + k;
                    for (int s = bx.start[bidx]; s < bx.start[bidx + 1]; ++s) {
                        int indi = bx.items[s];
                        if (indi >= n)
                            continue;
                        h->center_types[indi] = types[indi];
                        for (int l1 = -1; l1 <= 1; l1++)
                            for (int l2 = -1; l2 <= 1; l2++)
                                for (int l3 = -1; l3 <= 1; l3++) {
                                    int nb = ((i + l1) * bl[1] + (j + l2)) * bl[2] + (k + l3);
                                    for (int t = bx.start[nb]; t < bx.start[nb + 1]; ++t) {
                                        int indj = bx.items[t];
                                        double r0 = pts[3 * indj] - pts[3 * indi];
                                        double r1 = pts[3 * indj + 1] - pts[3 * indi + 1];
                                        double r2 = pts[3 * indj + 2] - pts[3 * indi + 2];
                                        const double dijsq = r0 * r0 + r1 * r1 + r2 * r2;
                                        int oj = orig[indj];
                                        if (dijsq < cutoffsq && indi != indj && indi <= oj) {
                                            if (pass == 0) {
                                                cnt[indi]++;
                                                if (indi != oj)
                                                    cnt[oj]++;
                                                continue;
                                            }
                                            const double dij = sqrt(dijsq);
                                            int q = cur[indi]++;
                                            h->idx[q] = oj;
                                            h->types[q] = types[oj];
                                            h->vec[3 * q] = r0;
                                            h->vec[3 * q + 1] = r1;
                                            h->vec[3 * q + 2] = r2;
                                            h->dist[q] = dij;
                                            h->pt[q] = indj;
                                            if (indi != oj) {
                                                q = cur[oj]++;
                                                h->idx[q] = indi;
                                                h->types[q] = types[indi];
                                                h->vec[3 * q] = -r0;
                                                h->vec[3 * q + 1] = -r1;
                                                h->vec[3 * q + 2] = -r2;
                                                h->dist[q] = dij;
                                                h->pt[q] = -1 - indj;
                                            }
                                        }
                                    }
                                }
                    }
                }
    }
    free(cnt);
    free(cur);
    free(pbox);
    free(bx.start);
    free(bx.items);
    h->npts = npts;
    h->pts = pts;
    h->orig = orig;
    h->boxle[0] = bl[0];
    h->boxle[1] = bl[1];
    h->boxle[2] = bl[2];
    return h;
}

orc_nbh *orc_nbh_from_csr(int n, const int *offsets, const int *idx, const int *types,
                          const double *vec, const double *dist, const int *center_types)
{
    orc_nbh *h = (orc_nbh *)calloc(1, sizeof(orc_nbh));
    h->n = n;
    h->P = offsets[n];
    size_t P = (size_t)(h->P > 0 ? h->P : 1);
    h->offsets = (int *)malloc(sizeof(int) * ((size_t)n + 1));
    memcpy(h->offsets, offsets, sizeof(int) * ((size_t)n + 1));
    h->idx = (int *)malloc(sizeof(int) * P);
    h->types = (int *)malloc(sizeof(int) * P);
    h->vec = (double *)malloc(sizeof(double) * 3 * P);
    h->dist = (double *)malloc(sizeof(double) * P);
    h->pt = (int *)calloc(P, sizeof(int));
    memcpy(h->idx, idx, sizeof(int) * (size_t)h->P);
    memcpy(h->types, types, sizeof(int) * (size_t)h->P);
    memcpy(h->vec, vec, sizeof(double) * 3 * (size_t)h->P);
    memcpy(h->dist, dist, sizeof(double) * (size_t)h->P);
    h->center_types = (int *)malloc(sizeof(int) * (size_t)(n > 0 ? n : 1));
    memcpy(h->center_types, center_types, sizeof(int) * (size_t)n);
    return h;
}

int64_t orc_nbh_size(const orc_nbh *h, int *n, int *npts, int *boxle)
{
    if (n)
        *n = h->n;
    if (npts)
        *npts = h->npts;
    if (boxle)
        memcpy(boxle, h->boxle, sizeof(int) * 3);
    return h->P;
}

void orc_nbh_export(const orc_nbh *h, int *offsets, int *idx, int *types, double *vec,
                    double *dist, int *pt, int *center_types)
{
    size_t P = (size_t)h->P;
    if (offsets)
        memcpy(offsets, h->offsets, sizeof(int) * ((size_t)h->n + 1));
    if (idx)
        memcpy(idx, h->idx, sizeof(int) * P);
    if (types)
        memcpy(types, h->types, sizeof(int) * P);
    if (vec)
        memcpy(vec, h->vec, sizeof(double) * 3 * P);
    if (dist)
        memcpy(dist, h->dist, sizeof(double) * P);
    if (pt)
        memcpy(pt, h->pt, sizeof(int) * P);
    if (center_types)
        memcpy(center_types, h->center_types, sizeof(int) * (size_t)h->n);
}

void orc_nbh_export_points(const orc_nbh *h, double *pts, int *orig)
{
    if (pts)
        memcpy(pts, h->pts, sizeof(double) * 3 * (size_t)h->npts);
    if (orig)
        memcpy(orig, h->orig, sizeof(int) * (size_t)h->npts);
}

/* ======================================================================
 * Per-site kernels
 * ====================================================================== */
typedef struct {
    int nmax;
    double *mv, *A, *rv, *rd, *vm, *dm, *dp, *cp; /* cp: [(max_nu1+1)][3] */
    double *mj;                                    /* [K or B][nmax][3] */
    double *ders;                                  /* [nmax][3] */
    /* training */
    double *mjc, *mjcc, *dsend, *dmom, *fw;
} ws_t;

static void ws_free(ws_t *w)
{
    free(w->mv);
    free(w->A);
    free(w->rv);
    free(w->rd);
    free(w->vm);
    free(w->dm);
    free(w->dp);
    free(w->cp);
    free(w->mj);
    free(w->ders);
    free(w->mjc);
    free(w->mjcc);
    free(w->dsend);
    free(w->dmom);
    free(w->fw);
    memset(w, 0, sizeof *w);
}

static void ws_init(ws_t *w, const orc_model *m, int nmax, int full_jac, int training)
{
    memset(w, 0, sizeof *w);
    w->nmax = nmax;
    size_t K = (size_t)(m->K > 0 ? m->K : 1);
    w->mv = (double *)calloc(K, sizeof(double));
    w->A = (double *)calloc(K, sizeof(double));
    w->rv = (double *)calloc((size_t)m->R, sizeof(double));
    w->rd = (double *)calloc((size_t)m->R, sizeof(double));
    w->vm = (double *)calloc((size_t)(m->max_mu > 0 ? m->max_mu : 1), sizeof(double));
    w->dm = (double *)calloc((size_t)(m->max_mu > 0 ? m->max_mu : 1), sizeof(double));
    w->dp = (double *)calloc((size_t)m->max_nu1 + 6, sizeof(double));
    w->cp = (double *)calloc(((size_t)m->max_nu1 + 1) * 3, sizeof(double));
    size_t rows = full_jac ? K : (size_t)(m->B > 0 ? m->B : 1);
    w->mj = (double *)calloc(rows * (size_t)(nmax > 0 ? nmax : 1) * 3, sizeof(double));
    w->ders = (double *)calloc((size_t)(nmax > 0 ? nmax : 1) * 3, sizeof(double));
    if (training) {
        size_t n = (size_t)(m->B > 0 ? m->B : 1) * (size_t)m->Z * (size_t)m->M * (size_t)m->R;
        w->mjc = (double *)calloc(n, sizeof(double));
        w->mjcc = (double *)calloc(n, sizeof(double));
        w->dsend = (double *)calloc(K, sizeof(double));
        w->dmom = (double *)calloc(K, sizeof(double));
        w->fw = (double *)calloc((size_t)(nmax > 0 ? nmax : 1) * 3, sizeof(double));
    }
    /* coords_powers rows 0 and 1 (potential_mtp.cpp:590-592) */
    w->cp[0] = w->cp[1] = w->cp[2] = 0;
    w->cp[3] = w->cp[4] = w->cp[5] = 1;
}

static int max_list(const orc_nbh *h)
{
    int mx = 0;
    for (int i = 0; i < h->n; ++i) {
        int c = h->offsets[i + 1] - h->offsets[i];
        if (c > mx)
            mx = c;
    }
    return mx;
}

/* CalcSiteDescriptorsImpl (potential_mtp.cpp:2813-2925): moment values and
 * the basic-moment Jacobian [B][n][3]; jac = 0 gives the energy-only
 * CalcSiteBasisImpl (:3024-3122). */
static void site_descriptors(const orc_model *m, const orc_nbh *h, int i, ws_t *w, int jac)
{
    const int n = h->offsets[i + 1] - h->offsets[i];
    const int off = h->offsets[i];
    const double *radial = m->coef;
    if (jac)
        memset(w->mj, 0, sizeof(double) * (size_t)m->B * (size_t)n * 3);
    memset(w->mv, 0, sizeof(double) * (size_t)m->K);
    const int itype = h->center_types[i];
    for (int jj = 0; jj < n; ++jj) {
        const double rij = h->dist[off + jj];
        const int jtype = h->types[off + jj];
        const double *pos = h->vec + 3 * (size_t)(off + jj);
        if (rij > pair_cutoff(m, itype, jtype)) /* :2842, r == cutoff is kept */
            continue;
        const double rijinv = 1.0 / rij;
        orc_rb_calc_der_pair(m, itype, jtype, rij, w->rv, w->rd);
        w->dp[0] = 1;
        for (int k = 1; k < m->max_nu1; ++k) {
            w->dp[k] = w->dp[k - 1] * rijinv;
            for (int a = 0; a < 3; a++)
                w->cp[(k + 1) * 3 + a] = w->cp[k * 3 + a] * pos[a];
        }
        for (int mu = 0; mu < m->max_mu; ++mu) {
            w->vm[mu] = 0;
            w->dm[mu] = 0;
            int idxoffset = (itype * m->Z + jtype) * m->M * m->R + mu * m->R;
            for (int xi = 0; xi < m->R; ++xi) {
                w->vm[mu] += radial[idxoffset + xi] * w->rv[xi];
                w->dm[mu] += radial[idxoffset + xi] * w->rd[xi];
            }
        }
        for (int b = 0; b < m->B; ++b) {
            const int *ab = m->basic + 4 * b;
            int mu = ab[0];
            double val = w->vm[mu];
            double der = w->dm[mu];
            int k = m->nu[b];
            double powk = w->dp[k];
            val *= powk;
            der = der * powk - k * val / rij;
            double pow0 = w->cp[(ab[1] + 1) * 3 + 0];
            double pow1 = w->cp[(ab[2] + 1) * 3 + 1];
            double pow2 = w->cp[(ab[3] + 1) * 3 + 2];
            double mult0 = pow0 * pow1 * pow2;
            w->mv[b] += val * mult0;
            if (!jac)
                continue;
            mult0 *= der / rij;
            double *J = w->mj + ((size_t)b * n + jj) * 3;
            J[0] += mult0 * pos[0];
            J[1] += mult0 * pos[1];
            J[2] += mult0 * pos[2];
            J[0] += ab[1] * val * w->cp[ab[1] * 3 + 0] * pow1 * pow2;
            J[1] += ab[2] * val * w->cp[ab[2] * 3 + 1] * pow0 * pow2;
            J[2] += ab[3] * val * w->cp[ab[3] * 3 + 2] * pow0 * pow1;
        }
    }
    for (int t = 0; t < m->T; ++t) { /* :2918-2924 */
        const int *r = m->times + 4 * t;
        double val0 = w->mv[r[0]];
        double val1 = w->mv[r[1]];
        int val2 = r[2];
        w->mv[r[3]] += val2 * val0 * val1;
    }
}

/* backpropagate_moments (potential_mtp.cpp:3292-3305) */
static void backpropagate(const orc_model *m, const double *mv, double *A)
{
    for (int t = m->T - 1; t >= 0; t--) {
        const int *r = m->times + 4 * t;
        double val0 = mv[r[0]];
        double val1 = mv[r[1]];
        int val2 = r[2];
        A[r[1]] += A[r[3]] * val2 * val0;
        A[r[0]] += A[r[3]] * val2 * val1;
    }
}

/* The activations of the neural heads (mtp_cpu.cpp:21-45). */
static double activate(double x, int act, double *der)
{
    if (act == 0) {
        const double v = tanh(x);
        *der = 1.0 - v * v;
        return v;
    }
    if (act == 1) {
        *der = x > 0.0 ? 1.0 : 0.0;
        return x > 0.0 ? x : 0.0;
    }
    if (act == 2) {
        const double v = 1.0 / (1.0 + exp(-x));
        *der = v * (1.0 - v);
        return v;
    }
    *der = 1.0;
    return x;
}

/* The MTP-M head (Executor::head, mtp_cpu.cpp:291-368; m_model_mtpq2,
 * m_model_mtpfs, m_model_nn1, m_model_nn2 of potential_mtp_m.h): the
 * energy of the descriptors Q [P] and, into dq, its gradient. */
static double mtpm_head(const orc_model *m, const double *Q, double *dq)
{
    const double *c = m->coef + m->nradial + m->Z * (m->P + 1) + m->P * m->S;
    const int q = m->P, h1 = m->h1, h2 = m->h2;
    if (m->head == 1) {
        dq[0] = 1.0;
        return Q[0];
    }
    if (m->head == 2) {
        const double x = Q[0], y = Q[1];
        dq[0] = c[0] + 2.0 * c[2] * x + c[4] * y;
        dq[1] = c[1] + 2.0 * c[3] * y + c[4] * x;
        return c[0] * x + c[1] * y + c[2] * x * x + c[3] * y * y + c[4] * x * y;
    }
    if (m->head == 3) {
        dq[0] = 1.0;
        dq[1] = c[0] / sqrt(1.0 + Q[1] * Q[1]);
        return Q[0] + c[0] * asinh(Q[1]);
    }
    const int nn2 = m->head == 5;
    const double *b1 = c + q * h1 + (nn2 ? 0 : h1);
    const double *w2 = nn2 ? b1 + h1 : NULL;
    const double *b2 = nn2 ? w2 + h1 * h2 : NULL;
    const double *out = nn2 ? b2 + h2 : c + q * h1;
    double *a1 = (double *)calloc((size_t)(2 * h1 + h2 + 1), sizeof(double));
    double *d1 = a1 + h1, *g2 = d1 + h1;
    double e = 0.0;
    for (int p = 0; p < q; ++p)
        dq[p] = 0.0;
    for (int h = 0; h < h1; ++h) {
        double v = b1[h];
        for (int p = 0; p < q; ++p)
            v += c[h * q + p] * Q[p];
        a1[h] = activate(v, m->act, &d1[h]);
        if (!nn2)
            e += out[h] * a1[h];
    }
    if (nn2)
        for (int h = 0; h < h2; ++h) {
            double v = b2[h], d = 0.0;
            for (int k = 0; k < h1; ++k)
                v += w2[h * h1 + k] * a1[k];
            e += out[h] * activate(v, m->act, &d);
            g2[h] = out[h] * d;
        }
    for (int h = 0; h < h1; ++h) {
        double resp = nn2 ? 0.0 : out[h];
        if (nn2)
            for (int k = 0; k < h2; ++k)
                resp += w2[k * h1 + h] * g2[k];
        resp *= d1[h];
        for (int p = 0; p < q; ++p)
            dq[p] += c[h * q + p] * resp;
    }
    free(a1);
    return e;
}

/* The site energy and the adjoint seeds dE/dm of the scalar moments: the
 * linear MTP (potential_mtp.cpp:2959-2970) or the MTP-M head over the
 * descriptors Q_p (potential_mtp_m.h:3403-3456). */
static double site_energy_seeds(const orc_model *m, int t, const double *mv, double *A)
{
    const double *species = m->coef + m->nradial;
    double e = species[t];
    if (!m->head) {
        const double *moment = species + m->Z;
        for (int s = 0; s < m->S; ++s)
            e += moment[s] * mv[m->map[s]];
        if (A)
            for (int s = 0; s < m->S; ++s)
                A[m->map[s]] += moment[s];
        return e;
    }
    const double *dsp = species + m->Z, *C = species + m->Z * (m->P + 1);
    double *Q = (double *)calloc((size_t)(2 * m->P), sizeof(double)), *dq = Q + m->P;
    for (int p = 0; p < m->P; ++p) {
        Q[p] = dsp[p * m->Z + t];
        for (int s = 0; s < m->S; ++s)
            Q[p] += mv[m->map[s]] * C[p * m->S + s];
    }
    const double hv = mtpm_head(m, Q, dq);
    if (A)
        for (int s = 0; s < m->S; ++s)
            for (int p = 0; p < m->P; ++p)
                A[m->map[s]] += C[p * m->S + s] * dq[p];
    free(Q);
    return hv + e;
}

/* CalcSiteEFS (potential_mtp.cpp:2959-2984) with contract_site_forces
 * (:2938-2957). */
static double site_efs(const orc_model *m, const orc_nbh *h, int i, ws_t *w)
{
    const int n = h->offsets[i + 1] - h->offsets[i];
    site_descriptors(m, h, i, w, 1);
    memset(w->A, 0, sizeof(double) * (size_t)m->K);
    const double site_energy = site_energy_seeds(m, h->center_types[i], w->mv, w->A);
    backpropagate(m, w->mv, w->A);
    memset(w->ders, 0, sizeof(double) * (size_t)n * 3);
    for (int b = 0; b < m->B; ++b) {
        const double weight = w->A[b];
        const double *row = w->mj + (size_t)b * n * 3;
        for (int j = 0; j < 3 * n; ++j)
            w->ders[j] += weight * row[j];
    }
    return site_energy;
}

void orc_site_efs(const orc_model *m, const orc_nbh *h, int i, double *site_energy, double *ders)
{
    ws_t w;
    ws_init(&w, m, max_list(h), 0, 0);
    *site_energy = site_efs(m, h, i, &w);
    int n = h->offsets[i + 1] - h->offsets[i];
    memcpy(ders, w.ders, sizeof(double) * 3 * (size_t)n);
    ws_free(&w);
}

void orc_site_moments(const orc_model *m, const orc_nbh *h, int i, double *moments)
{
    ws_t w;
    ws_init(&w, m, max_list(h), 0, 0);
    site_descriptors(m, h, i, &w, 0);
    memcpy(moments, w.mv, sizeof(double) * (size_t)m->K);
    ws_free(&w);
}

static void scatter_site(const orc_nbh *h, int i, const double *ders, double *forces,
                         double *stress)
{
    const int n = h->offsets[i + 1] - h->offsets[i];
    const int off = h->offsets[i];
    for (int q = 0; q < n; ++q) {
        const double *d = ders + 3 * q;
        const double *r = h->vec + 3 * (size_t)(off + q);
        int j = h->idx[off + q];
        for (int a = 0; a < 3; ++a)
            forces[3 * i + a] += d[a];
        for (int a = 0; a < 3; ++a)
            forces[3 * j + a] -= d[a];
        for (int a = 0; a < 3; a++)
            for (int b = 0; b < 3; b++)
                stress[3 * a + b] -= d[a] * r[b];
    }
}

/* PotMTP::getEFS (potential_mtp.cpp:1899-1933) */
void orc_efs(const orc_model *m, const orc_nbh *h, double *energy, double *forces,
             double *stress, double *site_energies)
{
    ws_t w;
    ws_init(&w, m, max_list(h), 0, 0);
    *energy = 0;
    memset(forces, 0, sizeof(double) * 3 * (size_t)h->n);
    memset(stress, 0, sizeof(double) * 9);
    if (site_energies)
        memset(site_energies, 0, sizeof(double) * (size_t)h->n);
    for (int i = 0; i < h->n; ++i) {
        double se = site_efs(m, h, i, &w);
        *energy += se;
        if (site_energies)
            site_energies[i] += se;
        scatter_site(h, i, w.ders, forces, stress);
    }
    ws_free(&w);
}

/* PotMTP::getEFSOMP (potential_mtp.cpp:2416-2486): atom-parallel with
 * schedule(static), per-thread buffers and a serial merge in thread order. */
void orc_efs_omp(const orc_model *m, const orc_nbh *h, int nthreads, double *energy,
                 double *forces, double *stress, double *site_energies)
{
#ifdef _OPENMP
    if (nthreads <= 0)
        nthreads = omp_get_max_threads();
#else
    nthreads = 1;
#endif
    const int n = h->n, nmax = max_list(h);
    double *tf = (double *)calloc((size_t)nthreads * 3 * (size_t)(n > 0 ? n : 1), sizeof(double));
    double *ts = (double *)calloc((size_t)nthreads * 9, sizeof(double));
    double *te = (double *)calloc((size_t)nthreads, sizeof(double));
    int actual = 1;
    if (site_energies)
        memset(site_energies, 0, sizeof(double) * (size_t)n);
#ifdef _OPENMP
#pragma omp parallel num_threads(nthreads)
#endif
    {
        int it = 0;
#ifdef _OPENMP
        it = omp_get_thread_num();
        if (it == 0)
            actual = omp_get_num_threads();
#endif
        ws_t w;
        ws_init(&w, m, nmax, 0, 0);
        double *F = tf + (size_t)it * 3 * n;
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int i = 0; i < n; ++i) {
            double se = site_efs(m, h, i, &w);
            te[it] += se;
            if (site_energies)
                site_energies[i] += se;
            scatter_site(h, i, w.ders, F, ts + 9 * it);
        }
        ws_free(&w);
    }
    *energy = 0;
    memset(forces, 0, sizeof(double) * 3 * (size_t)n);
    memset(stress, 0, sizeof(double) * 9);
    for (int t = 0; t < actual; ++t) {
        *energy += te[t];
        for (int q = 0; q < 9; ++q)
            stress[q] += ts[9 * t + q];
        for (int i = 0; i < 3 * n; ++i)
            forces[i] += tf[(size_t)t * 3 * n + i];
    }
    free(tf);
    free(ts);
    free(te);
}

/* PotMTP::getE (potential_mtp.cpp:2604-2621) */
void orc_energy(const orc_model *m, const orc_nbh *h, double *energy, double *site_energies)
{
    ws_t w;
    ws_init(&w, m, max_list(h), 0, 0);
    *energy = 0;
    for (int i = 0; i < h->n; ++i) {
        site_descriptors(m, h, i, &w, 0);
        const double se = site_energy_seeds(m, h->center_types[i], w.mv, NULL);
        *energy += se;
        if (site_energies)
            site_energies[i] = se;
    }
    ws_free(&w);
}

/* ======================================================================
 * Training: accumulate_site_parameter_gradient (potential_mtp.cpp:3348-3550)
 * ====================================================================== */
static void site_parameter_gradient(const orc_model *m, const orc_nbh *h, int i, ws_t *w,
                                    double se_weight, const double *f_weight,
                                    double *radial_gradient, double *moment_gradient)
{
    const int need = f_weight != NULL;
    const int Z = m->Z, M = m->M, R = m->R, K = m->K, B = m->B;
    const size_t njc = (size_t)B * Z * M * R;
    const int n = h->offsets[i + 1] - h->offsets[i];
    const int off = h->offsets[i];
    const double *radial = m->coef;
    const double *moment = m->coef + m->nradial + Z;
    memset(w->mjc, 0, sizeof(double) * njc);
    memset(w->rd, 0, sizeof(double) * (size_t)R);
    if (need) {
        memset(w->mjcc, 0, sizeof(double) * njc);
        memset(w->dm, 0, sizeof(double) * (size_t)m->max_mu);
        memset(w->dsend, 0, sizeof(double) * (size_t)K);
    }
    memset(w->mv, 0, sizeof(double) * (size_t)K);
    memset(w->rv, 0, sizeof(double) * (size_t)R);
    memset(w->vm, 0, sizeof(double) * (size_t)m->max_mu);
    memset(w->dmom, 0, sizeof(double) * (size_t)K);
    memset(w->A, 0, sizeof(double) * (size_t)K);
    const int itype = h->center_types[i];
#define MJC(arr, b, j, k) arr[(((size_t)(b) * Z + (j)) * (size_t)M * R) + (k)]
    for (int jj = 0; jj < n; ++jj) {
        const double rij = h->dist[off + jj];
        const int jtype = h->types[off + jj];
        const double *pos = h->vec + 3 * (size_t)(off + jj);
        if (rij > pair_cutoff(m, itype, jtype))
            continue;
        const double rijinv = 1.0 / rij;
        orc_rb_calc_der_pair(m, itype, jtype, rij, w->rv, w->rd);
        w->dp[0] = 1;
        for (int k = 1; k < m->max_nu1; ++k) {
            w->dp[k] = w->dp[k - 1] * rijinv;
            for (int a = 0; a < 3; a++)
                w->cp[(k + 1) * 3 + a] = w->cp[k * 3 + a] * pos[a];
        }
        for (int mu = 0; mu < m->max_mu; ++mu) {
            w->vm[mu] = 0;
            if (need)
                w->dm[mu] = 0;
            int idxoffset = (itype * Z + jtype) * M * R + mu * R;
            for (int xi = 0; xi < R; ++xi) {
                w->vm[mu] += radial[idxoffset + xi] * w->rv[xi];
                if (need)
                    w->dm[mu] += radial[idxoffset + xi] * w->rd[xi];
            }
        }
        const double *fw = need ? f_weight + 3 * (size_t)jj : NULL;
        for (int b = 0; b < B; ++b) {
            const int *index = m->basic + 4 * b;
            const int mu = index[0], x = index[1], y = index[2], z = index[3];
            const int k = m->nu[b];
            const double powk = w->dp[k];
            const double val = w->vm[mu] * powk;
            const double pow0 = w->cp[(x + 1) * 3 + 0];
            const double pow1 = w->cp[(y + 1) * 3 + 1];
            const double pow2 = w->cp[(z + 1) * 3 + 2];
            const double mult0 = pow0 * pow1 * pow2;
            w->mv[b] += val * mult0;
            for (int xi = 0; xi < R; xi++) {
                MJC(w->mjc, b, jtype, mu * R + xi) += w->rv[xi] * powk * mult0;
                if (need) {
                    const double dist = h->dist[off + jj];
                    double tail = (w->rd[xi] * powk * mult0 - w->rv[xi] * k * powk * mult0 / dist);
                    double derx = (pos[0] / dist) * tail;
                    double dery = (pos[1] / dist) * tail;
                    double derz = (pos[2] / dist) * tail;
                    derx += w->rv[xi] * powk * x * w->cp[x * 3 + 0] * pow1 * pow2;
                    dery += w->rv[xi] * powk * y * w->cp[y * 3 + 1] * pow0 * pow2;
                    derz += w->rv[xi] * powk * z * w->cp[z * 3 + 2] * pow0 * pow1;
                    MJC(w->mjcc, b, jtype, mu * R + xi) +=
                        fw[0] * derx + fw[1] * dery + fw[2] * derz;
                }
            }
            if (need) {
                const double der = w->dm[mu] * powk - k * val / rij;
                const double radialt = mult0 * (der / rij);
                const double dx = radialt * pos[0] + x * val * w->cp[x * 3 + 0] * pow1 * pow2;
                const double dy = radialt * pos[1] + y * val * w->cp[y * 3 + 1] * pow0 * pow2;
                const double dz = radialt * pos[2] + z * val * w->cp[z * 3 + 2] * pow0 * pow1;
                w->dsend[b] += fw[0] * dx;
                w->dsend[b] += fw[1] * dy;
                w->dsend[b] += fw[2] * dz;
            }
        }
    }
    for (int t = 0; t < m->T; ++t) { /* :3443-3450 */
        const int *r = m->times + 4 * t;
        double val0 = w->mv[r[0]];
        double val1 = w->mv[r[1]];
        double val2 = r[2];
        w->mv[r[3]] += val2 * val0 * val1;
    }
    for (int s = 0; s < m->S; ++s) /* :3453-3455 */
        w->A[m->map[s]] += moment[s];
    backpropagate(m, w->mv, w->A);
    for (int b = 0; b < B; ++b)
        w->dmom[b] = se_weight * w->A[b];
    if (need) {
        for (int t = 0; t < m->T; ++t) { /* :3463-3471 */
            const int *r = m->times + 4 * t;
            double val2 = r[2];
            double val0 = w->mv[r[0]];
            double val1 = w->mv[r[1]];
            w->dsend[r[3]] += w->dsend[r[0]] * val2 * val1 + w->dsend[r[1]] * val2 * val0;
        }
        for (int t = 0; t < m->T; ++t) { /* :3480-3490 */
            const int *r = m->times + 4 * t;
            double val2 = r[2];
            w->dmom[r[1]] += w->dsend[r[0]] * w->A[r[3]] * val2;
            w->dmom[r[0]] += w->dsend[r[1]] * w->A[r[3]] * val2;
        }
        for (int t = m->T - 1; t >= 0; --t) { /* :3493-3503 */
            const int *r = m->times + 4 * t;
            double val0 = w->mv[r[0]];
            double val1 = w->mv[r[1]];
            double val2 = r[2];
            w->dmom[r[0]] += w->dmom[r[3]] * val2 * val1;
            w->dmom[r[1]] += w->dmom[r[3]] * val2 * val0;
        }
    }
    for (int b = 0; b < B; ++b) { /* :3505-3524 */
        const int channel = m->basic[4 * b] * R;
        for (int j = 0; j < Z; ++j) {
            const int pair = itype * Z + j;
            for (int k = channel; k < channel + R; ++k) {
                const int idx = pair * R * M + k;
                radial_gradient[idx] += w->dmom[b] * MJC(w->mjc, b, j, k);
                if (need)
                    radial_gradient[idx] += w->A[b] * MJC(w->mjcc, b, j, k);
            }
        }
    }
#undef MJC
    if (moment_gradient) /* :3525-3533 */
        for (int s = 0; s < m->S; ++s) {
            moment_gradient[s] += se_weight * w->mv[m->map[s]];
            if (need)
                moment_gradient[s] += w->dsend[m->map[s]];
        }
}

/* AccumulateFPGard (potential_mtp.cpp:3312-3318) */
static void accumulate_fp_grad(const orc_model *m, const orc_nbh *h, int i, ws_t *w,
                               double se_weight, const double *f_weight, double *grad)
{
    site_parameter_gradient(m, h, i, w, se_weight, f_weight, grad, grad + m->nradial + m->Z);
    grad[m->nradial + h->center_types[i]] += se_weight;
}

void orc_accumulate_fp_grad(const orc_model *m, const orc_nbh *h, int i, double se_weight,
                            const double *f_weight, double *grad)
{
    ws_t w;
    ws_init(&w, m, max_list(h), 0, 1);
    accumulate_fp_grad(m, h, i, &w, se_weight, f_weight, grad);
    ws_free(&w);
}

/* AccumulateEFSCombinationGard (potential_mtp.cpp:6896-6923) */
static void efs_combination_grad(const orc_model *m, const orc_nbh *h, ws_t *w, double dLdE,
                                 const double *dLdF, const double *dLdS, double *grad)
{
    for (int i = 0; i < h->n; ++i) {
        const int n = h->offsets[i + 1] - h->offsets[i];
        const int off = h->offsets[i];
        memset(w->fw, 0, sizeof(double) * 3 * (size_t)n);
        for (int j = 0; j < n; ++j)
            for (int a = 0; a < 3; ++a) {
                w->fw[3 * j + a] += dLdF[3 * i + a];
                w->fw[3 * j + a] -= dLdF[3 * h->idx[off + j] + a];
            }
        for (int j = 0; j < n; ++j)
            for (int a = 0; a < 3; ++a)
                for (int b = 0; b < 3; ++b)
                    w->fw[3 * j + a] -= dLdS[3 * a + b] * h->vec[3 * (size_t)(off + j) + b];
        accumulate_fp_grad(m, h, i, w, dLdE, w->fw, grad);
    }
}

void orc_accumulate_efs_combination_grad(const orc_model *m, const orc_nbh *h, double dLdE,
                                         const double *dLdF, const double *dLdS, double *grad)
{
    ws_t w;
    ws_init(&w, m, max_list(h), 0, 1);
    efs_combination_grad(m, h, &w, dLdE, dLdF, dLdS, grad);
    ws_free(&w);
}

/* Trainer_MTP::AddLossGard (train/train_mtp.cpp:3839-3996) with the weights of
 * :2552-2568.  metrics (optional, 6): loss_e, loss_f, loss_s,
 * sq_energy_at_error, sq_force_error, sq_stress_error. */
static int add_loss_grad(const orc_model *m, const orc_nbh *h, ws_t *w,
                         const orc_loss_settings *s, const orc_config *c, double *loss,
                         double *grad, double *metrics)
{
    const int N = c->n;
    if (N == 0)
        return 0;
    const int energy_only = !(s->weight_force > 0 && c->has_forces) &&
                            !(s->weight_stress > 0 && c->has_stress);
    double E = 0, S[9] = {0};
    double *F = (double *)calloc((size_t)N * 3, sizeof(double));
    double *dLdF = (double *)calloc((size_t)N * 3, sizeof(double));
    if (energy_only) {
        orc_energy(m, h, &E, NULL);
    } else {
        orc_efs(m, h, &E, F, S, NULL);
    }
    double dLdE = 0, dLdS[9] = {0};
    double cc = 1.0;
    if (s->force_norm_f > 0 && c->has_forces) {
        double avef = 0;
        for (int i = 0; i < N; ++i) {
            const double *f = c->forces + 3 * i;
            avef += (f[0] * f[0] + f[1] * f[1]) + f[2] * f[2];
        }
        avef /= N;
        cc = s->force_norm_d / (s->force_norm_d + pow(s->force_norm_f * avef, s->force_norm_p));
    }
    if (s->weight_force > 0 && c->has_forces) {
        double wfi = s->weight_force / pow(N, s->force_pow) * cc;
        for (int i = 0; i < N; ++i) {
            double wi = wfi;
            if (c->atomic_fitness)
                wi *= c->atomic_fitness[i];
            double d0 = F[3 * i] - c->forces[3 * i], d1 = F[3 * i + 1] - c->forces[3 * i + 1],
                   d2 = F[3 * i + 2] - c->forces[3 * i + 2];
            double ff = (d0 * d0 + d1 * d1) + d2 * d2;
            double ll = wi * ff;
            *loss += ll;
            if (metrics) {
                metrics[1] += ll;
                metrics[4] += ff;
            }
            for (int a = 0; a < 3; ++a)
                dLdF[3 * i + a] = 2.0 * wi * (F[3 * i + a] - c->forces[3 * i + a]);
        }
    }
    if (s->weight_stress > 0 && c->has_stress) {
        double wsi = s->weight_stress / pow(N, s->stress_pow) * cc;
        double ff = 0;
        for (int q = 0; q < 9; ++q) {
            double d = S[q] - c->stress[q];
            ff += d * d;
        }
        double ll = wsi * ff;
        *loss += ll;
        if (metrics) {
            metrics[2] += ll;
            metrics[5] += ff;
        }
        for (int q = 0; q < 9; ++q)
            dLdS[q] = 2 * wsi * (S[q] - c->stress[q]);
    }
    if (s->weight_eng > 0 && c->has_energy) {
        double wei = s->weight_eng / pow(N, s->eng_pow) * c->fitness * cc;
        double ff = (E - c->energy) * (E - c->energy);
        double ll = wei * ff;
        *loss += ll;
        if (metrics) {
            metrics[0] += ll;
            metrics[3] += ff / N / N;
        }
        dLdE = 2 * wei * (E - c->energy);
    }
    if (energy_only) {
        for (int i = 0; i < h->n; ++i)
            accumulate_fp_grad(m, h, i, w, dLdE, NULL, grad);
    } else {
        efs_combination_grad(m, h, w, dLdE, dLdF, dLdS, grad);
    }
    free(F);
    free(dLdF);
    return 0;
}

int orc_add_loss_grad(const orc_model *m, const orc_nbh *h, const orc_loss_settings *s,
                      const orc_config *c, double *loss, double *grad, double *metrics)
{
    ws_t w;
    ws_init(&w, m, max_list(h), 0, 1);
    int rc = add_loss_grad(m, h, &w, s, c, loss, grad, metrics);
    ws_free(&w);
    return rc;
}

/* PotMTP::AddPenaltyGard, radial_mode 0 (potential_mtp.cpp:6568-6742) */
void orc_add_penalty_grad(const orc_model *m, double weight, double reg_l2, double reg_l1,
                          double *loss, double *grad)
{
    const int Z = m->Z, M = m->M, R = m->R;
    const double *c = m->coef;
    for (int k = 0; k < M; k++) {
        double norm = 0;
        for (int i = 0; i < Z; i++)
            for (int j = 0; j < Z; j++)
                for (int l = 0; l < R; l++) {
                    int idx = (i * Z + j) * R * M + k * R + l;
                    norm += c[idx] * c[idx];
                }
        *loss += weight * (norm - 1) * (norm - 1);
        for (int i = 0; i < Z; i++)
            for (int j = 0; j < Z; j++)
                for (int l = 0; l < R; l++) {
                    int idx = (i * Z + j) * R * M + k * R + l;
                    grad[idx] += weight * 4 * (norm - 1) * c[idx];
                }
    }
    for (int k1 = 0; k1 < M; k1++)
        for (int k2 = k1 + 1; k2 < M; k2++) {
            double scal = 0;
            for (int i = 0; i < Z; i++)
                for (int j = 0; j < Z; j++)
                    for (int l = 0; l < R; l++) {
                        int i1 = (i * Z + j) * R * M + k1 * R + l;
                        int i2 = (i * Z + j) * R * M + k2 * R + l;
                        scal += c[i1] * c[i2];
                    }
            *loss += weight * scal * scal;
            for (int i = 0; i < Z; i++)
                for (int j = 0; j < Z; j++)
                    for (int l = 0; l < R; l++) {
                        int i1 = (i * Z + j) * R * M + k1 * R + l;
                        int i2 = (i * Z + j) * R * M + k2 * R + l;
                        grad[i1] += weight * 2 * scal * c[i2];
                        grad[i2] += weight * 2 * scal * c[i1];
                    }
        }
    const double *lin = c + m->nradial;
    const int lsize = Z + m->S;
    for (int i = Z; i < lsize; i++) {
        *loss += lin[i] * lin[i] * reg_l2;
        *loss += fabs(lin[i]) * reg_l1;
    }
    for (int i = Z; i < lsize; i++) {
        grad[m->nradial + i] += 2 * lin[i] * reg_l2;
        grad[m->nradial + i] += lin[i] > 0 ? reg_l1 : -reg_l1;
    }
}

/* Trainer_MTP::AccumulateGard (train/train_mtp.cpp:3039-3094): f = sum L_c / M +
 * penalty, g = sum g_c / M + penalty gradient.  Configurations are split over
 * threads with per-thread accumulators merged in thread order, the
 * shared-memory analogue of the reference's MPI rank split. */
int orc_loss_grad_batch(const orc_model *m, int nconf, orc_nbh *const *hs,
                        const orc_config *cs, const orc_loss_settings *s, double penalty_weight,
                        double reg_l2, double reg_l1, int nthreads, double *f, double *g)
{
#ifdef _OPENMP
    if (nthreads <= 0)
        nthreads = omp_get_max_threads();
#else
    nthreads = 1;
#endif
    const int nc = m->ncoef;
    double *tl = (double *)calloc((size_t)nthreads, sizeof(double));
    double *tg = (double *)calloc((size_t)nthreads * nc, sizeof(double));
    int nmax = 0;
    for (int c = 0; c < nconf; ++c) {
        int q = max_list(hs[c]);
        if (q > nmax)
            nmax = q;
    }
    int actual = 1;
#ifdef _OPENMP
#pragma omp parallel num_threads(nthreads)
#endif
    {
        int it = 0;
#ifdef _OPENMP
        it = omp_get_thread_num();
        if (it == 0)
            actual = omp_get_num_threads();
#endif
        ws_t w;
        ws_init(&w, m, nmax, 0, 1);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int c = 0; c < nconf; ++c)
            add_loss_grad(m, hs[c], &w, s, cs + c, tl + it, tg + (size_t)it * nc, NULL);
        ws_free(&w);
    }
    double loss = 0;
    memset(g, 0, sizeof(double) * (size_t)nc);
    for (int t = 0; t < actual; ++t) {
        loss += tl[t];
        for (int q = 0; q < nc; ++q)
            g[q] += tg[(size_t)t * nc + q];
    }
    double ploss = 0;
    double *pg = (double *)calloc((size_t)nc, sizeof(double));
    orc_add_penalty_grad(m, penalty_weight, reg_l2, reg_l1, &ploss, pg);
    *f = loss / nconf + ploss;
    for (int q = 0; q < nc; ++q)
        g[q] = g[q] / nconf + pg[q];
    free(pg);
    free(tl);
    free(tg);
    return 0;
}

/* ======================================================================
 * Linear fit: CalcSiteBasisDers (potential_mtp.cpp:3163-3280), CalcEFSCmpt_R
 * (:2675-2707), AddLinearFast row order and sqrt(w) scaling
 * (train/train_mtp.cpp:1289-1395, 2570-2692), Gram (:2426-2427).
 * ====================================================================== */
static void site_basis_ders(const orc_model *m, const orc_nbh *h, int i, ws_t *w)
{
    const int n = h->offsets[i + 1] - h->offsets[i];
    const int off = h->offsets[i];
    const double *radial = m->coef;
    const size_t stride = 3 * (size_t)n;
    memset(w->mj, 0, sizeof(double) * (size_t)m->K * stride);
    memset(w->mv, 0, sizeof(double) * (size_t)m->K);
    const int itype = h->center_types[i];
    for (int jj = 0; jj < n; ++jj) {
        const double rij = h->dist[off + jj];
        const int jtype = h->types[off + jj];
        const double *pos = h->vec + 3 * (size_t)(off + jj);
        if (rij > pair_cutoff(m, itype, jtype))
            continue;
        const double rijinv = 1.0 / rij;
        orc_rb_calc_der_pair(m, itype, jtype, rij, w->rv, w->rd);
        w->dp[0] = 1;
        for (int k = 1; k < m->max_nu1; ++k) {
            w->dp[k] = w->dp[k - 1] * rijinv;
            for (int a = 0; a < 3; a++)
                w->cp[(k + 1) * 3 + a] = w->cp[k * 3 + a] * pos[a];
        }
        for (int mu = 0; mu < m->max_mu; ++mu) {
            w->vm[mu] = 0;
            w->dm[mu] = 0;
            int idxoffset = (itype * m->Z + jtype) * m->M * m->R + mu * m->R;
            for (int xi = 0; xi < m->R; xi++) {
                w->vm[mu] += radial[idxoffset + xi] * w->rv[xi];
                w->dm[mu] += radial[idxoffset + xi] * w->rd[xi];
            }
        }
        for (int b = 0; b < m->B; ++b) {
            const int *ab = m->basic + 4 * b;
            int mu = ab[0];
            double val = w->vm[mu];
            double der = w->dm[mu];
            int k = m->nu[b];
            double powk = w->dp[k];
            val *= powk;
            der = der * powk - k * val / rij;
            double pow0 = w->cp[(ab[1] + 1) * 3 + 0];
            double pow1 = w->cp[(ab[2] + 1) * 3 + 1];
            double pow2 = w->cp[(ab[3] + 1) * 3 + 2];
            double mult0 = pow0 * pow1 * pow2;
            w->mv[b] += val * mult0;
            mult0 *= der / rij;
            double *J = w->mj + (size_t)b * stride + 3 * (size_t)jj;
            J[0] += mult0 * pos[0];
            J[1] += mult0 * pos[1];
            J[2] += mult0 * pos[2];
            J[0] += val * ab[1] * w->cp[ab[1] * 3 + 0] * pow1 * pow2;
            J[1] += val * ab[2] * w->cp[ab[2] * 3 + 1] * pow0 * pow2;
            J[2] += val * ab[3] * w->cp[ab[3] * 3 + 2] * pow0 * pow1;
        }
    }
    for (int t = 0; t < m->T; ++t) {
        const int *rule = m->times + 4 * t;
        const double left = w->mv[rule[0]];
        const double right = w->mv[rule[1]];
        const int factor = rule[2];
        w->mv[rule[3]] += factor * left * right;
        const double *lrow = w->mj + (size_t)rule[0] * stride;
        const double *rrow = w->mj + (size_t)rule[1] * stride;
        double *orow = w->mj + (size_t)rule[3] * stride;
        for (size_t j = 0; j < stride; ++j)
            orow[j] += factor * (lrow[j] * right + left * rrow[j]);
    }
}

void orc_efs_components(const orc_model *m, const orc_nbh *h, double *energy_cmpts,
                        double *force_cmpts, double *stress_cmpts)
{
    const int Z = m->Z, p = m->Z + m->S, N = h->n;
    ws_t w;
    ws_init(&w, m, max_list(h), 1, 0);
    memset(energy_cmpts, 0, sizeof(double) * (size_t)p);
    memset(force_cmpts, 0, sizeof(double) * (size_t)N * 3 * p);
    memset(stress_cmpts, 0, sizeof(double) * 9 * (size_t)p);
    for (int id = 0; id < N; ++id) {
        site_basis_ders(m, h, id, &w);
        const int n = h->offsets[id + 1] - h->offsets[id];
        const int off = h->offsets[id];
        const size_t stride = 3 * (size_t)n;
        energy_cmpts[h->center_types[id]] += 1.0;
        for (int k = Z; k < p; ++k) {
            const int moment = m->map[k - Z];
            const double *bd = w.mj + (size_t)moment * stride;
            energy_cmpts[k] += w.mv[moment];
            for (int j = 0; j < n; ++j) {
                int jdx = h->idx[off + j];
                for (int a = 0; a < 3; ++a) {
                    force_cmpts[((size_t)id * 3 + a) * p + k] += bd[3 * j + a];
                    force_cmpts[((size_t)jdx * 3 + a) * p + k] -= bd[3 * j + a];
                }
            }
            for (int j = 0; j < n; ++j)
                for (int a = 0; a < 3; ++a)
                    for (int b = 0; b < 3; ++b)
                        stress_cmpts[(a * 3 + b) * p + k] -=
                            bd[3 * j + a] * h->vec[3 * (size_t)(off + j) + b];
        }
    }
    ws_free(&w);
}

static double force_norm_cc(const orc_loss_settings *s, const orc_config *c)
{
    double cc = 1.0;
    if (s->force_norm_f > 0 && c->has_forces) {
        double avef = 0;
        for (int i = 0; i < c->n; ++i) {
            const double *f = c->forces + 3 * i;
            avef += (f[0] * f[0] + f[1] * f[1]) + f[2] * f[2];
        }
        avef /= c->n;
        cc = s->force_norm_d / (s->force_norm_d + pow(s->force_norm_f * avef, s->force_norm_p));
    }
    return cc;
}

int64_t orc_linear_row_count(const orc_loss_settings *s, const orc_config *c)
{
    int64_t rows = 0;
    double cc = force_norm_cc(s, c);
    if (s->weight_force > 0 && c->has_forces) {
        double wfi = s->weight_force / pow(c->n, s->force_pow) * cc;
        for (int i = 0; i < c->n; ++i) {
            double wi = wfi * (c->atomic_fitness ? c->atomic_fitness[i] : 1.0);
            if (wi > 0)
                rows += 3;
        }
    }
    if (s->weight_stress > 0 && c->has_stress)
        rows += 9;
    if (s->weight_eng > 0 && c->has_energy)
        rows += 1;
    return rows;
}

int64_t orc_linear_rows(const orc_model *m, const orc_nbh *h, const orc_loss_settings *s,
                        const orc_config *c, double *A, double *y)
{
    return orc_linear_rows_ex(m, h, s, c, 0, A, y);
}

/* With fix_species (Trainer_MTP::fix_species_coeffs, train_mtp.cpp:1300-1302,
 * 1381-1392) every row drops the Z species columns (soffset = Z, rows of
 * n_size_mat = S values) and the energy target becomes
 * E - sum_s energy_cmpts[s] species_coeffs[s]. */
int64_t orc_linear_rows_ex(const orc_model *m, const orc_nbh *h, const orc_loss_settings *s,
                           const orc_config *c, int fix_species, double *A, double *y)
{
    const int p = m->Z + m->S, N = c->n;
    const int off = fix_species ? m->Z : 0, w = p - off;
    double *ec = (double *)calloc((size_t)p, sizeof(double));
    double *fc = (double *)calloc((size_t)N * 3 * p + 1, sizeof(double));
    double *sc = (double *)calloc(9 * (size_t)p, sizeof(double));
    orc_efs_components(m, h, ec, fc, sc);
    double cc = force_norm_cc(s, c);
    int64_t row = 0;
    if (s->weight_force > 0 && c->has_forces) {
        double wfi = s->weight_force / pow(N, s->force_pow) * cc;
        for (int iat = 0; iat < N; ++iat) {
            double wi = wfi * (c->atomic_fitness ? c->atomic_fitness[iat] : 1.0);
            if (c->atomic_fitness && !(c->atomic_fitness[iat] > 0))
                continue;
            double sw = sqrt(wi);
            for (int a = 0; a < 3; ++a) {
                for (int q = 0; q < w; ++q)
                    A[row * w + q] = fc[((size_t)iat * 3 + a) * p + off + q] * sw;
                y[row] = sw * c->forces[3 * iat + a];
                row++;
            }
        }
    }
    if (s->weight_stress > 0 && c->has_stress) {
        double sw = sqrt(s->weight_stress / pow(N, s->stress_pow) * cc);
        for (int q9 = 0; q9 < 9; ++q9) {
            for (int q = 0; q < w; ++q)
                A[row * w + q] = sc[(size_t)q9 * p + off + q] * sw;
            y[row] = sw * c->stress[q9];
            row++;
        }
    }
    if (s->weight_eng > 0 && c->has_energy) {
        double sw = sqrt(s->weight_eng / pow(N, s->eng_pow) * c->fitness * cc);
        for (int q = 0; q < w; ++q)
            A[row * w + q] = ec[off + q] * sw;
        double sub = 0;
        if (fix_species)
            for (int t = 0; t < m->Z; ++t)
                sub += ec[t] * m->coef[m->nradial + t];
        y[row] = sw * (c->energy - sub);
        row++;
    }
    free(ec);
    free(fc);
    free(sc);
    return row;
}

/* G += A^T A, b += A^T y; textbook definition accumulated in long double. */
void orc_gram(int64_t rows, int p, const double *A, const double *y, double *G, double *b)
{
    long double *g = (long double *)calloc((size_t)p * p, sizeof(long double));
    long double *v = (long double *)calloc((size_t)p, sizeof(long double));
    for (int64_t r = 0; r < rows; ++r) {
        const double *a = A + r * p;
        for (int i = 0; i < p; ++i) {
            v[i] += (long double)a[i] * y[r];
            for (int j = 0; j < p; ++j)
                g[(size_t)i * p + j] += (long double)a[i] * a[j];
        }
    }
    for (int i = 0; i < p; ++i) {
        b[i] += (double)v[i];
        for (int j = 0; j < p; ++j)
            G[(size_t)i * p + j] += (double)g[(size_t)i * p + j];
    }
    free(g);
    free(v);
}

int orc_linear_system_batch(const orc_model *m, int nconf, orc_nbh *const *hs,
                            const orc_config *cs, const orc_loss_settings *s, int nthreads,
                            double *G, double *b)
{
    return orc_linear_system_batch_ex(m, nconf, hs, cs, s, 0, nthreads, G, b);
}

int orc_linear_system_batch_ex(const orc_model *m, int nconf, orc_nbh *const *hs,
                               const orc_config *cs, const orc_loss_settings *s, int fix_species,
                               int nthreads, double *G, double *b)
{
#ifdef _OPENMP
    if (nthreads <= 0)
        nthreads = omp_get_max_threads();
#else
    nthreads = 1;
#endif
    const int p = m->Z + m->S - (fix_species ? m->Z : 0);
    double *tG = (double *)calloc((size_t)nthreads * p * p, sizeof(double));
    double *tb = (double *)calloc((size_t)nthreads * p, sizeof(double));
    int actual = 1;
#ifdef _OPENMP
#pragma omp parallel num_threads(nthreads)
#endif
    {
        int it = 0;
#ifdef _OPENMP
        it = omp_get_thread_num();
        if (it == 0)
            actual = omp_get_num_threads();
#endif
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int c = 0; c < nconf; ++c) {
            int64_t rows = orc_linear_row_count(s, cs + c);
            double *A = (double *)calloc((size_t)(rows > 0 ? rows : 1) * p, sizeof(double));
            double *y = (double *)calloc((size_t)(rows > 0 ? rows : 1), sizeof(double));
            orc_linear_rows_ex(m, hs[c], s, cs + c, fix_species, A, y);
            orc_gram(rows, p, A, y, tG + (size_t)it * p * p, tb + (size_t)it * p);
            free(A);
            free(y);
        }
    }
    memset(G, 0, sizeof(double) * (size_t)p * p);
    memset(b, 0, sizeof(double) * (size_t)p);
    for (int t = 0; t < actual; ++t) {
        for (int q = 0; q < p * p; ++q)
            G[q] += tG[(size_t)t * p * p + q];
        for (int q = 0; q < p; ++q)
            b[q] += tb[(size_t)t * p + q];
    }
    free(tG);
    free(tb);
    return 0;
}

/* Algorithmic flop convention for E/F/S (per atom):
 *   n_i * (8R + 4MR + 4 nu_max + 32B + 6B + 24) + (9T + 2S + 2)
 * following the loops of basis.cpp:148-164, potential_mtp.cpp:2854-2914,
 * :2938-2957, :1918-1931, :2918-2924, :3292-3305, :2966-2970. */
double orc_efs_flops(const orc_model *m, const orc_nbh *h)
{
    const double per_pair =
        8.0 * m->R + 4.0 * m->M * m->R + 4.0 * (m->max_nu1 - 1) + 32.0 * m->B + 6.0 * m->B + 24;
    const double per_site = 9.0 * m->T + 2.0 * m->S + 2;
    return (double)h->P * per_pair + (double)h->n * per_site;
}
