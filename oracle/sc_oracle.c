/*
 * sc_oracle.c -- CPU oracle for the enumerate-and-sparse-coarsen SpMM/SpMV path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker, never the product:
 * only tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py
 * load the library built from it.  Nothing in sparse-computation_amd/ links,
 * loads or calls it.
 *
 * Every function restates one reference function; the reference location
 * (relative to the hosseinal/sparse-computation tree) is cited on it.  The
 * restatements follow the reference's control flow on purpose (the literal
 * "min column of the row heads" loop of the format builder, the fp32 CSR
 * loop of the CPU SpMM), so that they can be checked against the reference's
 * own fixtures and then used to check the product, which is written
 * differently.
 *
 * Pinning (what checks each function against something other than itself):
 *   or_pattern_masks     -- closed form id = 2^km-1-int(bits,2); pattern lines
 *                           of the 47 reference .cfmtx fixtures (km = 1..6).
 *   or_build             -- byte-exact against the 47 reference .cfmtx fixtures
 *                           (written by oracle.py); brute-force decode -> COO
 *                           round trip on exhaustive tiny matrices; invariants.
 *   or_read_cfmtx        -- against oracle/_ref (the reference's own
 *                           utils/Sparse_io.cpp compiled from its sources) on
 *                           the fixtures and on generated files.
 *   or_spmm_csr_float    -- bit-exact on integer-valued inputs (all partial sums
 *   or_spmv_csr_float       exact in fp32); within the dot-product error bound
 *                           of or_spmm_f64 on random inputs.
 *   or_spmm_f64          -- exact on integer-valued inputs; against numpy's
 *                           float64 dense product.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define OR_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------------ */
/* Pattern enumeration                                                       */
/* ------------------------------------------------------------------------ */

/*
 * build_patterns_map(kernel_m, kernel_n)
 *   code_gen/pattern_utiles/pattern_dictionary.py:29-37
 * and generate_pattern_dictionary(m, n) (same file :40-46), which uses the
 * same order.  For i = 1 .. 2^bits-1 the id i-1 maps to the bit string of
 * x = 2^bits - i, zero-filled to `bits` characters.  Character c of that
 * string is returned as bit c of masks[id] (bit c set <=> char c == '1').
 * Returns the number of patterns, or -1 if bits is out of range.
 */
OR_API int or_pattern_masks(int kernel_m, int kernel_n, int32_t *masks) {
  int bits = kernel_m * kernel_n;
  if (bits <= 0 || bits > 24) return -1;
  int count = 0;
  for (int64_t i = 1; i < ((int64_t)1 << bits); ++i) {
    int64_t x = ((int64_t)1 << bits) - i;
    /* bin(x)[2:].zfill(bits): most significant character first */
    char s[32];
    for (int c = 0; c < bits; ++c) s[c] = ((x >> (bits - 1 - c)) & 1) ? '1' : '0';
    int32_t m = 0;
    for (int c = 0; c < bits; ++c)
      if (s[c] == '1') m |= (int32_t)1 << c;
    masks[i - 1] = m;
    ++count;
  }
  return count;
}

/* ------------------------------------------------------------------------ */
/* CSR -> compressed format (.cfmtx) builder                                 */
/* ------------------------------------------------------------------------ */

typedef struct {
  int32_t *v;
  int64_t n, cap;
} ivec;
typedef struct {
  double *v;
  uint8_t *pad;
  int64_t n, cap;
} dvec;

static void ivec_push(ivec *a, int32_t x) {
  if (a->n == a->cap) {
    a->cap = a->cap ? a->cap * 2 : 16;
    a->v = (int32_t *)realloc(a->v, (size_t)a->cap * sizeof(int32_t));
  }
  a->v[a->n++] = x;
}
static void dvec_push(dvec *a, double x, uint8_t pad) {
  if (a->n == a->cap) {
    a->cap = a->cap ? a->cap * 2 : 16;
    a->v = (double *)realloc(a->v, (size_t)a->cap * sizeof(double));
    a->pad = (uint8_t *)realloc(a->pad, (size_t)a->cap);
  }
  a->v[a->n] = x;
  a->pad[a->n] = pad;
  a->n++;
}

/* Result of or_build, read field by field from Python through ctypes. */
typedef struct {
  int32_t num_row, num_col, kernel_rows, vector_length, npat, npanels;
  int32_t *rpp;     /* [npat * (npanels + 1)] row_panels_pointer, id-major */
  int64_t *ncb;     /* [npat] */
  int32_t **cb;     /* [npat][ncb[p]] indices_array */
  int64_t *nval;    /* [npat] */
  double **val;     /* [npat][nval[p]] padded_values_data_array */
  uint8_t **pad;    /* [npat][nval[p]] 1 = padding entry (Python int 0) */
} or_cfmtx;

OR_API void or_cfmtx_free(or_cfmtx *f) {
  if (!f) return;
  for (int p = 0; p < f->npat; ++p) {
    free(f->cb[p]);
    free(f->val[p]);
    free(f->pad[p]);
  }
  free(f->cb);
  free(f->val);
  free(f->pad);
  free(f->rpp);
  free(f->ncb);
  free(f->nval);
  free(f);
}

/*
 * csr_to_compressed_format_converter(input_csr_matrix, patterns,
 *                                    row_panel_size, p_col_size)
 *   code_gen/ss_format/format_generator.py:68-129
 * followed, per row panel, by transform_row_panel (:36-65).
 *
 * The pattern dictionary `patterns` is passed as parallel arrays in dict
 * insertion order: key_mask[k] (bit c = element c of the bool tuple),
 * key_len[k] (tuple length) and key_id[k] (the dict value, an index into the
 * per-pattern lists).  ids must be 0..npat-1 (the reference indexes Python
 * lists with them).
 *
 * Returns NULL on invalid arguments (the reference raises in the same
 * situations: a pattern with no ones, which makes `len % 0` raise).
 */
OR_API or_cfmtx *or_build(int32_t num_rows, int32_t num_cols, const int32_t *indptr,
                          const int32_t *indices, const double *data, int32_t row_panel_size,
                          int32_t p_col_size, int32_t npat, const int32_t *key_mask,
                          const int32_t *key_len, const int32_t *key_id) {
  if (row_panel_size <= 0 || num_rows < 0 || npat <= 0 || p_col_size < 0) return NULL;
  for (int k = 0; k < npat; ++k) {
    if (key_id[k] < 0 || key_id[k] >= npat) return NULL;
    if (key_mask[k] == 0) return NULL; /* np.sum(key) == 0 -> modulo by zero */
  }
  const int km = row_panel_size;
  const int64_t nnz = indptr[num_rows];

  /* :73-82 -- vstack empty rows up to a multiple of km; the padded rows have
   * indptr == nnz. */
  int32_t rows_to_add = (num_rows % km) ? km - num_rows % km : 0;
  int32_t num_rows_new = num_rows + rows_to_add;
  /* :84-88 -- sentinel column num_cols at position tp_val = nnz. */
  const int64_t tp_val = nnz;
  int32_t *indices_all = (int32_t *)malloc((size_t)(nnz + 1) * sizeof(int32_t));
  double *values_all = (double *)malloc((size_t)(nnz + 1) * sizeof(double));
  memcpy(indices_all, indices, (size_t)nnz * sizeof(int32_t));
  memcpy(values_all, data, (size_t)nnz * sizeof(double));
  indices_all[nnz] = num_cols;
  values_all[nnz] = 0.0;

  int32_t npanels = (num_rows + km - 1) / km; /* range(0, num_rows, km) */
  or_cfmtx *f = (or_cfmtx *)calloc(1, sizeof(or_cfmtx));
  f->num_row = num_rows;
  f->num_col = num_cols;
  f->kernel_rows = km;
  f->vector_length = p_col_size;
  f->npat = npat;
  f->npanels = npanels;
  f->rpp = (int32_t *)calloc((size_t)npat * (npanels + 1), sizeof(int32_t));
  f->ncb = (int64_t *)calloc(npat, sizeof(int64_t));
  f->nval = (int64_t *)calloc(npat, sizeof(int64_t));
  f->cb = (int32_t **)calloc(npat, sizeof(int32_t *));
  f->val = (double **)calloc(npat, sizeof(double *));
  f->pad = (uint8_t **)calloc(npat, sizeof(uint8_t *));

  ivec *fmt_idx = (ivec *)calloc(npat, sizeof(ivec)); /* format_object.indices_array */
  dvec *fmt_val = (dvec *)calloc(npat, sizeof(dvec)); /* .padded_values_data_array */
  int32_t *rpp_len = (int32_t *)calloc(npat, sizeof(int32_t));
  /* row_panels_pointer starts as [0] for every pattern (:26) */
  for (int p = 0; p < npat; ++p) f->rpp[(int64_t)p * (npanels + 1) + rpp_len[p]++] = 0;

  ivec *rp_idx = (ivec *)calloc(npat, sizeof(ivec)); /* row_panel_indices_array */
  dvec *rp_val = (dvec *)calloc(npat, sizeof(dvec)); /* row_panel_values_array */
  int64_t *pointer = (int64_t *)malloc(sizeof(int64_t) * km);
  int64_t *pointer_end = (int64_t *)malloc(sizeof(int64_t) * km);
  uint8_t *matches = (uint8_t *)malloc(km);

  for (int32_t start_row = 0; start_row < num_rows; start_row += km) {
    int32_t end_row = start_row + km < num_rows_new ? start_row + km : num_rows_new;
    int len = end_row - start_row;
    for (int p = 0; p < npat; ++p) {
      rp_idx[p].n = 0;
      rp_val[p].n = 0;
    }
    for (int r = 0; r < len; ++r) {
      int32_t row = start_row + r;
      pointer[r] = row < num_rows ? indptr[row] : nnz;
      pointer_end[r] = row + 1 <= num_rows ? indptr[row + 1] : nnz;
    }
    for (;;) {
      /* while not np.all(pointer_end <= pointer) */
      int done = 1;
      for (int r = 0; r < len; ++r)
        if (!(pointer_end[r] <= pointer[r])) done = 0;
      if (done) break;
      for (int r = 0; r < len; ++r)
        if (pointer[r] == pointer_end[r]) pointer[r] = tp_val;
      int32_t min_col = indices_all[pointer[0]];
      for (int r = 1; r < len; ++r)
        if (indices_all[pointer[r]] < min_col) min_col = indices_all[pointer[r]];
      int32_t mmask = 0;
      for (int r = 0; r < len; ++r) {
        matches[r] = indices_all[pointer[r]] == min_col;
        if (matches[r]) mmask |= 1 << r;
      }
      /* val = patterns.get(tuple(matches), -1) */
      int val = -1;
      for (int k = 0; k < npat; ++k)
        if (key_len[k] == len && key_mask[k] == mmask) {
          val = key_id[k];
          break;
        }
      if (val != -1) {
        ivec_push(&rp_idx[val], min_col);
        for (int r = 0; r < len; ++r)
          if (matches[r]) {
            dvec_push(&rp_val[val], values_all[pointer[r]], 0);
          }
        for (int r = 0; r < len; ++r)
          if (matches[r]) values_all[pointer[r]] = 0.0;
      }
      for (int r = 0; r < len; ++r)
        if (matches[r]) pointer[r] += 1;
      for (int r = 0; r < len; ++r)
        if (pointer[r] == pointer_end[r]) pointer[r] = tp_val;
    }

    /* transform_row_panel (:36-65), iterating patterns.items() */
    for (int k = 0; k < npat; ++k) {
      int val = key_id[k];
      int nnzk = __builtin_popcount((unsigned)key_mask[k]); /* np.sum(key) */
      int pack_col_size = p_col_size;
      if (p_col_size == 0) pack_col_size = 32 / nnzk;
      int64_t vector_length = (int64_t)pack_col_size * nnzk;
      dvec *rv = &rp_val[val];
      if (vector_length == 0) { /* `len % 0` raises in the reference */
        or_cfmtx_free(f);
        f = NULL;
        goto cleanup;
      }
      int64_t reminder = rv->n % vector_length;
      if (rv->n != 0 && reminder != 0)
        for (int64_t q = 0; q < vector_length - reminder; ++q) dvec_push(rv, 0.0, 1);
      for (int64_t q = 0; q < rv->n; ++q) dvec_push(&fmt_val[val], rv->v[q], rv->pad[q]);
      ivec *ri = &rp_idx[val];
      for (int64_t q = 0; q < ri->n; ++q) ivec_push(&fmt_idx[val], ri->v[q]);
      int64_t reminder_cols = ri->n % pack_col_size;
      if (ri->n != 0 && reminder_cols != 0) {
        int32_t col_max = ri->v[0];
        for (int64_t q = 1; q < ri->n; ++q)
          if (ri->v[q] > col_max) col_max = ri->v[q];
        for (int64_t q = 0; q < pack_col_size - reminder_cols; ++q) ivec_push(&fmt_idx[val], col_max);
      }
      f->rpp[(int64_t)val * (npanels + 1) + rpp_len[val]++] = (int32_t)fmt_idx[val].n;
      /* transform_row_panel mutates row_panel_array[val] in place; it is
       * rebuilt for the next panel, so clearing it here is equivalent. */
      rv->n = 0;
      ri->n = 0;
    }
  }

  for (int p = 0; p < npat; ++p) {
    f->ncb[p] = fmt_idx[p].n;
    f->cb[p] = fmt_idx[p].v ? fmt_idx[p].v : (int32_t *)malloc(4);
    fmt_idx[p].v = NULL;
    f->nval[p] = fmt_val[p].n;
    f->val[p] = fmt_val[p].v ? fmt_val[p].v : (double *)malloc(8);
    f->pad[p] = fmt_val[p].pad ? fmt_val[p].pad : (uint8_t *)malloc(1);
    fmt_val[p].v = NULL;
    fmt_val[p].pad = NULL;
  }

cleanup:
  for (int p = 0; p < npat; ++p) {
    free(rp_idx[p].v);
    free(rp_val[p].v);
    free(rp_val[p].pad);
    free(fmt_idx[p].v);
    free(fmt_val[p].v);
    free(fmt_val[p].pad);
  }
  free(rp_idx);
  free(rp_val);
  free(fmt_idx);
  free(fmt_val);
  free(rpp_len);
  free(pointer);
  free(pointer_end);
  free(matches);
  free(indices_all);
  free(values_all);
  return f;
}

/* ------------------------------------------------------------------------ */
/* .cfmtx reader                                                             */
/* ------------------------------------------------------------------------ */

/* Result of or_read_cfmtx: what readCFMTXFile puts in each CompressedFormat. */
typedef struct {
  int32_t num_rows, num_columns, kernel_rows, num_patterns, vector_length;
  int32_t nrpp;     /* pm / km + 1 */
  int32_t *pop;     /* [num_patterns] count of '1' in the i-th pattern line */
  int32_t *rpp;     /* [num_patterns * nrpp] */
  int32_t *npp;     /* [num_patterns * nrpp] RPP * pop */
  int64_t *ncb;
  int32_t **cb;
  int64_t *nnz;
  float **val;
} or_read;

OR_API void or_read_free(or_read *r) {
  if (!r) return;
  for (int p = 0; p < r->num_patterns; ++p) {
    free(r->cb[p]);
    free(r->val[p]);
  }
  free(r->cb);
  free(r->val);
  free(r->pop);
  free(r->rpp);
  free(r->npp);
  free(r->ncb);
  free(r->nnz);
  free(r);
}

static char *read_line(FILE *fp) {
  size_t cap = 256, n = 0;
  char *s = (char *)malloc(cap);
  int ch;
  while ((ch = fgetc(fp)) != EOF && ch != '\n') {
    if (n + 1 >= cap) {
      cap *= 2;
      s = (char *)realloc(s, cap);
    }
    s[n++] = (char)ch;
  }
  if (ch == EOF && n == 0) {
    free(s);
    return NULL;
  }
  s[n] = 0;
  return s;
}

/*
 * readCFMTXFile(path)   utils/Sparse_io.cpp:84-182
 * with the CompressedFormat(M, N, Nnz, KM, KN) constructor it calls
 * (include/compressed_format/CompressedFormat.h:142-173).
 *
 * Header "rows cols km P kn"; then P pattern lines whose '1' count is the
 * pop of the i-th data block; then, per pattern, an RPP line (NPP = RPP*pop),
 * a CB line and a value line parsed as float (`iss >> float`, i.e. strtof
 * rounding straight from the decimal text).  vector_length 0 becomes 1.
 * RPP entries beyond nrpp are rejected here (the reference writes past its
 * allocation); NULL is returned for an unopenable file or such a mismatch.
 */
OR_API or_read *or_read_cfmtx(const char *path) {
  FILE *fp = fopen(path, "r");
  if (!fp) return NULL;
  or_read *r = (or_read *)calloc(1, sizeof(or_read));
  char *line = read_line(fp);
  if (!line || sscanf(line, "%d %d %d %d %d", &r->num_rows, &r->num_columns, &r->kernel_rows,
                      &r->num_patterns, &r->vector_length) != 5 ||
      r->num_patterns <= 0 || r->kernel_rows <= 0) {
    free(line);
    fclose(fp);
    free(r);
    return NULL;
  }
  free(line);
  int P = r->num_patterns;
  int64_t M = r->num_rows, KM = r->kernel_rows;
  int64_t pm = (M % KM == 0) ? M : M + KM - M % KM;
  r->nrpp = (int32_t)(pm / KM + 1);
  r->pop = (int32_t *)calloc(P, sizeof(int32_t));
  r->rpp = (int32_t *)calloc((size_t)P * r->nrpp, sizeof(int32_t));
  r->npp = (int32_t *)calloc((size_t)P * r->nrpp, sizeof(int32_t));
  r->ncb = (int64_t *)calloc(P, sizeof(int64_t));
  r->nnz = (int64_t *)calloc(P, sizeof(int64_t));
  r->cb = (int32_t **)calloc(P, sizeof(int32_t *));
  r->val = (float **)calloc(P, sizeof(float *));
  for (int i = 0; i < P; ++i) {
    line = read_line(fp);
    if (!line) break;
    char pat[256] = {0};
    sscanf(line, "%255s", pat);
    int n = 0;
    for (char *c = pat; *c; ++c) n += (*c == '1');
    r->pop[i] = n;
    free(line);
  }
  int bad = 0;
  for (int i = 0; i < P && !bad; ++i) {
    /* RPP */
    line = read_line(fp);
    int64_t cnt = 0;
    if (line) {
      char *s = line, *e;
      for (;;) {
        long v = strtol(s, &e, 10);
        if (e == s) break;
        if (cnt >= r->nrpp) {
          bad = 1;
          break;
        }
        r->rpp[(int64_t)i * r->nrpp + cnt] = (int32_t)v;
        r->npp[(int64_t)i * r->nrpp + cnt] = (int32_t)(v * r->pop[i]);
        ++cnt;
        s = e;
      }
      free(line);
    }
    /* CB */
    line = read_line(fp);
    int64_t cap = 16;
    r->cb[i] = (int32_t *)malloc(cap * sizeof(int32_t));
    if (line) {
      char *s = line, *e;
      for (;;) {
        long v = strtol(s, &e, 10);
        if (e == s) break;
        if (r->ncb[i] == cap) {
          cap *= 2;
          r->cb[i] = (int32_t *)realloc(r->cb[i], cap * sizeof(int32_t));
        }
        r->cb[i][r->ncb[i]++] = (int32_t)v;
        s = e;
      }
      free(line);
    }
    /* values */
    line = read_line(fp);
    cap = 16;
    r->val[i] = (float *)malloc(cap * sizeof(float));
    if (line) {
      char *s = line, *e;
      for (;;) {
        float v = strtof(s, &e);
        if (e == s) break;
        if (r->nnz[i] == cap) {
          cap *= 2;
          r->val[i] = (float *)realloc(r->val[i], cap * sizeof(float));
        }
        r->val[i][r->nnz[i]++] = v;
        s = e;
      }
      free(line);
    }
  }
  if (r->vector_length == 0) r->vector_length = 1;
  fclose(fp);
  if (bad) {
    or_read_free(r);
    return NULL;
  }
  return r;
}

/* ------------------------------------------------------------------------ */
/* CPU SpMM / SpMV                                                           */
/* ------------------------------------------------------------------------ */

/*
 * spmm_csr_float(m, n, Ap, Ai, Ax, B, C)
 *   example_cuda/spmm_demo_gpu_utils.h:25-36
 *   (generator text: code_gen/spmm/spmm_format_code_generator.py:381-392)
 * C += A*B with fp32 accumulation straight into C, CSR order, B and C
 * row-major with n columns.
 */
OR_API void or_spmm_csr_float(int m, int n, const int *Ap, const int *Ai, const float *Ax,
                              const float *B, float *C) {
  for (int i = 0; i < m; i++) {
    for (int j = Ap[i]; j < Ap[i + 1]; j++) {
      int col_index = Ai[j];
      float value = Ax[j];
      for (int k = 0; k < n; k++) {
        C[(int64_t)i * n + k] += value * B[(int64_t)col_index * n + k];
      }
    }
  }
}

/*
 * spmv_csr_float(n, Ap, Ai, Ax, x, y)
 *   example_cuda/spmv_demo_gpu_utils.h:86-98
 * y += A*x with the row sum accumulated in double from float operands.
 */
OR_API void or_spmv_csr_float(int n, const int *Ap, const int *Ai, const float *Ax, const float *x,
                              float *y) {
  for (int i = 0; i < n; i++) {
    double sum = 0.0;
    for (int j = Ap[i]; j < Ap[i + 1]; j++) {
      int col_index = Ai[j];
      double value = Ax[j];
      sum += value * x[col_index];
    }
    y[i] += sum;
  }
}

/*
 * fp64 check of C = A*B from the same fp32 operands (the correctness gate of
 * the path: max relative error normalised by (|A|*|B|)_ij).  C64 receives
 * sum a*b in double, Cabs receives sum |a|*|b|.
 */
OR_API void or_spmm_f64(int m, int n, const int *Ap, const int *Ai, const float *Ax, const float *B,
                        double *C64, double *Cabs) {
  for (int64_t t = 0; t < (int64_t)m * n; ++t) {
    C64[t] = 0.0;
    Cabs[t] = 0.0;
  }
  for (int i = 0; i < m; i++) {
    for (int j = Ap[i]; j < Ap[i + 1]; j++) {
      double a = (double)Ax[j];
      const float *b = B + (int64_t)Ai[j] * n;
      double *c = C64 + (int64_t)i * n;
      double *ca = Cabs + (int64_t)i * n;
      for (int k = 0; k < n; k++) {
        c[k] += a * (double)b[k];
        ca[k] += fabs(a) * fabs((double)b[k]);
      }
    }
  }
}
