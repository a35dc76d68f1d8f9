/* bench.c - decode-throughput yardsticks over a cumulative wall-time series
 * (reference surge.h:1784-1824, src/bench.c:23-78), and the leaderboard row
 * formatters (surge.h:1845-1955).
 *
 * t[i] is the wall time at which token i finished. Both estimators ignore
 * indices below `warmup`. The slope is a least-squares fit of token index
 * against time, done mean-centred in double so epoch-sized timestamps do not
 * cancel; the average is endpoint to endpoint. */
#include "surge.h"

#include <math.h>
#include <stdio.h>
#include <unistd.h>

double sg_bench_slope(const double *t, uint32_t n, uint32_t warmup) {
    if (!t || n <= warmup || n - warmup < 2) return 0.0;
    uint32_t k = n - warmup;
    double mt = 0.0, mi = 0.0;
    for (uint32_t i = warmup; i < n; i++) { mt += t[i]; mi += (double)i; }
    mt /= k; mi /= k;
    double sxy = 0.0, sxx = 0.0;
    for (uint32_t i = warmup; i < n; i++) {
        double dx = t[i] - mt;
        sxy += dx * ((double)i - mi);
        sxx += dx * dx;
    }
    return sxx > 0.0 ? sxy / sxx : 0.0;
}

double sg_bench_avg_tps(const double *t, uint32_t n, uint32_t warmup) {
    if (!t || n == 0 || warmup + 1 >= n) return 0.0;
    double dt = t[n - 1] - t[warmup];
    return dt > 0.0 ? (double)(n - 1 - warmup) / dt : 0.0;
}

uint32_t sg_bench_default_warmup(uint32_t n_gen) {
    uint32_t w = (uint32_t)(0.02 * (double)n_gen + 0.5);
    return w < 1 ? 1 : w;
}

/* The leaderboard row's formatters and admission rule (reference
 * surge.h:1916-1955, the surge-bench output contract): an 8-column pipe row
 * and a flat JSON object with the struct's field names as keys. */

bool sg_bench_admitted(const sg_bench_row *row) {
    return row && row->gemm_tflops > SG_BENCH_GEMM_MIN_TFLOPS && row->ingestion_ok;
}

void sg_bench_finalize_status(sg_bench_row *row) {
    if (!row) return;
    const bool ok = sg_bench_admitted(row);
    snprintf(row->status, sizeof row->status, "%s", ok ? "DONE" : "VOID");
    fprintf(stderr, "bench: status=%s (gemm_tflops=%.2f ingestion_ok=%s)\n", row->status, row->gemm_tflops,
            row->ingestion_ok ? "true" : "false");
}

void sg_bench_format_md_row(const sg_bench_row *row, char *buf, size_t cap) {
    if (!buf || !cap) return;
    if (!row) { buf[0] = '\0'; return; }
    char pf[32];
    if (row->prefill_tps < 0.0) snprintf(pf, sizeof pf, "-");
    else snprintf(pf, sizeof pf, "%.0f", row->prefill_tps);
    /* the %.Ns precisions bound each read to its array even without a NUL */
    snprintf(buf, cap, "| %.63s | %.63s | %s | %.2f | %.1f GiB | %u/%u | %ld min | %.15s |", row->model, row->engine,
             pf, row->decode_tps_slope, row->peak_ram_gib, row->recall_hits, row->recall_total,
             lround(row->wall_s / 60.0), row->status);
}

/* JSON string body of at most n source bytes of s: quote and backslash
 * escaped, bytes below 0x20 as \u00XX; never splits an escape when out fills. */
static void json_str(const char *s, size_t n, char *out, size_t cap) {
    size_t o = 0;
    for (size_t i = 0; s && i < n && s[i] && o + 1 < cap; i++) {
        const unsigned char c = (unsigned char)s[i];
        if (c == '"' || c == '\\') {
            if (o + 3 > cap) break;
            out[o++] = '\\';
            out[o++] = (char)c;
        } else if (c < 0x20) {
            if (o + 7 > cap) break;
            o += (size_t)snprintf(out + o, 7, "\\u%04x", c);
        } else {
            out[o++] = (char)c;
        }
    }
    out[o] = '\0';
}

void sg_bench_format_json(const sg_bench_row *row, char *buf, size_t cap) {
    if (!buf || !cap) return;
    if (!row) { buf[0] = '\0'; return; }
    char mo[6 * 64 + 8], en[6 * 64 + 8], st[6 * 16 + 8], li[6 * 96 + 8];
    json_str(row->model, sizeof row->model, mo, sizeof mo);
    json_str(row->engine, sizeof row->engine, en, sizeof en);
    json_str(row->status, sizeof row->status, st, sizeof st);
    json_str(row->log_id, sizeof row->log_id, li, sizeof li);
    snprintf(buf, cap,
             "{\"model\":\"%s\",\"engine\":\"%s\",\"prefill_tps\":%.6g,\"decode_tps_slope\":%.6g,"
             "\"decode_tps_avg\":%.6g,\"prefill_wall_s\":%.6g,\"decode_wall_s\":%.6g,\"prefill_rest_s\":%.6g,"
             "\"prefill_compute_tps\":%.6g,\"prefill_segments\":%llu,\"decode_rest_s\":%.6g,"
             "\"decode_compute_tps\":%.6g,\"decode_rests\":%u,\"decode_clamp_events\":%u,"
             "\"decode_baseline_ms\":%.6g,\"peak_ram_gib\":%.6g,\"gpu_alloc_gib\":%.6g,\"recall_hits\":%u,"
             "\"recall_total\":%u,\"assoc_hits\":%u,\"n_prompt_tok\":%llu,\"n_gen\":%u,\"wall_s\":%.6g,"
             "\"gemm_tflops\":%.6g,\"ingestion_ok\":%s,\"status\":\"%s\",\"log_id\":\"%s\"}",
             mo, en, row->prefill_tps, row->decode_tps_slope, row->decode_tps_avg, row->prefill_wall_s,
             row->decode_wall_s, row->prefill_rest_s, row->prefill_compute_tps, row->prefill_segments,
             row->decode_rest_s, row->decode_compute_tps, row->decode_rests, row->decode_clamp_events,
             row->decode_baseline_ms, row->peak_ram_gib, row->gpu_alloc_gib, row->recall_hits, row->recall_total,
             row->assoc_hits, (unsigned long long)row->n_prompt_tok, row->n_gen, row->wall_s, row->gemm_tflops,
             row->ingestion_ok ? "true" : "false", st, li);
}

/* The peak-memory probe (reference surge.h:2104-2142, src/bench.c:401-440).
 * Linux has no Mach phys_footprint; the resident set from /proc/self/statm
 * (its second field, in pages) is the nearest figure for host memory. */
uint64_t sg_proc_phys_footprint(void) {
    FILE *f = fopen("/proc/self/statm", "r");
    if (!f) {
        fprintf(stderr, "bench: proc_phys_footprint: cannot open /proc/self/statm\n");
        return 0;
    }
    unsigned long long size = 0, resident = 0;
    const int got = fscanf(f, "%llu %llu", &size, &resident);
    fclose(f);
    const long page = sysconf(_SC_PAGESIZE);
    if (got != 2 || page <= 0) {
        fprintf(stderr, "bench: proc_phys_footprint: unreadable /proc/self/statm\n");
        return 0;
    }
    return (uint64_t)resident * (uint64_t)page;
}

void sg_mem_tracker_reset(sg_mem_tracker *t) {
    if (t) t->peak = 0;
}

void sg_mem_tracker_sample(sg_mem_tracker *t, uint64_t current_alloc, uint64_t phys_footprint) {
    if (!t) return;
    const uint64_t hi = phys_footprint > current_alloc ? phys_footprint : current_alloc;
    if (hi > t->peak) t->peak = hi;
}

uint64_t sg_mem_tracker_peak(const sg_mem_tracker *t) { return t ? t->peak : 0; }

/* The row's ingestion guard (reference surge.h:1980-1993): the prompt was not
 * cut to fit the context and its id count is in the expected range. */
void sg_bench_check_ingestion(uint64_t n_ids, uint32_t max_ctx, uint64_t expect_min, uint64_t expect_max,
                              bool *ok) {
    if (!ok) return;
    *ok = n_ids <= (uint64_t)max_ctx && n_ids >= expect_min && n_ids <= expect_max;
    fprintf(stderr, "bench: ingestion guard: %llu ids, max_ctx %u, expected [%llu, %llu]: %s\n",
            (unsigned long long)n_ids, max_ctx, (unsigned long long)expect_min, (unsigned long long)expect_max,
            *ok ? "ok" : "failed");
}
