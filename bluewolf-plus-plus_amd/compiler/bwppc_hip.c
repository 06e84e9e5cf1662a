/*
 * bwppc-hip -- BW++'s compiler driver with the HIP target: the pipeline of
 * compiler/main.c:95-193 (parse, typecheck, graph build for --entry,
 * attention detection, autodiff), ending in bwpp_codegen_hip (lower_hip.h)
 * instead of bwpp_codegen_metal (main.c:186).  It links the reference
 * compiler's front end and graph IR unchanged.
 *
 *   bwppc-hip <in.bwpp> <out.plan> [--entry fn] [--dim NAME=N]...
 *             [--batch B] [--batch-dim NAME] [--heads H] [--causal]
 *             [--attn-scale S|auto] [--dtype f32|bf16]
 *             [--train none|seed|mean_square] [--no-fuse-attention] [--no-group-gemms]
 *             [--no-fuse-tails]
 *             [--const V]... [--attn-report] [--dump-graph]
 *             [--dot graph.dot] [--grad-dot grad.dot] [--mem-plan plan.txt]
 *
 * The inspection flags keep main.c:49-86's names: --dot and --grad-dot write
 * the forward and autodiff graphs with the front end's bwpp_graph_dump_dot
 * (main.c:133-157); --mem-plan writes the memory plan of the emitted launch
 * plan (main.c:169-182), placed by libbwpp_hip's own planner: the reference
 * dump's lines (mem_plan.c:176-193) with each buffer's byte size and arena
 * offset and the arena total, as bwpp_hip_plan_report gives them at run
 * time.  The library is loaded only for --mem-plan (from BWPP_HIP_LIB, else
 * ../../lib/libbwpp_hip.so next to this executable); it plans without a
 * device.
 */
#define _GNU_SOURCE
#include <dlfcn.h>
#include <libgen.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "graph_ir.h"
#include "lower_hip.h"
#include "parser.h"
#include "typecheck.h"

static char *read_file(const char *path) {
  FILE *f = fopen(path, "rb");
  if (!f) return NULL;
  if (fseek(f, 0, SEEK_END) != 0) {
    fclose(f);
    return NULL;
  }
  const long n = ftell(f);
  rewind(f);
  char *buf = n >= 0 ? (char *)malloc((size_t)n + 1) : NULL;
  if (!buf) {
    fclose(f);
    return NULL;
  }
  const size_t got = fread(buf, 1, (size_t)n, f);
  fclose(f);
  buf[got] = '\0';
  return buf;
}

static int usage(const char *argv0) {
  fprintf(stderr,
          "usage: %s <in.bwpp> <out.plan> [--entry fn] [--dim NAME=N]... [--batch B] [--batch-dim NAME]\n"
          "       [--heads H] [--causal] [--attn-scale S|auto] [--dtype f32|bf16]\n"
          "       [--train none|seed|mean_square] [--no-fuse-attention] [--no-group-gemms]\n"
          "       [--no-fuse-tails] [--const V]... [--attn-report] [--dump-graph]\n"
          "       [--dot graph.dot] [--grad-dot grad.dot] [--mem-plan plan.txt]\n",
          argv0);
  return 1;
}

static int write_dot(const BwppGraph *g, const char *path) {
  FILE *f = fopen(path, "w");
  if (!f) {
    fprintf(stderr, "failed to open dot output: %s\n", path);
    return 1;
  }
  bwpp_graph_dump_dot(g, f);
  fclose(f);
  return 0;
}

/* The memory plan of the launch plan `text`, from libbwpp_hip's planner. */
static int write_mem_plan(const char *text, const char *path) {
  char lib[4096];
  const char *env = getenv("BWPP_HIP_LIB");
  if (env && env[0]) {
    snprintf(lib, sizeof lib, "%s", env);
  } else {
    char exe[4000];
    const ssize_t n = readlink("/proc/self/exe", exe, sizeof exe - 1);
    if (n <= 0) {
      fprintf(stderr, "--mem-plan: cannot locate this executable; set BWPP_HIP_LIB\n");
      return 1;
    }
    exe[n] = '\0';
    snprintf(lib, sizeof lib, "%s/../../lib/libbwpp_hip.so", dirname(exe));
  }
  void *so = dlopen(lib, RTLD_NOW | RTLD_LOCAL);
  if (!so) {
    fprintf(stderr, "--mem-plan needs libbwpp_hip.so: %s\n", dlerror());
    return 1;
  }
  typedef int (*create_fn)(void *, const char *, void **);
  typedef void (*destroy_fn)(void *);
  typedef const char *(*error_fn)(const void *);
  typedef size_t (*report_fn)(const void *, char *, size_t);
  create_fn create = (create_fn)dlsym(so, "bwpp_hip_plan_create");
  destroy_fn destroy = (destroy_fn)dlsym(so, "bwpp_hip_plan_destroy");
  error_fn error = (error_fn)dlsym(so, "bwpp_hip_plan_last_error");
  report_fn report = (report_fn)dlsym(so, "bwpp_hip_plan_report");
  int rc = 1;
  void *plan = NULL;
  if (!create || !destroy || !error || !report) {
    fprintf(stderr, "--mem-plan: %s lacks the plan entry points\n", lib);
  } else if (create(NULL, text, &plan) != 0) {
    fprintf(stderr, "--mem-plan: the library rejected the plan: %s\n", plan ? error(plan) : "");
  } else {
    const size_t cap = report(plan, NULL, 0);
    char *buf = (char *)malloc(cap);
    FILE *f = buf ? fopen(path, "w") : NULL;
    if (!f) {
      fprintf(stderr, "failed to open mem plan output: %s\n", path);
    } else {
      report(plan, buf, cap);
      fputs(buf, f);
      fclose(f);
      rc = 0;
    }
    free(buf);
  }
  if (plan) destroy(plan);
  dlclose(so);
  return rc;
}

int main(int argc, char **argv) {
  const char *in_path = NULL, *out_path = NULL, *entry = NULL;
  const char *dot_path = NULL, *grad_dot_path = NULL, *mem_plan_path = NULL;
  int attn_report = 0, dump_graph = 0;
  BwppLowerOptions opt;
  bwpp_lower_options_init(&opt);
  static char names[BWPP_LOWER_MAX_DIMS][64];
  /* the command line, recorded at the top of the plan */
  static char header[4096];
  size_t hl = (size_t)snprintf(header, sizeof header, "# generated by bwppc-hip:");
  for (int i = 1; i < argc && hl < sizeof header - 2; ++i) {
    const char *a = argv[i];
    if (i == 1 || i == 2) {  /* keep only the file names of the paths */
      const char *slash = strrchr(a, '/');
      a = slash ? slash + 1 : a;
    }
    hl += (size_t)snprintf(header + hl, sizeof header - hl, " %s", a);
  }
  if (hl < sizeof header - 1) strcat(header, "\n");
  opt.header = header;

  for (int i = 1; i < argc; ++i) {
    const char *a = argv[i];
    const int more = i + 1 < argc;
    if (!strcmp(a, "--entry") && more) {
      entry = argv[++i];
    } else if (!strcmp(a, "--dim") && more) {
      const char *kv = argv[++i];
      const char *eq = strchr(kv, '=');
      if (!eq || opt.dim_count >= BWPP_LOWER_MAX_DIMS || (size_t)(eq - kv) >= sizeof names[0]) return usage(argv[0]);
      memcpy(names[opt.dim_count], kv, (size_t)(eq - kv));
      names[opt.dim_count][eq - kv] = '\0';
      opt.dim_names[opt.dim_count] = names[opt.dim_count];
      opt.dim_values[opt.dim_count++] = strtoull(eq + 1, NULL, 10);
    } else if (!strcmp(a, "--batch") && more) {
      opt.batch = (uint32_t)strtoul(argv[++i], NULL, 10);
    } else if (!strcmp(a, "--batch-dim") && more) {
      opt.batch_dim = argv[++i];
    } else if (!strcmp(a, "--heads") && more) {
      opt.heads = (uint32_t)strtoul(argv[++i], NULL, 10);
    } else if (!strcmp(a, "--causal")) {
      opt.causal = 1;
    } else if (!strcmp(a, "--attn-scale") && more) {
      const char *v = argv[++i];
      if (!strcmp(v, "auto"))
        opt.attn_scale_auto = 1;
      else
        opt.attn_scale = strtof(v, NULL);
    } else if (!strcmp(a, "--dtype") && more) {
      const char *v = argv[++i];
      if (!strcmp(v, "f32"))
        opt.f16_as = BWPP_DTYPE_F32;
      else if (!strcmp(v, "bf16"))
        opt.f16_as = BWPP_DTYPE_BF16;
      else
        return usage(argv[0]);
    } else if (!strcmp(a, "--train") && more) {
      const char *v = argv[++i];
      if (!strcmp(v, "none"))
        opt.train = BWPP_LOWER_TRAIN_NONE;
      else if (!strcmp(v, "seed"))
        opt.train = BWPP_LOWER_TRAIN_SEED;
      else if (!strcmp(v, "mean_square"))
        opt.train = BWPP_LOWER_TRAIN_MEAN_SQUARE;
      else
        return usage(argv[0]);
    } else if (!strcmp(a, "--no-fuse-attention")) {
      opt.fuse_attention = 0;
    } else if (!strcmp(a, "--no-group-gemms")) {
      opt.group_gemms = 0;
    } else if (!strcmp(a, "--no-fuse-tails")) {
      opt.fuse_tails = 0;
    } else if (!strcmp(a, "--const") && more) {
      if (opt.const_count >= BWPP_LOWER_MAX_CONSTS) return usage(argv[0]);
      opt.const_values[opt.const_count++] = strtof(argv[++i], NULL);
    } else if (!strcmp(a, "--attn-report")) {
      attn_report = 1;
    } else if (!strcmp(a, "--dump-graph")) {
      dump_graph = 1;
    } else if (!strcmp(a, "--dot") && more) {
      dot_path = argv[++i];
    } else if (!strcmp(a, "--grad-dot") && more) {
      grad_dot_path = argv[++i];
    } else if (!strcmp(a, "--mem-plan") && more) {
      mem_plan_path = argv[++i];
    } else if (a[0] == '-') {
      return usage(argv[0]);
    } else if (!in_path) {
      in_path = a;
    } else if (!out_path) {
      out_path = a;
    } else {
      return usage(argv[0]);
    }
  }
  if (!in_path || !out_path) return usage(argv[0]);

  char *src = read_file(in_path);
  if (!src) {
    fprintf(stderr, "failed to read input: %s\n", in_path);
    return 1;
  }
  BwppParser parser;
  bwpp_parser_init(&parser, src, strlen(src));
  BwppAstModule *module = bwpp_parse_module(&parser);
  if (!module) {
    fprintf(stderr, "parse failed\n");
    free(src);
    return 1;
  }
  int rc = 1;
  BwppGraph *graph = NULL, *grad = NULL;
  if (bwpp_typecheck_module(module) != BWPP_OK) {
    fprintf(stderr, "typecheck failed\n");
    goto out;
  }
  graph = bwpp_graph_build(module, entry);
  if (!graph) {
    fprintf(stderr, "graph build failed%s%s\n", entry ? " for entry " : "", entry ? entry : "");
    goto out;
  }
  if (attn_report) fprintf(stderr, "attention_candidate=%d\n", bwpp_graph_detect_attention(graph));
  if (dump_graph) bwpp_graph_dump(graph, stderr);
  if (dot_path && write_dot(graph, dot_path) != 0) goto out;
  if (opt.train != BWPP_LOWER_TRAIN_NONE || grad_dot_path) {
    grad = bwpp_graph_autodiff(graph);
    if (!grad) {
      fprintf(stderr, "failed to build autodiff graph\n");
      goto out;
    }
    if (grad_dot_path && write_dot(grad, grad_dot_path) != 0) goto out;
  }
  /* The plan goes to memory first: --mem-plan plans that same text. */
  char *text = NULL;
  size_t text_len = 0;
  FILE *mem = open_memstream(&text, &text_len);
  if (!mem) {
    fprintf(stderr, "out of memory\n");
    goto out;
  }
  char err[512];
  const BwppStatus cs =
      bwpp_codegen_hip(graph, opt.train != BWPP_LOWER_TRAIN_NONE ? grad : NULL, &opt, mem, err, sizeof err);
  fclose(mem);
  if (cs != BWPP_OK) {
    fprintf(stderr, "hip lowering failed: %s\n", err);
    free(text);
    goto out;
  }
  FILE *f = fopen(out_path, "w");
  if (!f || fwrite(text, 1, text_len, f) != text_len) {
    if (f) fclose(f);
    fprintf(stderr, "failed to write output: %s\n", out_path);
    free(text);
    goto out;
  }
  fclose(f);
  if (mem_plan_path && write_mem_plan(text, mem_plan_path) != 0) {
    free(text);
    goto out;
  }
  free(text);
  rc = 0;
out:
  bwpp_graph_destroy(grad);
  bwpp_graph_destroy(graph);
  bwpp_ast_module_destroy(module);
  free(src);
  return rc;
}
