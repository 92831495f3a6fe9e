// Host-side checks of the planner under AddressSanitizer / UndefinedBehaviorSanitizer: every
// plan given on the command line is created as a dry-run model (no device: planning, packing,
// memory plan and its overlap check, launch lists and their host bounds checks) with every
// flag set, at several batch sizes, and every node is described; malformed plans must fail
// with an error, not a crash.
//   dry_run_checks <plan>... -- <malformed plan>...
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "ivh.h"

static int fails = 0;
#define EXPECT(c, what)                                                       \
  do {                                                                        \
    if (!(c)) {                                                               \
      std::fprintf(stderr, "EXPECT failed: %s (%s)\n", #c, (what).c_str()); \
      ++fails;                                                                \
    }                                                                         \
  } while (0)

int main(int argc, char ** argv)
{
  std::vector<std::string> good, bad;
  bool sep = false;
  for (int i = 1; i < argc; ++i) {
    if (std::strcmp(argv[i], "--") == 0) sep = true;
    else (sep ? bad : good).push_back(argv[i]);
  }
  const uint32_t flag_sets[] = {0,
                                IVH_FLAG_NO_FUSE,
                                IVH_FLAG_NCHW_ONLY,
                                IVH_FLAG_DIRECT_ONLY,
                                IVH_FLAG_NO_REUSE,
                                IVH_FLAG_NO_SPLITK | IVH_FLAG_NO_HALO | IVH_FLAG_NO_RESIDENT,
                                IVH_FLAG_NO_FUSE_DECODE | IVH_FLAG_PROFILE};
  const int batches[] = {1, 5, 64, 3, 1};
  int models = 0;
  for (const auto & plan : good) {
    for (uint32_t f : flag_sets) {
      ivh_model * m = nullptr;
      const std::string what = plan + " flags " + std::to_string(f);
      if (ivh_create(plan.c_str(), 0, 64, f | IVH_FLAG_DRY_RUN, &m) != IVH_OK) {
        std::fprintf(stderr, "create failed: %s: %s\n", what.c_str(), ivh_last_error());
        ++fails;
        continue;
      }
      ++models;
      for (int b : batches) EXPECT(ivh_run(m, b) == IVH_OK, what + " batch " + std::to_string(b));
      int n = 0;
      EXPECT(ivh_node_count(m, &n) == IVH_OK && n > 0, what);
      for (int i = 0; i < n; ++i) {
        char op[64], kern[64], desc[256];
        double fl = 0, by = 0;
        EXPECT(ivh_node_info(m, i, op, sizeof op, kern, sizeof kern, desc, sizeof desc, &fl, &by) == IVH_OK, what);
      }
      size_t arena = 0, weights = 0;
      EXPECT(ivh_memory_info(m, 64, &arena, &weights) == IVH_OK && arena > 0, what);
      EXPECT(ivh_run(m, 65) != IVH_OK, what + " batch above the maximum");
      EXPECT(ivh_set_input_f16(m, nullptr, 1) != IVH_OK, what + " data call on a dry-run model");
      ivh_destroy(m);
    }
  }
  for (const auto & plan : bad) {
    // rejected when the model is created or, for node-level errors, when its launches are
    // first built (ivh_run), as PlanModel throws from its constructor or run()
    ivh_model * m = nullptr;
    int rc = ivh_create(plan.c_str(), 0, 4, IVH_FLAG_DRY_RUN, &m);
    if (rc == IVH_OK) {
      rc = ivh_run(m, 1);
      ivh_destroy(m);
    }
    EXPECT(rc != IVH_OK && std::strlen(ivh_last_error()) > 0, "malformed plan " + plan);
  }
  std::printf("dry_run_checks: %d models, %zu malformed plans, %d failures\n", models, bad.size(), fails);
  return fails == 0 ? 0 : 1;
}
