// Prints a model's product rules and the library's lane-major rule tables
// (build_plan in imr-mlp_amd/csrc/model.cpp) as plain text for the host
// tests in test_capi_host.py:
//   K B T K4 dummy part0 red0 pad
//   times: T lines "l r c o"
//   per direction (fwd, then bwd): "nlev ncomb nsteps", the level_step and
//   level_comb lines, nsteps * 64 lines "x y", ncomb lines "target first count"
#include "mtpx_internal.hpp"

#include <cstdio>
#include <fstream>
#include <sstream>

static void tables(const std::vector<int> &level_step, const std::vector<int> &level_comb,
                   const std::vector<int> &steps, const std::vector<int> &comb)
{
    const size_t nsteps = steps.size() / (2 * mtpx::kWave);
    std::printf("%zu %zu %zu\n", level_step.size() - 1, comb.size() / 4, nsteps);
    for (int v : level_step)
        std::printf("%d ", v);
    std::printf("\n");
    for (int v : level_comb)
        std::printf("%d ", v);
    std::printf("\n");
    for (size_t i = 0; i < steps.size(); i += 2)
        std::printf("%d %d\n", steps[i], steps[i + 1]);
    for (size_t i = 0; i < comb.size(); i += 4)
        std::printf("%d %d %d\n", comb[i], comb[i + 1], comb[i + 2]);
}

int main(int argc, char **argv)
{
    if (argc != 2) {
        std::fprintf(stderr, "usage: %s model.mtp\n", argv[0]);
        return 2;
    }
    std::ifstream f(argv[1]);
    std::stringstream ss;
    ss << f.rdbuf();
    mtpx::Model m;
    mtpx::Plan p;
    std::string err;
    if (!mtpx::parse_mtp(ss.str(), m, err) || !mtpx::build_plan(m, p, err)) {
        std::fprintf(stderr, "%s\n", err.c_str());
        return 1;
    }
    std::printf("%d %d %d %d %d %d %d %d\n", m.K, m.B, m.T, p.K4, p.dummy, p.part0, p.red0,
                mtpx::kRulePad);
    for (int t = 0; t < m.T; ++t)
        std::printf("%d %d %d %d\n", m.times[4 * t], m.times[4 * t + 1], m.times[4 * t + 2],
                    m.times[4 * t + 3]);
    tables(p.fwd_level_step, p.fwd_level_comb, p.fwd_steps, p.fwd_comb);
    tables(p.bwd_level_step, p.bwd_level_comb, p.bwd_steps, p.bwd_comb);
    return 0;
}
