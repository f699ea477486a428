// Driver for the reference GPM v2 container and MTP text adapter
// (tools/gpm_container.h, tools/gpm_mtp.h; header-only), compiled by
// oracle/Makefile into oracle/_ref/gpm_ref.  Test infrastructure only.
//
// usage: gpm_ref text <in.gpm> <out.mtp> [standalone]
//            the root model's .mtp text, GPM::mtp_text(reader, node,
//            standalone) (standalone folds each pair's scale into its
//            radial coefficients, as the runtime reader does)
//        gpm_ref rewrite <in.gpm> <out.gpm>
//            the bundle written again by GPM::Writer (manifest and blocks
//            preserved, header and layout the reference's own)
#include "gpm_mtp.h"

#include <cstdio>
#include <exception>
#include <fstream>
#include <memory>
#include <string>

int main(int argc, char **argv)
try
{
    if (argc < 4)
        return 2;
    const std::string mode = argv[1];
    if (mode == "text")
    {
        GPM::Reader reader(argv[2]);
        const auto &models = GPM::object(GPM::at(reader.manifest, "models"));
        const auto &node =
            GPM::object(GPM::at(models, GPM::string(GPM::at(reader.manifest, "root_model"))));
        const bool standalone = argc > 4 && std::string(argv[4]) == "standalone";
        std::ofstream out(argv[3], std::ios::binary);
        out << GPM::mtp_text(reader, node, standalone);
        return out ? 0 : 3;
    }
    if (mode == "rewrite")
    {
        GPM::Writer w;
        w.preserve(std::make_shared<GPM::Reader>(argv[2]));
        w.save(argv[3]);
        return 0;
    }
    return 2;
}
catch (const std::exception &e)
{
    std::fprintf(stderr, "%s\n", e.what());
    return 7;
}
