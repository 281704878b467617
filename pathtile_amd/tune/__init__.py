"""PathTile offline launch-configuration tuner, re-run on one MI355X.

* ``shapes``  - 30 seeded shapes from the BASELINE grid (20 tune / 10 held out);
* ``sweep``   - candidate validation and event timing on the GPU;
* ``select``  - per-path policy selection and held-out regret (CPU only);
* ``python -m pathtile_amd.tune`` - the end-to-end CLI.

The frozen policy (``frozen_policy.json``) supplies the runtime's launch
defaults.
"""
