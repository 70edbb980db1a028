#!/bin/bash
# Writes the reference model's batch predictions for the reference's own A100
# sweep (data/measured/a100.csv) as fixtures, using the reference's model built
# from its own sources by `make -C oracle ref` (oracle/_ref/ridge-predict).
# Run from the repository root in the container that holds /root/reference.
set -euo pipefail
REF=oracle/_ref/ridge-predict
G=tests/golden
test -x "$REF" || make -C oracle ref
$REF --hw $G/a100-sxm4-40gb.json --batch $G/a100_measured.csv --out $G/a100_predictions_ref_calibrated.csv
$REF --gpu a100 --batch $G/a100_measured.csv --out $G/a100_predictions_ref_placeholder.csv
