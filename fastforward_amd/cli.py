"""Command line entry point, as the reference's ``fastforward-accel``
(cli.py:6-15): one image, one question, two to eight choices; prints the
response JSON. ``python -m fastforward_amd.cli --bundle B --image I
--question Q --choices A B ...``"""
import argparse
import json
import sys


def main(argv=None):
    p = argparse.ArgumentParser(description="FastForward visual choice inference on MI355X")
    p.add_argument("--bundle", required=True)
    p.add_argument("--image", required=True)
    p.add_argument("--question", required=True)
    p.add_argument("--choices", nargs="+", required=True)
    p.add_argument("--backend", choices=["fast", "native", "established"], default="fast")
    a = p.parse_args(argv)
    from .api import Accelerator
    rt = Accelerator(a.bundle, backend=a.backend)
    print(json.dumps(rt.predict(a.image, a.question, a.choices), ensure_ascii=False))
    return 0


if __name__ == "__main__":
    sys.exit(main())
