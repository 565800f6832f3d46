"""python -m hearth_amd <command>"""
import sys

from .cli import main

sys.exit(main())
