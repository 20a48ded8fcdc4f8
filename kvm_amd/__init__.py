"""kvm_amd: an MI355X-native persistent task-graph executor for Magni VM task bundles (ABI v2)."""
from pathlib import Path

ROOT = Path(__file__).resolve().parent
REPO = ROOT.parent
