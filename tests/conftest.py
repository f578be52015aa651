import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs an MI355X (runs the HIP library)')
    config.addinivalue_line('markers', 'long: runs for minutes; collected after every other test of its run')


def pytest_collection_modifyitems(session, config, items):
    """Long tests go after the rest (stable order otherwise), so that a run stopped by a time limit has already
    passed through the quick parity tests; files named test_zz_* stay last of all."""
    def key(item):
        last = os.path.basename(str(item.fspath)).startswith('test_zz_')
        return (last, item.get_closest_marker('long') is not None)
    items[:] = sorted(items, key=key)
