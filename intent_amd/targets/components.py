import json
from pathlib import Path

COMPONENTS: dict[str, str] = json.loads((Path(__file__).with_name("components.json")).read_text())
